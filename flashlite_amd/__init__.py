"""flashlite_amd -- FlashAttention-2 forward for AMD Instinct MI355X (gfx950).

Drop-in for the ``flash_attn_wmma`` extension of thebigblender/FlashLite:

    from flashlite_amd import forward_flash2, forward_naive
    out = forward_flash2(q, k, v, sm_scale=0.0, is_causal=False, out=None)

(``import flash_attn_wmma`` works too, from the repository root.)  The
functions are the torch binding built from ``csrc/flash_attn.cpp``; the
kernels are hand-written HIP for gfx950 in ``csrc/*.hip`` behind the C ABI
declared in ``include/flashlite_attn.h``.  There is no fallback: if the
extension is not built, importing raises ImportError.
"""

from __future__ import annotations

import os

import torch  # noqa: F401  (loads libtorch/libc10 before the extension)

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))

try:
    from . import flash_attn_wmma as _ext
except ImportError as exc:  # pragma: no cover - exercised only without a build
    raise ImportError(
        "flashlite_amd: the HIP extension is not built. Run `python flashlite_amd/build.py` "
        "(or `python -c 'import __graft_entry__ as g; g.build()'`) from the repository root."
    ) from exc

forward_flash2 = _ext.forward_flash2
forward_naive = _ext.forward_naive
# Beyond the reference surface: strided [B, H, N, 64] views (a [B, N, H, 64]
# tensor passes as x.transpose(1, 2)), N_k != N_q with the causal diagonal
# aligned bottom-right, and the fp32 log-sum-exp with return_lse=True.
# num_splits / workspace select split-KV for few query rows over many keys.
forward_flash2_ex = _ext.forward_flash2_ex
splitkv_workspace_bytes = _ext.splitkv_workspace_bytes

__all__ = ["forward_flash2", "forward_naive", "forward_flash2_ex", "splitkv_workspace_bytes"]
