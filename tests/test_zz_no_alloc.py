"""GPU test of the allocation-free split-KV entry point
(``fl_attn_fwd_f16_splitkv_noalloc``), through the C ABI.

Its partials go to the library's static device scratch array instead of a
caller workspace; the kernels are the same, so its outputs (O and the
log-sum-exp) must equal ``fl_attn_fwd_f16_splitkv``'s bit for bit.  Two calls
in a row, the second on a smaller problem: the array keeps the first call's
partials, so a combine that read a row the second call did not write would
differ.  Both calls are also held to the north_star bound against the fp32
oracle.  A plan whose partials exceed the array is rejected before launch.
"""

import numpy as np
import pytest

from flashlite_amd import capi
from gpu_util import assert_close_oracle, to_dev
from oracle import attention_fp32

pytestmark = pytest.mark.gpu

# (B, H, N_q, N_k, causal, num_splits): the first uses about half the array
# (8 chunks x 32 heads x 64 rows x 272 bytes = 4.5 MB), the second far less.
CALLS = [(4, 8, 64, 8192, False, 0), (1, 4, 1, 1000, True, 3)]


def _qkv(b, h, nq, nk, seed):
    rs = np.random.RandomState(seed)
    mk = lambda n: rs.standard_normal((b, h, n, 64)).astype(np.float32).astype(np.float16)  # noqa: E731
    return mk(nq), mk(nk), mk(nk)


def _launch(tq, tk, tv, causal, splits, noalloc):
    import torch

    dev = tq.device
    o = torch.full_like(tq, float("nan"))
    ls = torch.full(tq.shape[:3], float("nan"), dtype=torch.float32, device=dev)
    p = capi.tensor_params_ex(tq, tk, tv, o, 0.125, causal, lse=ls)
    stream = torch.cuda.current_stream(dev).cuda_stream
    need = capi.splitkv_workspace_bytes(p, splits)
    assert 0 < need <= capi.SCRATCH_BYTES, need
    if noalloc:
        capi.check(capi.fwd_splitkv_noalloc(p, stream, splits))
    else:
        ws = torch.full((need // 4,), float("nan"), dtype=torch.float32, device=dev)
        capi.check(capi.fwd_splitkv(p, ws.data_ptr(), need, stream, splits))
    torch.cuda.synchronize(dev)
    return o, ls


def test_noalloc_matches_workspace_entry_point(cuda):
    import torch

    for i, (b, h, nq, nk, causal, splits) in enumerate(CALLS):
        print(f"noalloc call {i}: B{b} H{h} Nq{nq} Nk{nk} causal={causal} splits={splits}",
              flush=True)
        q16, k16, v16 = _qkv(b, h, nq, nk, seed=100 + i)
        tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
        o_ws, l_ws = _launch(tq, tk, tv, causal, splits, noalloc=False)
        o_na, l_na = _launch(tq, tk, tv, causal, splits, noalloc=True)
        assert torch.equal(o_na, o_ws), f"call {i}: O differs from the workspace entry point"
        assert torch.equal(l_na, l_ws), f"call {i}: lse differs from the workspace entry point"
        assert_close_oracle(o_na.float().cpu().numpy(), q16, k16, v16, 0.125, causal,
                            ref=attention_fp32(q16, k16, v16, 0.125, causal))


def test_noalloc_rejects_oversized_plan(cuda):
    import torch

    # 16 chunks x 64 heads x 256 rows x 272 bytes = 71 MB of partials
    tq = torch.zeros((4, 16, 256, 64), dtype=torch.float16, device=cuda)
    tk = torch.zeros((4, 16, 4096, 64), dtype=torch.float16, device=cuda)
    o = torch.full_like(tq, 7.0)
    p = capi.tensor_params_ex(tq, tk, tk, o, 0.125, False)
    assert capi.splitkv_workspace_bytes(p, 16) > capi.SCRATCH_BYTES
    rc = capi.fwd_splitkv_noalloc(p, torch.cuda.current_stream(cuda).cuda_stream, 16)
    assert rc == capi.FL_ERR_UNSUPPORTED
    assert "scratch" in capi.last_error()
    torch.cuda.synchronize(cuda)
    assert bool((o == 7.0).all()), "a rejected call launched work"
