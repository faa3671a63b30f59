"""ctypes view of the C ABI in ``include/flashlite_attn.h``.

This is the binding a non-torch host (or a test) uses to reach the HIP
library directly: raw device pointers, sizes, an opaque ``hipStream_t``.
Loading the library does not touch the GPU.
"""

from __future__ import annotations

import ctypes
import os

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libflashlite_attn.so")

FL_OK = 0
FL_ERR_INVALID_ARGUMENT = 1
FL_ERR_UNSUPPORTED = 2
FL_ERR_MISALIGNED = 3
FL_ERR_LAUNCH = 4
FL_ERR_BAD_CONFIG = 5

# Every symbol the header declares.
EXPORTED = (
    "fl_attn_fwd_f16",
    "fl_attn_fwd_f16_cfg",
    "fl_attn_naive_f16",
    "fl_attn_last_error",
    "fl_attn_num_configs",
    "fl_attn_config_name",
    "fl_attn_select_config",
    "fl_attn_fwd_f16_ex",
    "fl_attn_fwd_bf16_ex",
    "fl_attn_splitkv_workspace_bytes",
    "fl_attn_fwd_f16_splitkv",
    "fl_attn_fwd_f16_splitkv_noalloc",
    "fl_attn_splitkv_noalloc_bytes",
    "fl_attn_config_id",
)

SCRATCH_BYTES = 8 << 20  # FL_ATTN_SCRATCH_BYTES


class FlAttnParams(ctypes.Structure):
    """Mirror of ``fl_attn_params``."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("batch", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("seq_q", ctypes.c_int64),
        ("seq_k", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("sm_scale", ctypes.c_double),
        ("causal", ctypes.c_int32),
    ]


class FlAttnParamsEx(ctypes.Structure):
    """Mirror of ``fl_attn_params_ex``: strides {batch, head, row} in elements."""

    _fields_ = [
        ("base", FlAttnParams),
        ("q_stride", ctypes.c_int64 * 3),
        ("k_stride", ctypes.c_int64 * 3),
        ("v_stride", ctypes.c_int64 * 3),
        ("o_stride", ctypes.c_int64 * 3),
        ("lse", ctypes.c_void_p),
    ]


class FlashLiteError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load ``libflashlite_attn.so`` (once) and declare its signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built; run `python flashlite_amd/build.py`")
    lib = ctypes.CDLL(path)
    P = ctypes.POINTER(FlAttnParams)
    lib.fl_attn_fwd_f16.argtypes = [P, ctypes.c_void_p]
    lib.fl_attn_fwd_f16.restype = ctypes.c_int
    lib.fl_attn_fwd_f16_cfg.argtypes = [P, ctypes.c_int32, ctypes.c_void_p]
    lib.fl_attn_fwd_f16_cfg.restype = ctypes.c_int
    lib.fl_attn_naive_f16.argtypes = [P, ctypes.c_void_p]
    lib.fl_attn_naive_f16.restype = ctypes.c_int
    lib.fl_attn_last_error.argtypes = []
    lib.fl_attn_last_error.restype = ctypes.c_char_p
    lib.fl_attn_num_configs.argtypes = []
    lib.fl_attn_num_configs.restype = ctypes.c_int
    lib.fl_attn_config_name.argtypes = [ctypes.c_int32]
    lib.fl_attn_config_name.restype = ctypes.c_char_p
    lib.fl_attn_select_config.argtypes = [P]
    lib.fl_attn_select_config.restype = ctypes.c_int
    lib.fl_attn_fwd_f16_ex.argtypes = [ctypes.POINTER(FlAttnParamsEx), ctypes.c_int32,
                                       ctypes.c_void_p]
    lib.fl_attn_fwd_f16_ex.restype = ctypes.c_int
    lib.fl_attn_fwd_bf16_ex.argtypes = [ctypes.POINTER(FlAttnParamsEx), ctypes.c_int32,
                                        ctypes.c_void_p]
    lib.fl_attn_fwd_bf16_ex.restype = ctypes.c_int
    lib.fl_attn_splitkv_workspace_bytes.argtypes = [ctypes.POINTER(FlAttnParamsEx), ctypes.c_int32]
    lib.fl_attn_splitkv_workspace_bytes.restype = ctypes.c_int64
    lib.fl_attn_fwd_f16_splitkv.argtypes = [ctypes.POINTER(FlAttnParamsEx), ctypes.c_int32,
                                            ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    lib.fl_attn_fwd_f16_splitkv.restype = ctypes.c_int
    lib.fl_attn_fwd_f16_splitkv_noalloc.argtypes = [ctypes.POINTER(FlAttnParamsEx), ctypes.c_int32,
                                                    ctypes.c_void_p]
    lib.fl_attn_fwd_f16_splitkv_noalloc.restype = ctypes.c_int
    lib.fl_attn_splitkv_noalloc_bytes.argtypes = [ctypes.POINTER(FlAttnParamsEx), ctypes.c_int32]
    lib.fl_attn_splitkv_noalloc_bytes.restype = ctypes.c_int64
    lib.fl_attn_config_id.argtypes = [ctypes.c_char_p]
    lib.fl_attn_config_id.restype = ctypes.c_int
    _lib = lib
    return lib


def make_params(q=0, k=0, v=0, o=0, batch=1, heads=1, seq_q=1, seq_k=None, head_dim=64,
                sm_scale=0.0, causal=False) -> FlAttnParams:
    """Build a params struct from raw addresses (ints) and sizes."""
    return FlAttnParams(q or None, k or None, v or None, o or None, batch, heads, seq_q,
                        seq_q if seq_k is None else seq_k, head_dim, float(sm_scale),
                        1 if causal else 0)


def last_error() -> str:
    msg = load().fl_attn_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    if rc != FL_OK:
        raise FlashLiteError(rc, last_error())


def fwd(params: FlAttnParams, stream: int = 0, config: int = -1) -> int:
    """``fl_attn_fwd_f16_cfg``; returns the status code."""
    return load().fl_attn_fwd_f16_cfg(ctypes.byref(params), config, stream or None)


def fwd_ex(params: FlAttnParamsEx, stream: int = 0, config: int = -1) -> int:
    """``fl_attn_fwd_f16_ex``; returns the status code."""
    return load().fl_attn_fwd_f16_ex(ctypes.byref(params), config, stream or None)


def fwd_bf16_ex(params: FlAttnParamsEx, stream: int = 0, config: int = -1) -> int:
    """``fl_attn_fwd_bf16_ex``; returns the status code."""
    return load().fl_attn_fwd_bf16_ex(ctypes.byref(params), config, stream or None)


def splitkv_workspace_bytes(params: FlAttnParamsEx, num_splits: int = 0) -> int:
    """``fl_attn_splitkv_workspace_bytes``: 0 = no split, -1 = rejected."""
    return load().fl_attn_splitkv_workspace_bytes(ctypes.byref(params), num_splits)


def fwd_splitkv(params: FlAttnParamsEx, workspace: int, workspace_bytes: int, stream: int = 0,
                num_splits: int = 0) -> int:
    """``fl_attn_fwd_f16_splitkv``; returns the status code."""
    return load().fl_attn_fwd_f16_splitkv(ctypes.byref(params), num_splits, workspace or None,
                                          workspace_bytes, stream or None)


def splitkv_noalloc_bytes(params: FlAttnParamsEx, num_splits: int = 0) -> int:
    """``fl_attn_splitkv_noalloc_bytes``: scratch bytes the allocation-free
    call uses (0 = one pass, -1 = rejected)."""
    return load().fl_attn_splitkv_noalloc_bytes(ctypes.byref(params), num_splits)


def fwd_splitkv_noalloc(params: FlAttnParamsEx, stream: int = 0, num_splits: int = 0) -> int:
    """``fl_attn_fwd_f16_splitkv_noalloc`` (partials in the library's scratch
    array); returns the status code."""
    return load().fl_attn_fwd_f16_splitkv_noalloc(ctypes.byref(params), num_splits, stream or None)


def make_params_ex(base: FlAttnParams, q_stride, k_stride, v_stride, o_stride,
                   lse: int = 0) -> FlAttnParamsEx:
    """Extended params from a base struct, four {batch, head, row} stride
    triples (elements) and an optional lse address."""
    t3 = ctypes.c_int64 * 3
    return FlAttnParamsEx(base, t3(*q_stride), t3(*k_stride), t3(*v_stride), t3(*o_stride),
                          lse or None)


def tensor_params_ex(q, k, v, o, sm_scale=0.0, causal=False, lse=None) -> FlAttnParamsEx:
    """Extended params for strided [B, H, N, D] torch views (unit-stride D)."""
    base = tensor_params(q, k, v, o, sm_scale, causal)
    strides = [tuple(int(s) for s in t.stride()[:3]) for t in (q, k, v, o)]
    return make_params_ex(base, *strides, lse=0 if lse is None else lse.data_ptr())


def naive(params: FlAttnParams, stream: int = 0) -> int:
    """``fl_attn_naive_f16``; returns the status code."""
    return load().fl_attn_naive_f16(ctypes.byref(params), stream or None)


def num_configs() -> int:
    return load().fl_attn_num_configs()


def config_name(cfg: int) -> str | None:
    n = load().fl_attn_config_name(cfg)
    return n.decode() if n else None


def config_id(name: str) -> int:
    """``fl_attn_config_id``: index of the tile configuration called `name`
    (KeyError if none)."""
    i = load().fl_attn_config_id(name.encode())
    if i < 0:
        raise KeyError(name)
    return i


def select_config(params: FlAttnParams) -> int:
    return load().fl_attn_select_config(ctypes.byref(params))


def tensor_params(q, k, v, o, sm_scale=0.0, causal=False) -> FlAttnParams:
    """Params for torch tensors q, k, v, o of shape [B, H, N, D] (device memory)."""
    b, h, n, d = q.shape
    return make_params(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), b, h, n,
                       k.shape[2], d, sm_scale, causal)
