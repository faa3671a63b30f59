"""The C-ABI library on a machine without a GPU: it loads, exports every
symbol the header declares, and rejects bad arguments before any launch.
No call here reaches the GPU (each returns from validation)."""

import ctypes
import os
import re

import pytest

from flashlite_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flashlite_attn.h")

# Fake, 256-byte aligned device addresses: never dereferenced by these tests.
A = 0x7F0000000000
STREAM = capi.config_id("br256_kv256_w8_stream")


def test_library_loads_and_exports_header_symbols():
    lib = capi.load()
    with open(HEADER) as f:
        text = f.read()
    declared = set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(fl_\w+)\s*\(", text, re.M))
    assert declared == set(capi.EXPORTED)
    for name in declared:
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)


def test_config_table():
    assert capi.num_configs() == 10
    names = [capi.config_name(i) for i in range(10)]
    # ids are stable: a new configuration is appended, never inserted
    assert names == ["br32_bc64_w1", "br64_bc64_w2", "br128_bc64_w4x2_slot", "br256_bc64_w8_slot",
                     "br128_bc64_w4_slot", "br256_kv256_w8_stream", "br32_kv512_w4_quarters",
                     "br64_bc64_w2x2_slot", "br128_bc64_w4x2_pair", "br64_bc64_w2x2_pair"]
    assert capi.config_name(10) is None and capi.config_name(-1) is None
    assert capi.config_id("br256_bc64_w8_slot") == 3


def _p(**kw):
    base = dict(q=A, k=A + 0x100000, v=A + 0x200000, o=A + 0x300000, batch=2, heads=8,
                seq_q=4096, head_dim=64, sm_scale=0.125, causal=False)
    base.update(kw)
    return capi.make_params(**base)


def test_null_params():
    lib = capi.load()
    assert lib.fl_attn_fwd_f16(None, None) == capi.FL_ERR_INVALID_ARGUMENT
    assert "NULL" in capi.last_error()
    assert lib.fl_attn_naive_f16(None, None) == capi.FL_ERR_INVALID_ARGUMENT


def test_head_dim_must_be_64_for_flash2():
    assert capi.fwd(_p(head_dim=128)) == capi.FL_ERR_UNSUPPORTED
    assert capi.last_error() == "FlashLite WMMA kernel currently requires head_dim == 64"


def test_seq_k_may_differ_from_seq_q():
    # validated (no launch): the dispatcher picks a configuration
    assert capi.select_config(_p(seq_k=100)) >= 0
    assert capi.select_config(_p(seq_q=1, seq_k=4096, causal=True)) >= 0
    # the key-side limits are checked on N_k
    assert capi.select_config(_p(seq_q=16, seq_k=1 << 24)) == -1
    assert "N_k" in capi.last_error()
    assert capi.naive(_p(seq_q=16, seq_k=1 << 20)) == capi.FL_ERR_UNSUPPORTED
    assert "N_k" in capi.last_error()


def _ex(q_stride=(8 * 4096 * 64, 4096 * 64, 64), k_stride=None, v_stride=None, o_stride=None,
        lse=0, **kw):
    c = (8 * 4096 * 64, 4096 * 64, 64)
    return capi.make_params_ex(_p(**kw), q_stride, k_stride or c, v_stride or c, o_stride or c,
                               lse)


def test_ex_null_and_config():
    lib = capi.load()
    assert lib.fl_attn_fwd_f16_ex(None, -1, None) == capi.FL_ERR_INVALID_ARGUMENT
    assert capi.fwd_ex(_ex(), config=capi.num_configs()) == capi.FL_ERR_BAD_CONFIG
    # the streaming configuration needs N_k <= 256 (rejected before any pointer check)
    assert capi.fwd_ex(_ex(), config=STREAM) == capi.FL_ERR_BAD_CONFIG
    assert "needs N_k <= 256" in capi.last_error()
    assert capi.fwd_ex(_ex(head_dim=128)) == capi.FL_ERR_UNSUPPORTED


def test_ex_stride_checks():
    # not a multiple of 8 elements (rows would lose 16-byte alignment)
    assert capi.fwd_ex(_ex(q_stride=(8 * 4096 * 64, 4096 * 64, 68))) == capi.FL_ERR_UNSUPPORTED
    assert "multiples of 8" in capi.last_error()
    assert capi.fwd_ex(_ex(k_stride=(4, 4096 * 64, 64))) == capi.FL_ERR_UNSUPPORTED
    # rows closer than D
    assert capi.fwd_ex(_ex(o_stride=(0, 0, 32))) == capi.FL_ERR_UNSUPPORTED
    assert "row stride" in capi.last_error()
    assert capi.fwd_ex(_ex(v_stride=(-64, 64, 64))) == capi.FL_ERR_UNSUPPORTED
    # [B, N, H, D] strides are fine; K/V rows must stay within 2^31 bytes of the head
    bnhd = (4096 * 8 * 64, 64, 8 * 64)
    big = (1 << 40, 64, 1 << 16)
    assert capi.fwd_ex(_ex(k_stride=big, batch=1, heads=1, seq_q=1 << 14)) == capi.FL_ERR_UNSUPPORTED
    assert "addressing limit" in capi.last_error()
    assert capi.fwd_ex(_ex(q_stride=bnhd, k_stride=bnhd, v_stride=bnhd, o_stride=bnhd,
                           o=0)) == capi.FL_ERR_INVALID_ARGUMENT  # got past the stride checks
    assert "non-NULL" in capi.last_error()


def test_ex_no_keys_ignores_kv_strides_and_pointers():
    # N_k = 0: k and v are never read, so neither their strides nor NULL
    # pointers are errors (o = NULL still is, and shows the checks got there)
    p = _ex(k_stride=(0, 0, 0), v_stride=(0, 0, 0), seq_k=0, k=0, v=0, o=0)
    assert capi.fwd_ex(p) == capi.FL_ERR_INVALID_ARGUMENT
    assert "non-NULL" in capi.last_error()


def test_ex_lse_alignment():
    assert capi.fwd_ex(_ex(lse=A + 2)) == capi.FL_ERR_MISALIGNED
    assert "lse" in capi.last_error()


def test_sequence_addressing_limit():
    # K/V tiles are addressed with 32-bit offsets inside one head
    assert capi.fwd(_p(batch=1, heads=1, seq_q=1 << 24)) == capi.FL_ERR_UNSUPPORTED
    assert "addressing limit" in capi.last_error()


def test_negative_sizes():
    assert capi.fwd(_p(batch=-1)) == capi.FL_ERR_INVALID_ARGUMENT
    assert capi.naive(_p(head_dim=0)) == capi.FL_ERR_INVALID_ARGUMENT


def test_null_pointers_and_alignment():
    assert capi.fwd(_p(o=0)) == capi.FL_ERR_INVALID_ARGUMENT
    assert capi.fwd(_p(k=A + 8)) == capi.FL_ERR_MISALIGNED
    assert "16-byte" in capi.last_error()
    # the naive kernel reads fp16 scalars: 2-byte alignment suffices, 1 does not
    assert capi.naive(_p(k=A + 1, seq_q=16)) == capi.FL_ERR_MISALIGNED


def test_non_finite_scale():
    assert capi.fwd(_p(sm_scale=float("inf"))) == capi.FL_ERR_INVALID_ARGUMENT
    assert capi.fwd(_p(sm_scale=float("nan"))) == capi.FL_ERR_INVALID_ARGUMENT
    assert capi.fwd(_p(sm_scale=1e-300)) == capi.FL_ERR_INVALID_ARGUMENT  # underflows to 0


def test_bad_config():
    assert capi.fwd(_p(), config=capi.num_configs()) == capi.FL_ERR_BAD_CONFIG
    assert capi.fwd(_p(), config=-2) == capi.FL_ERR_BAD_CONFIG
    assert capi.fwd(_p(seq_q=256, seq_k=257), config=STREAM) == capi.FL_ERR_BAD_CONFIG
    assert "needs N_k <= 256" in capi.last_error()
    quarter = capi.config_id("br32_kv512_w4_quarters")
    assert capi.fwd(_p(seq_q=256, seq_k=513), config=quarter) == capi.FL_ERR_BAD_CONFIG
    assert "needs N_k <= 512" in capi.last_error()
    assert capi.fwd_ex(_ex(seq_k=4096), config=quarter) == capi.FL_ERR_BAD_CONFIG
    assert "needs N_k <= 512" in capi.last_error()


def test_empty_problems_are_noops():
    # zero-size work returns OK without touching pointers or the device
    for kw in (dict(seq_q=0), dict(batch=0), dict(heads=0)):
        p = _p(q=0, k=0, v=0, o=0, **kw)
        assert capi.fwd(p) == capi.FL_OK
        assert capi.naive(p) == capi.FL_OK


def test_naive_limits():
    assert capi.naive(_p(seq_q=1 << 20)) == capi.FL_ERR_UNSUPPORTED
    assert "LDS" in capi.last_error()
    assert capi.naive(_p(batch=256, heads=512, seq_q=16)) == capi.FL_ERR_UNSUPPORTED


def test_dispatcher_choices():
    sel = lambda **kw: capi.config_name(capi.select_config(_p(**kw)))  # noqa: E731
    W8, W4, SPLIT, STRM = ("br256_bc64_w8_slot", "br128_bc64_w4_slot", "br128_bc64_w4x2_slot",
                           "br256_kv256_w8_stream")
    W1, W2, QTR = "br32_bc64_w1", "br64_bc64_w2", "br32_kv512_w4_quarters"
    PAIR, PAIR64 = "br128_bc64_w4x2_pair", "br64_bc64_w2x2_pair"
    SPLIT64 = "br64_bc64_w2x2_slot"
    # non-causal: 8-wave 256-row slot-scheduled groups when there are more
    # than 128 and the key range is long
    assert sel(batch=2, heads=8, seq_q=4096) == W8      # 256 groups
    assert sel(batch=1, heads=16, seq_q=16384) == W8
    assert sel(batch=2, heads=8, seq_q=2560) == W8      # 160 groups
    assert sel(batch=4, heads=8, seq_q=2048) == W8
    # short key ranges (N_k <= 256): streaming groups
    assert sel(batch=32, heads=32, seq_q=256) == STRM     # 1024 units
    assert sel(batch=8, heads=32, seq_q=130) == STRM      # 256 units
    assert sel(batch=2, heads=8, seq_q=256) == STRM       # 16 units
    assert sel(batch=1, heads=1, seq_q=1000, seq_k=256) == STRM
    # at most one 128-row group per CU over long key ranges: split key range
    # (non-causal from N_k 4096, or with fewer than 128 groups)
    assert sel(batch=2, heads=8, seq_q=2048) == SPLIT      # 256 groups of 128 rows
    assert sel(batch=2, heads=8, seq_q=2048, causal=True) == SPLIT
    assert sel(batch=1, heads=8, seq_q=4096) == SPLIT
    assert sel(batch=1, heads=1, seq_q=2048) == SPLIT64    # 32 groups of 64 rows
    assert sel(batch=1, heads=8, seq_q=4096, causal=True) == PAIR64   # 256 pairs of 64 rows
    assert sel(batch=1, heads=1, seq_q=1024, seq_k=4096) == SPLIT64
    assert sel(batch=1, heads=1, seq_q=2048, seq_k=8192) == SPLIT64
    assert sel(batch=1, heads=1, seq_q=1000, seq_k=4096) == SPLIT64
    # past 512 keys with 128-256 groups of 64 rows: the split on 64-row groups
    assert sel(batch=2, heads=8, seq_q=1024) == SPLIT64    # 256 groups of 64 rows
    assert sel(batch=2, heads=8, seq_q=1024, causal=True) == SPLIT64
    assert sel(batch=1, heads=8, seq_q=2048) == SPLIT64
    assert sel(batch=1, heads=4, seq_q=4096, causal=True) == SPLIT64
    assert sel(batch=1, heads=8, seq_q=1024) == SPLIT64    # 128 groups
    assert sel(batch=1, heads=1, seq_q=4096) == SPLIT64    # 64 groups
    assert sel(batch=1, heads=1, seq_q=4096, causal=True) == SPLIT64
    assert sel(batch=2, heads=8, seq_q=640) == SPLIT64
    assert sel(batch=2, heads=8, seq_q=513) == W4          # N_k <= 576: 128-row groups
    assert sel(batch=1, heads=1, seq_q=2048, causal=True) == SPLIT64
    assert sel(batch=3, heads=8, seq_q=1024) == W4         # 384 groups of 64 rows
    assert sel(batch=4, heads=4, seq_q=1536, causal=True) == W4
    # causal from N_k 4096 with 257-512 groups of 128 rows: the block pairs;
    # square causal over 2048-4095 keys: the one-block split up to 384
    # groups, the block pairs to 512 from 2560 keys; beyond, 128-row
    # slot-scheduled groups balanced by dispatch order
    assert sel(batch=2, heads=8, seq_q=4096, causal=True) == PAIR
    assert sel(batch=1, heads=8, seq_q=8192, causal=True) == PAIR
    assert sel(batch=4, heads=8, seq_q=4096, causal=True) == W4
    assert sel(batch=2, heads=16, seq_q=2048, causal=True) == W4
    assert sel(batch=2, heads=8, seq_q=4096) == W8
    assert sel(batch=1, heads=16, seq_q=16384, causal=True) == W4
    assert sel(batch=3, heads=8, seq_q=2048, causal=True) == SPLIT   # 384 groups, 2 rounds
    assert sel(batch=2, heads=8, seq_q=3072, causal=True) == SPLIT   # 384 groups
    assert sel(batch=2, heads=10, seq_q=2560, causal=True) == PAIR   # 400 groups
    assert sel(batch=2, heads=8, seq_q=3584, causal=True) == PAIR    # 448 groups
    assert sel(batch=5, heads=8, seq_q=2048, causal=True) == W4      # 640 groups
    assert sel(batch=4, heads=8, seq_q=2048, causal=True) == W4      # 512 groups, N 2048
    assert sel(batch=2, heads=8, seq_q=3072) == W8                   # non-causal
    # at most 32 query rows over at least 256 heads: 4-wave groups
    assert sel(batch=32, heads=32, seq_q=1, seq_k=4096) == W4
    assert sel(batch=8, heads=32, seq_q=1, seq_k=8192) == W4
    assert sel(batch=8, heads=32, seq_q=32, seq_k=8192, causal=True) == W4
    assert sel(batch=4, heads=32, seq_q=1, seq_k=8192) == SPLIT64  # 128 heads
    assert sel(batch=8, heads=32, seq_q=33, seq_k=8192) == SPLIT64  # 33 rows: not this rule
    # square causal from N 4096 with 129-256 pairs of 64-row blocks: the
    # 64-row block pairs (one round)
    assert sel(batch=1, heads=2, seq_q=16384, causal=True) == PAIR64
    assert sel(batch=1, heads=1, seq_q=32768, causal=True) == PAIR64
    assert sel(batch=1, heads=3, seq_q=8192, causal=True) == PAIR64   # 192 pairs
    assert sel(batch=4, heads=2, seq_q=4096, causal=True) == PAIR64
    assert sel(batch=1, heads=4, seq_q=16384, causal=True) == PAIR    # 512 pairs
    assert sel(batch=1, heads=2, seq_q=16384) == SPLIT                # non-causal
    assert sel(batch=1, heads=2, seq_q=16000, seq_k=16384, causal=True) == SPLIT  # N_q != N_k
    assert sel(batch=2, heads=8, seq_q=2048, causal=True) == SPLIT    # N 2048
    assert sel(batch=32, heads=32, seq_q=256, causal=True) == STRM   # streaming, any count
    assert sel(batch=1, heads=1, seq_q=128, causal=True) == STRM
    # 256 < N_k <= 512 with at most 512 blocks of 32 rows: key quarters
    assert sel(batch=2, heads=8, seq_q=512) == QTR      # C1: 256 groups of 32 rows
    assert sel(batch=2, heads=8, seq_q=512, causal=True) == QTR
    assert sel(batch=1, heads=1, seq_q=257, causal=True) == QTR
    assert sel(batch=1, heads=1, seq_q=257) == QTR
    assert sel(batch=1, heads=1, seq_q=100, seq_k=512) == QTR
    # more groups, or longer key ranges: 128-row or smaller groups
    assert sel(batch=4, heads=8, seq_q=512) == QTR      # 512 blocks: 8-wave groups of 64 rows
    assert sel(batch=4, heads=8, seq_q=320, causal=True) == QTR
    assert sel(batch=8, heads=8, seq_q=512) == W4       # 1024 blocks of 32 rows
    assert sel(batch=2, heads=4, seq_q=576) == W2       # 72 groups of 64 rows
    assert sel(batch=1, heads=1, seq_q=600) == SPLIT64     # 10 groups of 64 rows
    assert sel(batch=1, heads=1, seq_q=576) == W1          # N_k <= 576: small groups
    assert capi.select_config(_p(head_dim=80)) == -1


@pytest.mark.parametrize("fn", ["fwd", "naive"])
def test_error_message_is_thread_local(fn):
    import threading

    seen = {}

    def worker():
        getattr(capi, fn)(_p(batch=-1))
        seen["msg"] = capi.last_error()

    capi.fwd(_p(head_dim=128))
    t = threading.Thread(target=worker)
    t.start()
    t.join()
    assert "non-negative" in seen["msg"]
    assert capi.last_error() == "FlashLite WMMA kernel currently requires head_dim == 64"


def test_splitkv_plan():
    c = (8 * 1 * 64, 1 * 64, 64)
    kc = (8 * 4096 * 64, 4096 * 64, 64)

    def bytes_for(nq, nk, splits, batch=2, heads=8, causal=False):
        base = _p(batch=batch, heads=heads, seq_q=nq, seq_k=nk, causal=causal)
        qs = (heads * nq * 64, nq * 64, 64)
        ks = (heads * nk * 64, nk * 64, 64)
        return capi.splitkv_workspace_bytes(capi.make_params_ex(base, qs, ks, ks, qs), splits)

    # decode step B2 H8, one query over 4096 keys: 16 one-wave groups would
    # leave most CUs idle; key-quarter chunks of 8 tiles when they fit one
    # round (16 x 8 groups of 4 waves), else one-wave chunks covering the
    # 256 CUs twice, of at least 4 tiles (multi-wave chunks: once)
    assert bytes_for(1, 4096, 0) == 8 * 16 * 1 * 68 * 4
    assert bytes_for(1, 1 << 16, 0) == 32 * 16 * 1 * 68 * 4
    # fewer than 8 tiles: at most tiles / 4 chunks, and no split below 2
    assert bytes_for(1, 512, 0) == 2 * 16 * 1 * 68 * 4
    assert bytes_for(1, 192, 0) == 0
    # at least half as many one-wave groups as CUs (128 and more): one pass;
    # 64 groups still cut their ranges (8 one-wave chunks: 16 would not fit
    # one round of key-quarter groups)
    assert bytes_for(1, 4096, 0, batch=32, heads=32) == 0
    assert bytes_for(1, 1024, 0, batch=32, heads=32) == 0
    assert bytes_for(16, 4096, 0, batch=32, heads=32) == 0
    assert bytes_for(64, 4096, 0, batch=32, heads=32) == 0
    assert bytes_for(1, 8192, 0, batch=4, heads=32) == 0
    assert bytes_for(1, 8192, 0, batch=2, heads=32) == 8 * 64 * 1 * 68 * 4
    # long query ranges (the headline shape): one pass
    assert bytes_for(4096, 4096, 0) == 0
    assert bytes_for(129, 1 << 16, 0) == 0
    assert bytes_for(128, 1 << 16, 0) == 16 * 16 * 128 * 68 * 4
    assert bytes_for(64, 8192, 0, batch=4) == 8 * 32 * 64 * 68 * 4
    assert bytes_for(1, 4096, 0, batch=4) == 8 * 32 * 1 * 68 * 4      # 256 quarter groups
    assert bytes_for(1, 4096, 0, batch=8) == 8 * 64 * 1 * 68 * 4      # one-wave chunks: 512 / 64
    # forced: as asked, clamped to the number of 64-key tiles
    assert bytes_for(4096, 4096, 5) == 5 * 16 * 4096 * 68 * 4
    assert bytes_for(3, 130, 100) == 3 * 16 * 3 * 68 * 4
    assert bytes_for(1, 1 << 20, 1000) == 256 * 16 * 68 * 4
    # rejected params
    assert bytes_for(1, 4096, 0, heads=-1) == -1


def test_splitkv_workspace_checks():
    qs = (8 * 64, 64, 64)
    ks = (8 * 4096 * 64, 4096 * 64, 64)
    p = capi.make_params_ex(_p(seq_q=1, seq_k=4096), qs, ks, ks, qs)
    need = capi.splitkv_workspace_bytes(p, 0)
    assert need > 0
    assert capi.fwd_splitkv(p, 0, need) == capi.FL_ERR_INVALID_ARGUMENT
    assert "workspace" in capi.last_error() and "NULL" in capi.last_error()
    assert capi.fwd_splitkv(p, A + 0x400000, need - 4) == capi.FL_ERR_INVALID_ARGUMENT
    assert capi.fwd_splitkv(p, A + 0x400008, need) == capi.FL_ERR_MISALIGNED
    assert capi.load().fl_attn_fwd_f16_splitkv(None, 0, None, 0, None) == capi.FL_ERR_INVALID_ARGUMENT


def _ex_shape(batch, heads, nq, nk, causal=False):
    base = _p(batch=batch, heads=heads, seq_q=nq, seq_k=nk, causal=causal)
    qs = (heads * nq * 64, nq * 64, 64)
    ks = (heads * nk * 64, nk * 64, 64)
    return capi.make_params_ex(base, qs, ks, ks, qs)


def test_noalloc_plan_fits_the_scratch_array():
    """Every plan the library chooses for the allocation-free entry point fits
    its static scratch (num_splits <= 0 never fails for lack of scratch): the
    chunk count is lowered to what fits, or the call runs one pass."""
    per_row = 68 * 4
    checked = 0
    for batch, heads in ((1, 1), (1, 16), (2, 8), (4, 8), (8, 16), (32, 32), (64, 64)):
        for nq in (1, 2, 16, 32, 33, 64, 65, 100, 128, 129, 1024):
            for nk in (64, 192, 512, 1000, 4096, 8192, 65536, 1 << 20):
                for causal in (False, True):
                    p = _ex_shape(batch, heads, nq, nk, causal)
                    ws = capi.splitkv_workspace_bytes(p, 0)
                    na = capi.splitkv_noalloc_bytes(p, 0)
                    assert 0 <= na <= capi.SCRATCH_BYTES, (batch, heads, nq, nk, ws, na)
                    assert na % (batch * heads * nq * per_row) == 0
                    if ws <= capi.SCRATCH_BYTES:
                        assert na == ws  # the cap changes only plans that do not fit
                    else:
                        # the most chunks that fit, and never a single chunk
                        per_chunk = batch * heads * nq * per_row
                        fit = capi.SCRATCH_BYTES // per_chunk
                        assert na == (fit * per_chunk if fit >= 2 else 0)
                    checked += 1
    assert checked > 1000


def test_noalloc_plan_of_reported_shapes():
    # B8 H16, 128 query rows over 65536 keys (128 groups): one pass, with or
    # without a workspace; B4 H31 (124 groups): 3 chunks of 124 x 128 rows
    # (12.9 MB) with a workspace, and one 4.3 MB chunk is no split
    p = _ex_shape(8, 16, 128, 65536)
    assert capi.splitkv_workspace_bytes(p, 0) == capi.splitkv_noalloc_bytes(p, 0) == 0
    p = _ex_shape(4, 31, 128, 65536)
    assert capi.splitkv_workspace_bytes(p, 0) == 3 * 124 * 128 * 272
    assert capi.splitkv_noalloc_bytes(p, 0) == 0
    # B32 H32, 32 query rows over 4096 keys (1024 one-wave groups): one pass
    # with or without a workspace; so too the B32 H32 decode step and 16 rows
    # of B16 H64 over 65536 keys
    for shape in ((32, 32, 32, 4096), (32, 32, 1, 4096), (16, 64, 16, 65536)):
        p = _ex_shape(*shape)
        assert capi.splitkv_workspace_bytes(p, 0) == capi.splitkv_noalloc_bytes(p, 0) == 0
    # B4 H16, 128 rows over 1024 keys: 4 chunks of 64 x 128 rows (8.9 MB),
    # lowered to the 3 that fit; B2 H16, 128 rows over 4096 keys: 8 chunks of
    # 32 x 128 rows, lowered to 7
    p = _ex_shape(4, 16, 128, 1024)
    assert capi.splitkv_workspace_bytes(p, 0) == 4 * 64 * 128 * 272
    assert capi.splitkv_noalloc_bytes(p, 0) == 3 * 64 * 128 * 272
    p = _ex_shape(2, 16, 128, 4096)
    assert capi.splitkv_workspace_bytes(p, 0) == 8 * 32 * 128 * 272
    assert capi.splitkv_noalloc_bytes(p, 0) == 7 * 32 * 128 * 272
    # a requested count is kept as asked, even when it will be refused
    p = _ex_shape(4, 16, 256, 4096)
    assert capi.splitkv_noalloc_bytes(p, 16) == capi.splitkv_workspace_bytes(p, 16) \
        == 16 * 64 * 256 * 272
    assert capi.splitkv_noalloc_bytes(_ex_shape(1, -1, 1, 4096), 0) == -1


def test_config_id_lookup():
    for i in range(capi.num_configs()):
        assert capi.load().fl_attn_config_id(capi.config_name(i).encode()) == i
    assert capi.load().fl_attn_config_id(b"br128_bc64_w4_slot") == 4
    assert capi.load().fl_attn_config_id(b"no_such_config") == -1
    assert capi.load().fl_attn_config_id(None) == -1
    with pytest.raises(KeyError):
        capi.config_id("no_such_config")
