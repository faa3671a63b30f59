"""Helpers shared by the GPU tests: run the HIP library through its C ABI on
torch-allocated device memory and compare with the CPU oracle."""

import numpy as np

from flashlite_amd import capi
from oracle import attention_fp32, error_stats

# north_star tolerance for fp16 outputs against the fp32 oracle
MAX_ABS = 2e-3
MEAN_ABS = 2e-4
# bf16: 8x that (unit roundoff 2^-8 against fp16's 2^-11).  The log-sum-exp
# in natural-log units: l sums the rounded p that weight V, so a row whose
# sum one p dominates moves ln l by up to that p's rounding, 2^-11 (fp16)
# or 2^-8 = 3.9e-3 (bf16).
BF16_MAX_ABS = 8 * MAX_ABS
BF16_MEAN_ABS = 8 * MEAN_ABS
LSE_MAX_ABS = {"fp16": 2e-3, "bf16": 4e-3}
LSE_MEAN_ABS = {"fp16": 3e-4, "bf16": 1e-3}

# Tile configurations by name.  The streaming configuration takes key ranges
# of at most 256 keys only.
SLOT_W8_CFG = capi.config_id("br256_bc64_w8_slot")
SLOT_W4_CFG = capi.config_id("br128_bc64_w4_slot")
SPLIT2_CFG = capi.config_id("br128_bc64_w4x2_slot")
SPLIT2W2_CFG = capi.config_id("br64_bc64_w2x2_slot")
PAIR_CFG = capi.config_id("br128_bc64_w4x2_pair")
PAIR64_CFG = capi.config_id("br64_bc64_w2x2_pair")
STREAM_CFG = capi.config_id("br256_kv256_w8_stream")
STREAM_MAX_KEYS = 256
QUARTER_CFG = capi.config_id("br32_kv512_w4_quarters")
QUARTER_MAX_KEYS = 512
# configuration -> the N_k limit it is built for (the others take any N_k)
KEY_LIMITS = {STREAM_CFG: STREAM_MAX_KEYS, QUARTER_CFG: QUARTER_MAX_KEYS}


def config_fits(config, n_k):
    return n_k <= KEY_LIMITS.get(config, n_k)


def to_dev(x, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def run_capi(q16, k16, v16, sm_scale, causal, dev, config=-1, naive=False, out_fill=float("nan")):
    """Launch through the C ABI; unwritten outputs stay NaN and fail later."""
    import torch

    tq, tk, tv = (to_dev(x, dev) for x in (q16, k16, v16))
    o = torch.full_like(tq, out_fill)
    p = capi.tensor_params(tq, tk, tv, o, sm_scale, causal)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = capi.naive(p, stream) if naive else capi.fwd(p, stream, config)
    capi.check(rc)
    torch.cuda.synchronize(dev)
    return o.cpu().numpy()


def wide_tol(kind):
    """(max-abs, mean-abs) bound of an output of element type `kind`."""
    return (BF16_MAX_ABS, BF16_MEAN_ABS) if kind == "bf16" else (MAX_ABS, MEAN_ABS)


def wide_inputs(kind, b, h, nq, nk, d, seed, qk_scale=1.0):
    """Seeded inputs (float32 arrays of the element type's values)."""
    rs = np.random.RandomState(seed)
    mk = lambda n, c: (rs.standard_normal((b, h, n, d)) * c).astype(np.float32)  # noqa: E731
    q, k, v = mk(nq, qk_scale), mk(nk, qk_scale), mk(nk, 1.0)
    if kind == "bf16":
        from flashlite_amd.workloads import round_bf16

        return tuple(round_bf16(x) for x in (q, k, v))
    return tuple(x.astype(np.float16).astype(np.float32) for x in (q, k, v))


def run_wide(kind, q, k, v, sm_scale, causal, dev, config=-1, lse=False, views=None):
    """fp16 or bf16 (`kind`) at any head dim through fl_attn_fwd_{f16,bf16}_ex;
    `views` maps the contiguous tensors to the strided ones to pass (default:
    the contiguous tensors).  Returns (O, log-sum-exp or None) as float32."""
    import torch

    dt = torch.bfloat16 if kind == "bf16" else torch.float16
    tq, tk, tv = (torch.from_numpy(np.ascontiguousarray(x)).to(dev).to(dt) for x in (q, k, v))
    o = torch.full_like(tq, float("nan"))
    if views is not None:
        tq, tk, tv, o = views(tq, tk, tv, o)
    ls = torch.full(tq.shape[:3], float("nan"), dtype=torch.float32, device=dev) if lse else None
    p = capi.tensor_params_ex(tq, tk, tv, o, sm_scale, causal, lse=ls)
    stream = torch.cuda.current_stream(dev).cuda_stream
    fn = capi.fwd_bf16_ex if kind == "bf16" else capi.fwd_ex
    capi.check(fn(p, stream, config))
    torch.cuda.synchronize(dev)
    return o.float().cpu().numpy(), (ls.cpu().numpy() if lse else None)


def run_splitkv(tq, tk, tv, sm_scale, causal, splits, lse=True, o_fill=float("nan")):
    """Split-KV through fl_attn_fwd_f16_splitkv with a NaN-filled workspace of
    exactly the size the library asks for; returns (O, log-sum-exp or None,
    workspace bytes) as device tensors."""
    import torch

    dev = tq.device
    o = torch.full_like(tq, o_fill)
    ls = torch.full(tq.shape[:3], float("nan"), dtype=torch.float32, device=dev) if lse else None
    p = capi.tensor_params_ex(tq, tk, tv, o, sm_scale, causal, lse=ls)
    need = capi.splitkv_workspace_bytes(p, splits)
    assert need >= 0, capi.last_error()
    ws = torch.full((max(need, 4) // 4,), float("nan"), dtype=torch.float32, device=dev)
    capi.check(capi.fwd_splitkv(p, ws.data_ptr() if need else 0, need,
                                torch.cuda.current_stream(dev).cuda_stream, splits))
    torch.cuda.synchronize(dev)
    return o, ls, need


def sample_rows(n, count=256, seed=0):
    """Query rows to check on big shapes: both ends, block edges, random."""
    rs = np.random.RandomState(seed)
    rows = set(range(min(n, 40))) | set(range(max(0, n - 40), n))
    for edge in range(0, n, 128):
        for r in (edge - 1, edge, edge + 31, edge + 32, edge + 63, edge + 64):
            if 0 <= r < n:
                rows.add(r)
    rows |= set(rs.randint(0, n, size=min(count, n)).tolist())
    return np.array(sorted(rows), dtype=np.int64)


def half_ulp(ref, mant_bits=10):
    """Half a unit in the last place of |ref| in a binary format with
    `mant_bits` stored significand bits (10: fp16, 7: bf16), elementwise:
    2^(floor(log2 |x|) - mant_bits - 1), floored at fp16's subnormal step."""
    _, e = np.frexp(np.abs(np.asarray(ref, dtype=np.float64)))  # |x| = f 2^e, f in [0.5, 1)
    e = np.where(np.asarray(ref) == 0, -64, e)
    return np.ldexp(1.0, np.maximum(e - 1 - mant_bits - 1, -25))


def assert_close_oracle(out, q16, k16, v16, sm_scale, causal, rows=None, max_abs=MAX_ABS,
                        mean_abs=MEAN_ABS, ref=None, peaked=False, mant_bits=10):
    """max-abs <= max_abs and mean-abs <= mean_abs against the fp32 oracle.

    peaked=True (a nearly one-hot softmax, |O| near a single V row of 4-5):
    the max-abs bound holds per element on top of the output's own rounding,
    |out - ref| <= max_abs + half_ulp(|ref|); the mean bound is unchanged."""
    if ref is None:
        ref = attention_fp32(q16, k16, v16, sm_scale, causal, rows=rows)
    got = out if rows is None else out[:, :, rows]
    assert np.isfinite(got).all(), "non-finite (or unwritten) outputs"
    mx, mean = error_stats(got, ref)
    if peaked:
        err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
        excess = err - (max_abs + half_ulp(ref, mant_bits))
        worst = np.unravel_index(np.argmax(excess), excess.shape)
        assert excess[worst] <= 0, (
            f"element {worst}: |out - ref| {err[worst]:.3e} above {max_abs:.1e} + half-ulp of "
            f"|ref| {abs(float(ref[worst])):.3e}")
        assert mean <= mean_abs, f"mean-abs {mean:.3e}"
    else:
        assert mx <= max_abs and mean <= mean_abs, f"max-abs {mx:.3e} mean-abs {mean:.3e}"
    return mx, mean


def redo_expected(q16, k16, sm_scale, causal):
    """True when a branch-free first pass with a per-tile range check (the
    pipelined, streaming and head_dim-128 kernels) must hand the block to
    its checked pass: some row has, in a 64-key tile after its first, a lane
    half (32 of the 64 keys) whose sum of 2^(s - m0) exceeds 2^15, m0 being
    the row's max over the first tile and s its base-2 logits.  (The
    slot-scheduled kernels take m0 over the first tile's first 32 keys and
    check once, at the end: a p past fp16's range (2^16) or a row sum past
    2^40 hands the block over.  The peaked inputs of the tests reach gaps
    of 2^30 and more, which does both.)"""
    import numpy as np

    log2e = float(np.float32(1.4426950408889634))
    q = q16.astype(np.float64)
    k = k16.astype(np.float64)
    nq, nk = q.shape[2], k.shape[2]
    s = np.einsum("bhid,bhjd->bhij", q, k) * abs(sm_scale) * log2e
    if sm_scale < 0:
        s = -s
    if causal:  # bottom-right aligned: key j is visible to row i when j <= i + nk - nq
        vis = np.arange(nk)[None, :] <= np.arange(nq)[:, None] + (nk - nq)
        s = np.where(vis, s, -np.inf)
    m0 = s[..., :64].max(axis=-1, keepdims=True)
    # key j of a tile sits in lane half ((j % 32) // 4) % 2
    half = ((np.arange(64) % 32) // 4) % 2
    for t0 in range(64, nk, 64):
        p = np.exp2(np.minimum(s[..., t0:t0 + 64] - m0, 200.0))
        h = half[: p.shape[-1]]
        for g in (0, 1):
            if (p[..., h == g].sum(axis=-1) > 2.0 ** 15).any():
                return True
    return False
