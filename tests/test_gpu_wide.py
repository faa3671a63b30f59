"""GPU parity of the paths beyond the reference's element type and head dim:
head_dim 128 (fp16 and bf16) and bf16 at head_dim 64, through the C ABI
(``fl_attn_fwd_f16_ex`` / ``fl_attn_fwd_bf16_ex``) and the binding
(``forward_flash2_ex``).  The reference accepts fp16 at D = 64 only
(csrc/kernel_flash2.cu:745-757).

Tolerances against the fp32 oracle on the same inputs:
* fp16 (any head dim): the north_star bound, max-abs <= 2e-3, mean-abs <= 2e-4.
* bf16: 8x that, max-abs <= 1.6e-2 and mean-abs <= 1.6e-3.  bf16 keeps 8
  significand bits against fp16's 11, so its unit roundoff (2^-8) is 8x
  fp16's (2^-11); the output rounding alone reaches 2^-9 |O| and P is
  rounded to bf16 before the PV product.  The inputs are bf16-exact values
  (``workloads.round_bf16``), so the oracle sees exactly what the kernel reads.
* log-sum-exp (natural-log units): max-abs <= 2e-3 for fp16 and 4e-3 for
  bf16; mean-abs <= 3e-4 for fp16 and 1e-3 for bf16.  Every path keeps Q
  unscaled and scales the fp32 scores, as the reference does; but at D = 64
  the row sum l is taken on the matrix core over the rounded p that weight V,
  so that O is normalised by exactly its weights.  A bf16 p carries a
  relative rounding error of up to 2^-8 = 3.9e-3 (about 2^-10 on average),
  and on a row whose sum one p dominates ln l moves by up to that much
  (2.9e-3 measured on a seeded random shape at sm_scale -0.3).
A strided launch equals the contiguous launch of the same data bit for bit.
"""

import numpy as np
import pytest

from flashlite_amd import capi
from gpu_util import (BF16_MAX_ABS, BF16_MEAN_ABS, LSE_MAX_ABS, LSE_MEAN_ABS, MAX_ABS, MEAN_ABS,
                      PAIR64_CFG, PAIR_CFG, QUARTER_CFG, SLOT_W4_CFG, SLOT_W8_CFG, SPLIT2_CFG,
                      SPLIT2W2_CFG, STREAM_CFG, half_ulp, sample_rows)
from gpu_util import run_wide as _run
from gpu_util import wide_inputs as _inputs
from gpu_util import wide_tol as _tol
from oracle import attention_fp32, attention_lse, error_stats

pytestmark = pytest.mark.gpu

SLOT_CFGS = [-1, SLOT_W8_CFG, SLOT_W4_CFG]
KINDS = [("fp16", 64), ("fp16", 128), ("bf16", 64), ("bf16", 128)]
WIDE = [k for k in KINDS if k != ("fp16", 64)]




def _check(kind, out, ref, what):
    mx_tol, mean_tol = _tol(kind)
    assert np.isfinite(out).all(), f"{what}: non-finite (or unwritten) outputs"
    mx, mean = error_stats(out, ref)
    assert mx <= mx_tol and mean <= mean_tol, f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e}"
    return mx, mean


RAGGED = [1, 17, 31, 32, 33, 63, 64, 65, 100, 129, 257, 513]


@pytest.mark.parametrize("kind,d", WIDE)
@pytest.mark.parametrize("config", SLOT_CFGS)
@pytest.mark.parametrize("causal", [False, True])
def test_ragged(cuda, kind, d, config, causal):
    for n in RAGGED:
        q, k, v = _inputs(kind, 2, 3, n, n, d, seed=2000 + n + d)
        out, _ = _run(kind, q, k, v, 0.0, causal, cuda, config=config)
        _check(kind, out, attention_fp32(q, k, v, 0.0, causal), f"N={n}")


RECT = [(1, 1), (1, 300), (5, 64), (37, 100), (100, 37), (64, 65), (200, 513), (513, 200),
        (129, 1000), (1000, 129)]


@pytest.mark.parametrize("kind,d", WIDE)
@pytest.mark.parametrize("config", [SLOT_W8_CFG, SLOT_W4_CFG])
@pytest.mark.parametrize("causal", [False, True])
def test_rectangular_with_lse(cuda, kind, d, config, causal):
    for nq, nk in RECT:
        q, k, v = _inputs(kind, 1, 2, nq, nk, d, seed=nq * 7 + nk + d)
        out, lse = _run(kind, q, k, v, 0.125, causal, cuda, config=config, lse=True)
        ref = attention_fp32(q, k, v, 0.125, causal)
        _check(kind, out, ref, f"{nq}x{nk}")
        ref_lse = attention_lse(q, k, 0.125, causal)
        fin = np.isfinite(ref_lse)
        assert np.array_equal(fin, np.isfinite(lse)), f"{nq}x{nk}: lse -inf pattern"
        mx, mean = error_stats(lse[fin], ref_lse[fin]) if fin.any() else (0.0, 0.0)
        assert mx <= LSE_MAX_ABS[kind] and mean <= LSE_MEAN_ABS[kind], (
            f"{nq}x{nk}: lse max-abs {mx:.3e} mean-abs {mean:.3e}")


@pytest.mark.parametrize("kind,d", KINDS)
@pytest.mark.parametrize("causal", [False, True])
def test_headline_shape(cuda, kind, d, causal):
    """B2 H8 N4096 at each element type and head dim, sampled rows."""
    q, k, v = _inputs(kind, 2, 8, 4096, 4096, d, seed=77 + d)
    out, _ = _run(kind, q, k, v, 0.125, causal, cuda)
    rows = sample_rows(4096, seed=d)
    ref = attention_fp32(q, k, v, 0.125, causal, rows=rows)
    _check(kind, out[:, :, rows], ref, f"{kind} D={d}")


@pytest.mark.parametrize("kind,d", WIDE)
@pytest.mark.parametrize("scale,sm", [(1.0, 1.0), (3.0, 1.0), (1.0, -0.3)])
def test_peaked_and_negative_scales(cuda, kind, d, scale, sm):
    """Large and negative scales: the stabiliser's checked pass and the sign
    flip.  For |scale| >= 1 the output nears a single V row (|O| ~ 4-5), and
    the max-abs bound holds per element on top of the output's own half-ulp
    (2^-12 |O| in fp16, 2^-9 |O| in bf16), as in the fp16 tests."""
    q, k, v = _inputs(kind, 1, 2, 300, 300, d, seed=31, qk_scale=scale)
    for causal in (False, True):
        out, _ = _run(kind, q, k, v, sm, causal, cuda)
        ref = attention_fp32(q, k, v, sm, causal)
        mx_tol, mean_tol = _tol(kind)
        mx, mean = error_stats(out, ref)
        assert np.isfinite(out).all()
        assert mean <= mean_tol, f"causal={causal}: mean-abs {mean:.3e}"
        if abs(sm) >= 1.0:
            bound = mx_tol + half_ulp(ref, 7 if kind == "bf16" else 10)
            assert (np.abs(out.astype(np.float64) - ref) <= bound).all(), (
                f"causal={causal}: max-abs {mx:.3e} above {mx_tol:.1e} + half-ulp")
        else:
            assert mx <= mx_tol, f"causal={causal}: max-abs {mx:.3e}"


@pytest.mark.parametrize("kind,d", WIDE)
@pytest.mark.parametrize("causal", [False, True])
def test_strided_bit_exact(cuda, kind, d, causal):
    """[B, N, H, D] views (the flash_attn layout) and padded rows give the
    same bits as the contiguous launch."""
    import torch

    q, k, v = _inputs(kind, 2, 3, 200, 333, d, seed=5 + d)
    base, _ = _run(kind, q, k, v, 0.125, causal, cuda)

    def bnhd(tq, tk, tv, o):
        f = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)  # noqa: E731
        return f(tq), f(tk), f(tv), f(o)

    def padded(tq, tk, tv, o):
        def pad(t):
            b, h, n, dd = t.shape
            big = torch.zeros((b, h, n, dd + 64), dtype=t.dtype, device=t.device)
            big[..., :dd] = t
            return big[..., :dd]
        return pad(tq), pad(tk), pad(tv), pad(o)

    for views in (bnhd, padded):
        out, _ = _run(kind, q, k, v, 0.125, causal, cuda, views=views)
        assert np.array_equal(out, base), views.__name__


@pytest.mark.parametrize("config", [SPLIT2_CFG, SPLIT2W2_CFG, PAIR_CFG, PAIR64_CFG])
@pytest.mark.parametrize("causal", [False, True])
def test_bf16_key_range_splits(cuda, config, causal):
    """bf16 at D = 64 on the key-range splits (128- and 64-row groups, and
    the 128- and 64-row block pairs):
    ragged lengths, every output row of B1 H4 N1024, and a peaked scale whose
    row sums leave the first pass's range (the checked pass)."""
    for n in RAGGED:
        q, k, v = _inputs("bf16", 2, 3, n, n, 64, seed=3000 + n)
        out, _ = _run("bf16", q, k, v, 0.0, causal, cuda, config=config)
        _check("bf16", out, attention_fp32(q, k, v, 0.0, causal), f"N={n}")
    q, k, v = _inputs("bf16", 1, 4, 1024, 1024, 64, seed=41)
    out, _ = _run("bf16", q, k, v, 0.125, causal, cuda, config=config)
    _check("bf16", out, attention_fp32(q, k, v, 0.125, causal), "B1 H4 N1024")
    q, k, v = _inputs("bf16", 1, 2, 700, 700, 64, seed=43, qk_scale=3.0)
    out, _ = _run("bf16", q, k, v, 1.0, causal, cuda, config=config)
    ref = attention_fp32(q, k, v, 1.0, causal)
    mx_tol, mean_tol = _tol("bf16")
    assert np.isfinite(out).all()
    assert error_stats(out, ref)[1] <= mean_tol
    assert (np.abs(out.astype(np.float64) - ref) <= mx_tol + half_ulp(ref, 7)).all()


@pytest.mark.parametrize("config", [STREAM_CFG, QUARTER_CFG])
@pytest.mark.parametrize("causal", [False, True])
def test_bf16_short_key_kernels(cuda, config, causal):
    """bf16 at D = 64 on the streaming (N_k <= 256) and key-quarter (N_k <=
    512) kernels: ragged lengths, N_k != N_q with the log-sum-exp, many heads
    (several units per streaming group; two-block key-quarter groups) and a
    peaked scale."""
    limit = 256 if config == STREAM_CFG else 512
    for n in [x for x in RAGGED if x <= limit]:
        q, k, v = _inputs("bf16", 2, 3, n, n, 64, seed=4000 + n)
        out, _ = _run("bf16", q, k, v, 0.0, causal, cuda, config=config)
        _check("bf16", out, attention_fp32(q, k, v, 0.0, causal), f"N={n}")
    for nq, nk in [(37, 100), (100, 37), (300, limit), (limit, 130)]:
        q, k, v = _inputs("bf16", 1, 2, nq, nk, 64, seed=nq * 7 + nk)
        out, lse = _run("bf16", q, k, v, 0.125, causal, cuda, config=config, lse=True)
        _check("bf16", out, attention_fp32(q, k, v, 0.125, causal), f"{nq}x{nk}")
        ref_lse = attention_lse(q, k, 0.125, causal)
        fin = np.isfinite(ref_lse)
        assert np.array_equal(fin, np.isfinite(lse)), f"{nq}x{nk}: lse -inf pattern"
        mx, mean = error_stats(lse[fin], ref_lse[fin]) if fin.any() else (0.0, 0.0)
        assert mx <= LSE_MAX_ABS["bf16"] and mean <= LSE_MEAN_ABS["bf16"], f"{nq}x{nk}: lse {mx:.3e}"
    b, h, n = (32, 32, 256) if config == STREAM_CFG else (4, 8, 512)
    q, k, v = _inputs("bf16", b, h, n, n, 64, seed=7)
    out, _ = _run("bf16", q, k, v, 0.125, causal, cuda, config=config)
    _check("bf16", out, attention_fp32(q, k, v, 0.125, causal), f"B{b} H{h} N{n}")
    q, k, v = _inputs("bf16", 1, 2, 200, 200, 64, seed=43, qk_scale=3.0)
    out, _ = _run("bf16", q, k, v, 1.0, causal, cuda, config=config)
    ref = attention_fp32(q, k, v, 1.0, causal)
    mx_tol, mean_tol = _tol("bf16")
    assert np.isfinite(out).all()
    assert error_stats(out, ref)[1] <= mean_tol
    assert (np.abs(out.astype(np.float64) - ref) <= mx_tol + half_ulp(ref, 7)).all()


@pytest.mark.parametrize("kind,d", WIDE)
def test_config_choice_equal(cuda, kind, d):
    """The two slot configurations give the same bits (per row they run the
    same arithmetic in the same order with fp32 row sums; only the
    work-group shape differs)."""
    q, k, v = _inputs(kind, 2, 4, 700, 700, d, seed=9)
    a, _ = _run(kind, q, k, v, 0.125, True, cuda, config=SLOT_W8_CFG)
    b, _ = _run(kind, q, k, v, 0.125, True, cuda, config=SLOT_W4_CFG)
    assert np.array_equal(a, b)


def test_binding_wide(cuda):
    import torch

    import flashlite_amd

    for kind, d in WIDE:
        q, k, v = _inputs(kind, 1, 4, 257, 300, d, seed=3)
        dt = torch.bfloat16 if kind == "bf16" else torch.float16
        tq, tk, tv = (torch.from_numpy(x).to(cuda).to(dt) for x in (q, k, v))
        for causal in (False, True):
            out, lse = flashlite_amd.forward_flash2_ex(tq, tk, tv, 0.0, causal, return_lse=True)
            assert out.dtype == dt and lse.dtype == torch.float32
            _check(kind, out.float().cpu().numpy(), attention_fp32(q, k, v, 0.0, causal),
                   f"binding {kind} D={d}")
            buf = torch.empty_like(tq)
            ret = flashlite_amd.forward_flash2_ex(tq, tk, tv, 0.0, causal, out=buf)
            assert ret.data_ptr() == buf.data_ptr()
        with pytest.raises(RuntimeError, match="split-KV"):
            flashlite_amd.forward_flash2_ex(tq, tk, tv, num_splits=2)
        with pytest.raises(RuntimeError, match="out tensor dtype must match q"):
            other = torch.float16 if kind == "bf16" else torch.bfloat16
            flashlite_amd.forward_flash2_ex(tq, tk, tv, out=torch.empty_like(tq, dtype=other))
    # the reference surface keeps the reference's checks
    q16 = torch.zeros((1, 2, 8, 128), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="requires head_dim == 64"):
        flashlite_amd.forward_flash2(q16, q16, q16)
    qb = torch.zeros((1, 2, 8, 64), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(RuntimeError, match="FP16"):
        flashlite_amd.forward_flash2(qb, qb, qb)
    q96 = torch.zeros((1, 2, 8, 96), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="head_dim 64 or 128"):
        flashlite_amd.forward_flash2_ex(q96, q96, q96)
