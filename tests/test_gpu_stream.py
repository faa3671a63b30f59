"""GPU parity of the streaming configuration (br256_kv256_w8_stream): one
persistent work-group per CU walks units of up to 256 query rows whose keys
(N_k <= 256) fit one LDS buffer, with the next unit's loads in flight while
the current one computes.  The cases cover more units than work-groups (so
buffers and Q registers are reused, with odd and even unit counts), several
units per head (N_q > 256), N_k != N_q with the bottom-right causal
diagonal, the log-sum-exp output, strided views, peaked and negative scales
(the stabiliser's checked path) and the C4 workload.

Tolerance (north_star): max-abs <= 2e-3, mean-abs <= 2e-4 of the fp16
output against the fp32 oracle; log-sum-exp max-abs <= 2e-3 and mean-abs
<= 3e-4 (natural-log units), as for the other configurations.  Outputs
start as NaN, so a row the kernel fails to write fails the check.
"""

import numpy as np
import pytest

from flashlite_amd import capi
from flashlite_amd.workloads import WORKLOADS, make_qkv, workload_inputs
from gpu_util import SLOT_W4_CFG, STREAM_CFG, assert_close_oracle, run_capi, sample_rows, to_dev
from oracle import attention_fp32, attention_lse, error_stats

pytestmark = pytest.mark.gpu

LSE_MAX_ABS = 2e-3
LSE_MEAN_ABS = 3e-4


def _run_ex(q16, k16, v16, sm_scale, causal, dev, views=None):
    import torch

    tq, tk, tv = (to_dev(x, dev) for x in (q16, k16, v16))
    o = torch.full_like(tq, float("nan"))
    ls = torch.full(tq.shape[:3], float("nan"), dtype=torch.float32, device=dev)
    if views is not None:
        tq, tk, tv, o = views(tq, tk, tv, o)
    p = capi.tensor_params_ex(tq, tk, tv, o, sm_scale, causal, lse=ls)
    capi.check(capi.fwd_ex(p, torch.cuda.current_stream(dev).cuda_stream, STREAM_CFG))
    torch.cuda.synchronize(dev)
    return o.cpu().numpy(), ls.cpu().numpy()


# (batch, heads, N_q, N_k): units = B*H*ceil(N_q/256) against 256 work-groups
SHAPES = [
    (1, 1, 1, 1),          # one unit, one row, one key
    (1, 1, 256, 256),      # one full unit
    (2, 3, 100, 100),      # 6 units, ragged
    (8, 40, 64, 64),       # 320 units: two rounds on some work-groups
    (16, 32, 130, 130),    # 512 units: exactly two rounds
    (9, 61, 33, 200),      # 549 units (odd rounds), N_k > N_q
    (3, 5, 700, 256),      # 3 units per head (N_q > 256)
    (2, 2, 513, 129),      # N_q > N_k, rows with no visible key when causal
    (64, 48, 96, 160),     # 3072 units: 12 per work-group, both buffers reused many times
]


# The kernel's instances and modes by shape: the next unit's K/V fetches
# spread over the tile steps (at least 4 units per work-group, N_k > 192),
# or all issued first; causal waves 0-3 fetching for waves 4-7 (N_q > 224).
# Sampled rows keep the CPU oracle short at 512-1024 heads.
MODES = [
    (32, 32, 250, 250),    # 1024 units: spread, and causal sharing
    (32, 32, 200, 200),    # 1024 units: spread, no sharing
    (8, 64, 256, 256),     # 512 units: all first, causal sharing
    (16, 32, 225, 225),    # 512 units: sharing from N_q 225 on
]


@pytest.mark.parametrize("b,h,nq,nk", MODES)
@pytest.mark.parametrize("causal", [False, True])
def test_fetch_modes(cuda, b, h, nq, nk, causal):
    rs = np.random.RandomState(b * 100 + h + nq)
    mk = lambda n: rs.standard_normal((b, h, n, 64)).astype(np.float32).astype(np.float16)  # noqa: E731
    q, k, v = mk(nq), mk(nk), mk(nk)
    out, _ = _run_ex(q, k, v, 0.125, causal, cuda)
    assert np.isfinite(out).all(), "unwritten outputs"
    rows = sample_rows(nq, count=48, seed=nq)
    assert_close_oracle(out, q, k, v, 0.125, causal, rows=rows)


@pytest.mark.parametrize("b,h,nq,nk", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_shapes_with_lse(cuda, b, h, nq, nk, causal):
    rs = np.random.RandomState(b * 1000 + h * 10 + nq + nk)
    mk = lambda n: rs.standard_normal((b, h, n, 64)).astype(np.float32).astype(np.float16)  # noqa: E731
    q, k, v = mk(nq), mk(nk), mk(nk)
    out, lse = _run_ex(q, k, v, 0.125, causal, cuda)
    ref = attention_fp32(q, k, v, 0.125, causal)
    if causal and nq > nk:
        assert np.all(out[:, :, :nq - nk] == 0.0)
    assert_close_oracle(out, q, k, v, 0.125, causal, ref=ref)
    ref_lse = attention_lse(q, k, 0.125, causal)
    assert np.array_equal(np.isneginf(lse), np.isneginf(ref_lse))
    fin = np.isfinite(ref_lse)
    mx, mean = error_stats(lse[fin], ref_lse[fin])
    assert mx <= LSE_MAX_ABS and mean <= LSE_MEAN_ABS, f"lse max-abs {mx:.3e} mean-abs {mean:.3e}"


@pytest.mark.parametrize("causal", [False, True])
def test_c4_matches_oracle_and_slot_kernel(cuda, causal):
    w = WORKLOADS["C4_many_B32H32N256"]
    q, k, v = workload_inputs(w)
    out = run_capi(q, k, v, w.sm_scale, causal, cuda, config=STREAM_CFG)
    assert_close_oracle(out, q, k, v, w.sm_scale, causal)
    # causal row 0 sees only key 0: the output is V[0] exactly
    if causal:
        assert np.array_equal(out[:, :, 0], v[:, :, 0])
    slot = run_capi(q, k, v, w.sm_scale, causal, cuda, config=SLOT_W4_CFG)
    assert error_stats(out, slot)[0] <= 2e-3


@pytest.mark.parametrize("scale", [-0.2, 0.05, 1.0, 3.0])
def test_other_scales(cuda, scale):
    # The scales of the other configurations' test: std-8 and std-24 logits
    # move the row max above the first tile's, so the checked softmax
    # rescales; the negative scale flips the sign of Q.  Bound: 2e-3, plus
    # (peaked cases, per element) the output's own fp16 half-ulp.
    q, k, v = make_qkv(4, 8, 256, 64, seed=97)
    for causal in (False, True):
        out = run_capi(q, k, v, scale, causal, cuda, config=STREAM_CFG)
        assert_close_oracle(out, q, k, v, scale, causal, peaked=scale >= 1)


def test_strided_bit_exact(cuda):
    """[B, N, H, D] views and padded rows give the contiguous launch's bits."""
    import torch

    q, k, v = make_qkv(3, 7, 200, 64, seed=5)
    for causal in (False, True):
        base, _ = _run_ex(q, k, v, 0.125, causal, cuda)

        def bnhd(tq, tk, tv, o):
            f = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)  # noqa: E731
            return f(tq), f(tk), f(tv), f(o)

        def padded(tq, tk, tv, o):
            def pad(t):
                b, h, n, d = t.shape
                big = torch.zeros((b, h, n, d + 64), dtype=t.dtype, device=t.device)
                big[..., :d] = t
                return big[..., :d]
            return pad(tq), pad(tk), pad(tv), pad(o)

        for views in (bnhd, padded):
            out, _ = _run_ex(q, k, v, 0.125, causal, cuda, views=views)
            assert np.array_equal(out, base), (views.__name__, causal)


def test_no_writes_outside_output(cuda):
    import torch

    b, h, n = 5, 9, 77
    q, k, v = make_qkv(b, h, n, 64, seed=61)
    tq, tk, tv = (to_dev(x, cuda) for x in (q, k, v))
    guard = 4096
    numel = b * h * n * 64
    buf = torch.full((guard + numel + guard,), 7.0, dtype=torch.float16, device=cuda)
    o = buf[guard:guard + numel].view(b, h, n, 64)
    p = capi.tensor_params(tq, tk, tv, o, 0.125, True)
    capi.check(capi.fwd(p, torch.cuda.current_stream().cuda_stream, STREAM_CFG))
    torch.cuda.synchronize()
    host = buf.cpu().numpy()
    assert (host[:guard] == 7.0).all() and (host[guard + numel:] == 7.0).all()
    assert_close_oracle(o.cpu().numpy(), q, k, v, 0.125, True)


def test_deterministic_and_repeatable(cuda):
    # back-to-back launches into one reused buffer (the C4 pattern)
    import torch

    q, k, v = make_qkv(8, 64, 256, 64, seed=7)
    tq, tk, tv = (to_dev(x, cuda) for x in (q, k, v))
    o = torch.empty_like(tq)
    stream = torch.cuda.current_stream().cuda_stream
    p = capi.tensor_params(tq, tk, tv, o, 0.125, True)
    capi.check(capi.fwd(p, stream, STREAM_CFG))
    torch.cuda.synchronize()
    first = o.cpu().numpy()
    for _ in range(5):
        capi.check(capi.fwd(p, stream, STREAM_CFG))
    torch.cuda.synchronize()
    assert np.array_equal(o.cpu().numpy(), first)
