"""GPU parity of the balanced causal launch (``fl_attn_fwd_f16_ws``): causal
attention with N_q = N_k, where the longer half of the 128-row query blocks
have their key ranges split between two work-groups that merge through the
caller's workspace.

Tolerances as for every fp16 path against the fp32 oracle (north_star):
max-abs <= 2e-3 and mean-abs <= 2e-4 on every output row; the log-sum-exp
within 2e-3 / 3e-4 (natural-log units, as in test_gpu_rect_strided.py); on
peaked scales the max-abs bound holds per element on top of the output's own
half-ulp.  The merge is symmetric in the two halves, so results do not depend
on which half finishes first: repeated calls give the same bits.  Every call
must leave the workspace's semaphore words at zero.
"""

import numpy as np
import pytest

from flashlite_amd import capi
from gpu_util import assert_close_oracle, sample_rows, to_dev
from oracle import attention_fp32, attention_lse, error_stats

pytestmark = pytest.mark.gpu

LSE_MAX_ABS = 2e-3
LSE_MEAN_ABS = 3e-4


def _qkv(b, h, n, seed, qk_scale=1.0):
    rs = np.random.RandomState(seed)
    mk = lambda c: (rs.standard_normal((b, h, n, 64)) * c).astype(np.float32).astype(np.float16)  # noqa: E731
    return mk(qk_scale), mk(qk_scale), mk(1.0)


def _sem_words(b, h, n):
    return (b * h * (n // 256) * 8 + 255) // 256 * 64  # float32 words of the semaphore region


def _run_ws(tq, tk, tv, sm_scale, ws=None, lse=True):
    import torch

    dev = tq.device
    o = torch.full_like(tq, float("nan"))
    ls = torch.full(tq.shape[:3], float("nan"), dtype=torch.float32, device=dev) if lse else None
    p = capi.tensor_params_ex(tq, tk, tv, o, sm_scale, True, lse=ls)
    need = capi.fwd_workspace_bytes(p)
    assert need > 0, "the balanced launch should apply"
    if ws is None:
        ws = torch.zeros(need // 4, dtype=torch.float32, device=dev)
    capi.check(capi.fwd_ws(p, ws.data_ptr(), ws.numel() * 4,
                           torch.cuda.current_stream(dev).cuda_stream))
    torch.cuda.synchronize(dev)
    return o, ls, ws


SHAPES = [(1, 8, 1024), (2, 8, 2048), (2, 8, 4096), (1, 16, 4096)]


@pytest.mark.parametrize("b,h,n", SHAPES)
def test_balanced_matches_oracle(cuda, b, h, n):
    print(f"balanced B{b} H{h} N{n}", flush=True)
    q16, k16, v16 = _qkv(b, h, n, seed=n + h)
    tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
    o, ls, ws = _run_ws(tq, tk, tv, 0.125)
    assert bool((ws[: _sem_words(b, h, n)] == 0).all()), "semaphores not left at zero"
    assert_close_oracle(o.float().cpu().numpy(), q16, k16, v16, 0.125, True,
                        ref=attention_fp32(q16, k16, v16, 0.125, True))
    lse, ref = ls.cpu().numpy(), attention_lse(q16, k16, 0.125, True)
    mx, mean = error_stats(lse, ref)
    assert mx <= LSE_MAX_ABS and mean <= LSE_MEAN_ABS, f"lse max-abs {mx:.3e} mean-abs {mean:.3e}"


def test_balanced_long(cuda):
    """C3's shape (B1 H16 N16384), sampled rows."""
    q16, k16, v16 = _qkv(1, 16, 16384, seed=3, qk_scale=0.5)
    tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
    o, _, ws = _run_ws(tq, tk, tv, 0.125, lse=False)
    assert bool((ws[: _sem_words(1, 16, 16384)] == 0).all())
    rows = sample_rows(16384, count=192, seed=4)
    out = o.float().cpu().numpy()
    assert_close_oracle(out, q16, k16, v16, 0.125, True, rows=rows)
    assert np.array_equal(out[:, :, 0], v16[:, :, 0].astype(np.float32))


def test_balanced_repeat_same_bits_and_matches_binding(cuda):
    """Calls in a row reuse the workspace as left; the halves may finish in
    either order and give the same bits; forward_flash2 runs this launch."""
    import torch

    import flashlite_amd

    q16, k16, v16 = _qkv(2, 8, 4096, seed=21)
    tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
    o1, l1, ws = _run_ws(tq, tk, tv, 0.125)
    for _ in range(3):
        o2, l2, ws = _run_ws(tq, tk, tv, 0.125, ws=ws)
        assert torch.equal(o1, o2) and torch.equal(l1, l2)
    out = flashlite_amd.forward_flash2(tq, tk, tv, 0.125, True)
    torch.cuda.synchronize()
    assert torch.equal(out, o1)
    out_ex, lse_ex = flashlite_amd.forward_flash2_ex(tq, tk, tv, 0.125, True, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out_ex, o1) and torch.equal(lse_ex, l1)


@pytest.mark.parametrize("scale,sm", [(3.0, 1.0), (1.0, -0.3)])
def test_balanced_peaked_and_negative(cuda, scale, sm):
    """Peaked scores send halves to the checked pass (each half on its own);
    a negative scale flips Q."""
    from gpu_util import redo_expected

    q16, k16, v16 = _qkv(1, 8, 1024, seed=31, qk_scale=scale)
    if sm > 0:
        assert redo_expected(q16, k16, sm, True)
    tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
    o, ls, ws = _run_ws(tq, tk, tv, sm)
    assert bool((ws[: _sem_words(1, 8, 1024)] == 0).all())
    assert_close_oracle(o.float().cpu().numpy(), q16, k16, v16, sm, True,
                        ref=attention_fp32(q16, k16, v16, sm, True), peaked=abs(sm) * scale >= 1)
    ref = attention_lse(q16, k16, sm, True)
    mx, _ = error_stats(ls.cpu().numpy(), ref)
    assert mx <= LSE_MAX_ABS + 2.0 ** -11 * np.abs(ref).max(), f"lse max-abs {mx:.3e}"


def test_balanced_strided_bit_exact(cuda):
    """[B, N, H, D] storage passed as transposed views gives the contiguous bits."""
    import torch

    q16, k16, v16 = _qkv(2, 8, 2048, seed=41)
    tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
    o, ls, ws = _run_ws(tq, tk, tv, 0.125)
    qb, kb, vb = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (tq, tk, tv))
    o2, l2, _ = _run_ws(qb, kb, vb, 0.125, ws=ws)
    assert torch.equal(o2, o) and torch.equal(l2, ls)


def test_not_applicable_runs_one_pass(cuda):
    """Non-causal, or N_q != N_k: no workspace; fl_attn_fwd_f16_ws runs the
    dispatcher's one-pass kernel (same bits as fl_attn_fwd_f16_ex)."""
    import torch

    q16, k16, v16 = _qkv(1, 8, 1024, seed=51)
    tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
    stream = torch.cuda.current_stream(cuda).cuda_stream
    for causal, kv in ((False, (tk, tv)), (True, (tk[:, :, :1000], tv[:, :, :1000]))):
        o1, o2 = torch.empty_like(tq), torch.empty_like(tq)
        p1 = capi.tensor_params_ex(tq, kv[0], kv[1], o1, 0.125, causal)
        assert capi.fwd_workspace_bytes(p1) == 0
        capi.check(capi.fwd_ws(p1, 0, 0, stream))
        capi.check(capi.fwd_ex(capi.tensor_params_ex(tq, kv[0], kv[1], o2, 0.125, causal), stream,
                               -1))
        torch.cuda.synchronize()
        assert torch.equal(o1, o2), causal
