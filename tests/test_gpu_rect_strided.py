"""GPU parity of the path beyond the reference's shapes: N_k != N_q with the
causal diagonal aligned bottom-right, strided [B, H, N, D] views (the
[B, N, H, D] layout of the flash_attn package, padded rows), and the
log-sum-exp output.

Output tolerance as everywhere (north_star): max-abs <= 2e-3, mean-abs <=
2e-4 against the fp32 oracle.  The log-sum-exp is compared with the fp64
oracle at max-abs <= 2e-3 and mean-abs <= 3e-4 (natural-log units): l sums
the fp16-rounded p (2^-12 relative each), which moves ln l by up to ~1e-3 on
rows that see few keys.  A strided launch must equal the contiguous launch
of the same data bit for bit: the kernels read the same values in the same
order.
"""

import numpy as np
import pytest

from flashlite_amd import capi
from gpu_util import assert_close_oracle, config_fits, to_dev
from oracle import attention_fp32, attention_lse, error_stats

pytestmark = pytest.mark.gpu

NCFG = capi.num_configs()
LSE_MAX_ABS = 2e-3
LSE_MEAN_ABS = 3e-4


def _qkv(b, h, nq, nk, seed, qk_scale=1.0):
    """Seeded fp16 inputs; qk_scale multiplies Q and K only (V stays N(0, 1)
    so the fp16 output keeps the absolute tolerance meaningful)."""
    rs = np.random.RandomState(seed)
    mk = lambda n, c: (rs.standard_normal((b, h, n, 64)) * c).astype(np.float32).astype(np.float16)
    return mk(nq, qk_scale), mk(nk, qk_scale), mk(nk, 1.0)


def _run(q16, k16, v16, sm_scale, causal, dev, config=-1, lse=False):
    import torch

    tq, tk, tv = (to_dev(x, dev) for x in (q16, k16, v16))
    o = torch.full_like(tq, float("nan"))
    ls = torch.full(tq.shape[:3], float("nan"), dtype=torch.float32, device=dev) if lse else None
    p = capi.tensor_params_ex(tq, tk, tv, o, sm_scale, causal, lse=ls)
    capi.check(capi.fwd_ex(p, torch.cuda.current_stream(dev).cuda_stream, config))
    torch.cuda.synchronize(dev)
    return o.cpu().numpy(), (ls.cpu().numpy() if lse else None)


RECT = [(1, 1), (1, 300), (5, 64), (37, 100), (100, 37), (64, 65), (200, 513), (513, 200),
        (129, 1000), (1000, 129)]


@pytest.mark.parametrize("config", list(range(NCFG)))
@pytest.mark.parametrize("nq,nk", RECT)
@pytest.mark.parametrize("causal", [False, True])
def test_rectangular_each_config(cuda, config, nq, nk, causal):
    q, k, v = _qkv(1, 2, nq, nk, seed=nq * 7 + nk)
    if not config_fits(config, nk):
        with pytest.raises(RuntimeError, match="needs N_k <= "):
            _run(q, k, v, 0.125, causal, cuda, config=config, lse=True)
        return
    out, lse = _run(q, k, v, 0.125, causal, cuda, config=config, lse=True)
    ref = attention_fp32(q, k, v, 0.125, causal)
    if causal and nq > nk:
        # rows with no visible key are written as exactly 0
        assert np.all(out[:, :, :nq - nk] == 0.0)
    assert_close_oracle(out, q, k, v, 0.125, causal, ref=ref)
    ref_lse = attention_lse(q, k, 0.125, causal)
    assert np.array_equal(np.isneginf(lse), np.isneginf(ref_lse))
    fin = np.isfinite(ref_lse)
    mx, mean = error_stats(lse[fin], ref_lse[fin])
    assert mx <= LSE_MAX_ABS and mean <= LSE_MEAN_ABS, f"lse max-abs {mx:.3e} mean-abs {mean:.3e}"


@pytest.mark.parametrize("causal", [False, True])
def test_no_keys(cuda, causal):
    # N_k = 0: every row has no visible key -> O = 0, lse = -inf
    q, k, v = _qkv(1, 2, 70, 0, seed=3)
    out, lse = _run(q, k, v, 0.125, causal, cuda, lse=True)
    assert np.all(out == 0.0) and np.all(np.isneginf(lse))


@pytest.mark.parametrize("nq,nk", [(1, 4096), (16, 4096), (4096, 1024), (2048, 4096)])
@pytest.mark.parametrize("causal", [False, True])
def test_rectangular_dispatcher_larger(cuda, nq, nk, causal):
    q, k, v = _qkv(2, 4, nq, nk, seed=nq + nk)
    out, lse = _run(q, k, v, 0.125, causal, cuda, lse=True)
    rows = np.unique(np.concatenate([np.arange(min(nq, 48)), np.arange(max(0, nq - 48), nq),
                                     np.random.RandomState(1).randint(0, nq, 64)]))
    ref = attention_fp32(q, k, v, 0.125, causal, rows=rows)
    assert_close_oracle(out, q, k, v, 0.125, causal, rows=rows, ref=ref)
    ref_lse = attention_lse(q[:, :, rows], k, 0.125, False) if not causal else None
    if ref_lse is not None:
        mx, mean = error_stats(lse[:, :, rows], ref_lse)
        assert mx <= LSE_MAX_ABS and mean <= LSE_MEAN_ABS


def test_binding_rectangular(cuda):
    import torch

    import flashlite_amd as fl

    q16, k16, v16 = _qkv(2, 3, 77, 300, seed=9)
    q, k, v = (to_dev(x, cuda) for x in (q16, k16, v16))
    for causal in (False, True):
        out = fl.forward_flash2(q, k, v, 0.125, causal)
        torch.cuda.synchronize()
        assert_close_oracle(out.float().cpu().numpy(), q16, k16, v16, 0.125, causal)
        nv = fl.forward_naive(q, k, v, 0.125, causal)
        torch.cuda.synchronize()
        assert_close_oracle(nv.float().cpu().numpy(), q16, k16, v16, 0.125, causal)
    # more queries than keys, causal: the naive kernel also writes 0 rows
    q16, k16, v16 = _qkv(1, 2, 50, 20, seed=10)
    q, k, v = (to_dev(x, cuda) for x in (q16, k16, v16))
    nv = fl.forward_naive(q, k, v, 0.125, True).float().cpu().numpy()
    assert np.all(nv[:, :, :30] == 0.0)
    assert_close_oracle(nv, q16, k16, v16, 0.125, True)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("nq,nk", [(333, 333), (200, 700)])
def test_strided_layouts_bit_exact(cuda, causal, nq, nk):
    """[B, N, H, D] storage (passed as transposed views), padded rows and an
    [B, N, H, D] output view give exactly the contiguous result."""
    import torch

    import flashlite_amd as fl

    b, h = 2, 3
    q16, k16, v16 = _qkv(b, h, nq, nk, seed=11)
    q, k, v = (to_dev(x, cuda) for x in (q16, k16, v16))
    ref, ref_lse = fl.forward_flash2_ex(q, k, v, 0.125, causal, return_lse=True)
    torch.cuda.synchronize()
    assert_close_oracle(ref.float().cpu().numpy(), q16, k16, v16, 0.125, causal)

    # [B, N, H, D] storage
    qb, kb, vb = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (q, k, v))
    assert qb.stride() == (nq * h * 64, 64, h * 64, 1)
    out_bnhd = torch.full((b, nq, h, 64), float("nan"), dtype=torch.float16, device=cuda)
    got, got_lse = fl.forward_flash2_ex(qb, kb, vb, 0.125, causal, out=out_bnhd.transpose(1, 2),
                                        return_lse=True)
    torch.cuda.synchronize()
    assert got.data_ptr() == out_bnhd.data_ptr()
    assert torch.equal(got, ref) and torch.equal(got_lse, ref_lse)
    # omitted out: allocated with q's (BNHD) layout
    got2 = fl.forward_flash2_ex(qb, kb, vb, 0.125, causal)
    assert got2.stride() == qb.stride() and torch.equal(got2, ref)

    # padded rows: row stride 128 (a [.., 128] buffer sliced to 64), head stride with a gap
    def padded(x):
        buf = torch.full((b, h, x.shape[2] + 3, 128), float("nan"), dtype=torch.float16,
                         device=cuda)
        buf[:, :, : x.shape[2], :64] = x
        return buf[:, :, : x.shape[2], :64]

    qp, kp, vp = padded(q), padded(k), padded(v)
    assert qp.stride(2) == 128 and qp.stride(1) == (nq + 3) * 128
    got3 = fl.forward_flash2_ex(qp, kp, vp, 0.125, causal)
    torch.cuda.synchronize()
    assert torch.equal(got3, ref)


def test_strided_each_config_bit_exact(cuda):
    import torch

    q16, k16, v16 = _qkv(1, 4, 300, 300, seed=12)
    q, k, v = (to_dev(x, cuda) for x in (q16, k16, v16))
    qb, kb, vb = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (q, k, v))
    stream = torch.cuda.current_stream(cuda).cuda_stream
    for config in range(NCFG):
        if not config_fits(config, 300):
            continue
        for causal in (False, True):
            o1 = torch.empty_like(q)
            capi.check(capi.fwd(capi.tensor_params(q, k, v, o1, 0.125, causal), stream, config))
            o2 = torch.empty_like(qb)
            capi.check(capi.fwd_ex(capi.tensor_params_ex(qb, kb, vb, o2, 0.125, causal), stream,
                                   config))
            torch.cuda.synchronize()
            assert torch.equal(o1, o2), (config, causal)


@pytest.mark.parametrize("scale,sm", [(1.0, 0.125), (3.0, 1.0), (1.0, -0.3)])
def test_lse_scales(cuda, scale, sm):
    """Peaked softmax (the kernel's checked pass) and a negative scale.  As
    in the other peaked-scale tests, the output bound adds, per element, the
    output's own fp16 half-ulp once |O| nears a single V row; the lse bound
    adds 2^-11 of |lse| (its scores come from fp16 operands)."""
    q, k, v = _qkv(1, 2, 500, 500, seed=13, qk_scale=scale)
    peaked = abs(sm) * scale * scale > 0.2
    for causal in (False, True):
        out, lse = _run(q, k, v, sm, causal, cuda, lse=True)
        assert_close_oracle(out, q, k, v, sm, causal, peaked=peaked)
        ref_lse = attention_lse(q, k, sm, causal)
        mx, mean = error_stats(lse, ref_lse)
        mag = np.abs(ref_lse)
        assert mx <= LSE_MAX_ABS + 2.0 ** -11 * mag.max(), f"lse max-abs {mx:.3e}"
        assert mean <= LSE_MEAN_ABS + 2.0 ** -11 * mag.mean(), f"lse mean-abs {mean:.3e}"


def test_binding_lse_out(cuda):
    """forward_flash2_ex(..., return_lse=True, lse=buf) writes the log-sum-exp
    into `buf` (no allocation) with the same values as an allocated one, and
    rejects a wrong dtype, shape, layout or a missing return_lse."""
    import torch

    import flashlite_amd as fl

    q16, k16, v16 = _qkv(2, 3, 200, 333, seed=14)
    q, k, v = (to_dev(x, cuda) for x in (q16, k16, v16))
    for causal in (False, True):
        ref_o, ref_l = fl.forward_flash2_ex(q, k, v, 0.125, causal, return_lse=True)
        out = torch.empty_like(q)
        buf = torch.full((2, 3, 200), float("nan"), dtype=torch.float32, device=cuda)
        got_o, got_l = fl.forward_flash2_ex(q, k, v, 0.125, causal, out=out, return_lse=True,
                                            lse=buf)
        torch.cuda.synchronize()
        assert got_l.data_ptr() == buf.data_ptr() and got_o.data_ptr() == out.data_ptr()
        assert torch.equal(got_l, ref_l) and torch.equal(got_o, ref_o)
    bad = [(torch.empty((2, 3, 200), dtype=torch.float16, device=cuda), "float32"),
           (torch.empty((2, 3, 199), dtype=torch.float32, device=cuda), r"\[B, H, N_q\]"),
           (torch.empty((2, 200, 3), dtype=torch.float32, device=cuda).transpose(1, 2),
            r"\[B, H, N_q\]")]
    for t, msg in bad:
        with pytest.raises(RuntimeError, match=msg):
            fl.forward_flash2_ex(q, k, v, return_lse=True, lse=t)
    with pytest.raises(RuntimeError, match="return_lse"):
        fl.forward_flash2_ex(q, k, v, lse=torch.empty((2, 3, 200), device=cuda))
