"""Seeded random shapes against the CPU oracle, through the C ABI: every tile
configuration that takes the key range, plus the dispatcher's choice, on the
same inputs.  A broad sweep beside the targeted tests: batch and head counts,
query and key lengths drawn independently (N_k != N_q both ways, so causal
rows with no visible key occur), both masks, and the scale sentinel (0.0),
negative, small and peaked (1.0) scales.  Inputs are N(0,1) in fp16, as the
reference's tests draw them (tests/test_correctness.py:38-41).

Bound: the north_star budget per element on top of the output's own
rounding, |out - ref| <= 2e-3 + half an ulp of |ref| in the output type
(bf16: 1.6e-2 + its half-ulp), mean-abs <= 2e-4 (1.6e-3).  At sm_scale 1/8
|O| stays below 1 and the allowance is a few 1e-4; at -0.3 or 1.0 the
softmax is peaked, |O| reaches 2-5, and the half-ulp alone is 1e-3 to 2e-3
of fp16.  The kernels that sum the unrounded p (the reference's row sums:
the pipelined, streaming, key-quarter and head_dim-128 ones) also carry up
to one rounding of the largest weight in the normalisation there, about
1e-3 beyond the allowance at |O| near 3 (the slot-scheduled kernels sum
the rounded p on the matrix core and land about 3x closer).  The second
test does the same for the wider types (fp16 at head_dim 128, bf16 at 64 and
128) through fl_attn_fwd_{f16,bf16}_ex, on contiguous or [B, N, H, D]
layouts, with the log-sum-exp; the third for split-KV decode (few query rows
over up to 20000 keys, automatic, single and forced chunk counts), the
fourth for the library's own decode plan over 64-512 heads; the fifth for
the naive kernel (forward_naive) at head dims 1-200."""

import numpy as np
import pytest

from flashlite_amd import capi
from gpu_util import (LSE_MAX_ABS, LSE_MEAN_ABS, assert_close_oracle, config_fits, run_capi,
                      run_splitkv, run_wide, to_dev, wide_inputs, wide_tol)
from oracle import attention_fp32, attention_lse, error_stats

NCFG = capi.num_configs()
SCALES = (0.0, 0.125, -0.3, 0.05, 1.0)


def _cases(n=40, seed=20261202):
    rs = np.random.RandomState(seed)
    out = []
    for i in range(n):
        b = int(rs.randint(1, 4))
        h = int(rs.randint(1, 5))
        lo, hi = ((1, 129), (129, 700), (700, 1300))[rs.randint(3)]
        nq = int(rs.randint(lo, hi))
        nk = nq if rs.rand() < 0.5 else int(rs.randint(1, 1300))
        causal = bool(rs.rand() < 0.5)
        scale = float(SCALES[rs.randint(len(SCALES))])
        out.append((i, b, h, nq, nk, causal, scale))
    return out


def _case_id(c):
    i, b, h, nq, nk, causal, scale = c
    return f"{i}-B{b}H{h}-q{nq}-k{nk}-{'causal' if causal else 'full'}-s{scale}"


@pytest.mark.gpu
@pytest.mark.parametrize("case", _cases(), ids=_case_id)
def test_random_shape_every_config(cuda, case):
    i, b, h, nq, nk, causal, scale = case
    rs = np.random.RandomState(1000 + i)
    q = rs.standard_normal((b, h, nq, 64)).astype(np.float32).astype(np.float16)
    k = rs.standard_normal((b, h, nk, 64)).astype(np.float32).astype(np.float16)
    v = rs.standard_normal((b, h, nk, 64)).astype(np.float32).astype(np.float16)
    ref = attention_fp32(q, k, v, scale, causal)
    for config in [-1] + list(range(NCFG)):
        if config >= 0 and not config_fits(config, nk):
            continue
        print(f"random shape {_case_id(case)} config={config}", flush=True)
        out = run_capi(q, k, v, scale, causal, cuda, config=config)
        assert_close_oracle(out, q, k, v, scale, causal, ref=ref, peaked=True)


# configurations built for each wider type (the others answer FL_ERR_BAD_CONFIG)
_SLOT = ("br256_bc64_w8_slot", "br128_bc64_w4_slot")
_BF16_D64 = _SLOT + ("br128_bc64_w4x2_slot", "br64_bc64_w2x2_slot", "br128_bc64_w4x2_pair",
                     "br64_bc64_w2x2_pair", "br256_kv256_w8_stream", "br32_kv512_w4_quarters")
WIDE_CONFIGS = {("fp16", 128): _SLOT, ("bf16", 128): _SLOT, ("bf16", 64): _BF16_D64}


def _wide_cases(n=24, seed=20261203):
    rs = np.random.RandomState(seed)
    kinds = sorted(WIDE_CONFIGS)
    out = []
    for i in range(n):
        kind, d = kinds[rs.randint(len(kinds))]
        b = int(rs.randint(1, 3))
        h = int(rs.randint(1, 4))
        nq = int(rs.randint(1, 1100))
        nk = nq if rs.rand() < 0.5 else int(rs.randint(1, 1100))
        causal = bool(rs.rand() < 0.5)
        scale = float(SCALES[rs.randint(len(SCALES))])
        strided = bool(rs.rand() < 0.5)
        out.append((i, kind, d, b, h, nq, nk, causal, scale, strided))
    return out


def _wide_id(c):
    i, kind, d, b, h, nq, nk, causal, scale, strided = c
    return (f"{i}-{kind}-D{d}-B{b}H{h}-q{nq}-k{nk}-{'causal' if causal else 'full'}-s{scale}"
            f"{'-bnhd' if strided else ''}")


def _bnhd(*ts):
    """The same values in [B, N, H, D] memory, passed as [B, H, N, D] views."""
    return tuple(t.transpose(1, 2).contiguous().transpose(1, 2) for t in ts)


@pytest.mark.gpu
@pytest.mark.parametrize("case", _wide_cases(), ids=_wide_id)
def test_random_shape_wide(cuda, case):
    i, kind, d, b, h, nq, nk, causal, scale, strided = case
    q = wide_inputs(kind, b, h, nq, nq, d, seed=3000 + i)[0]
    _, k, v = wide_inputs(kind, b, h, nk, nk, d, seed=4000 + i)
    ref = attention_fp32(q, k, v, scale, causal)
    peaked = abs(scale) >= 1.0
    ref_lse = None if peaked else attention_lse(q, k, scale, causal)
    max_abs, mean_abs = wide_tol(kind)
    names = [n for n in WIDE_CONFIGS[(kind, d)]
             if config_fits(capi.config_id(n), nk)]
    for config in [-1] + [capi.config_id(n) for n in names]:
        print(f"random wide {_wide_id(case)} config={config}", flush=True)
        out, lse = run_wide(kind, q, k, v, scale, causal, cuda, config=config, lse=not peaked,
                            views=_bnhd if strided else None)
        assert_close_oracle(out, q, k, v, scale, causal, ref=ref, max_abs=max_abs,
                            mean_abs=mean_abs, peaked=True,
                            mant_bits=7 if kind == "bf16" else 10)
        if ref_lse is not None:
            fin = np.isfinite(ref_lse)
            assert np.array_equal(fin, np.isfinite(lse)), "lse -inf pattern"
            if fin.any():
                mx, mean = error_stats(lse[fin], ref_lse[fin])
                assert mx <= LSE_MAX_ABS[kind] and mean <= LSE_MEAN_ABS[kind], (
                    f"lse max-abs {mx:.3e} mean-abs {mean:.3e}")


def _split_cases(n=24, seed=20261204):
    rs = np.random.RandomState(seed)
    out = []
    for i in range(n):
        b = int(rs.randint(1, 4))
        h = int(rs.randint(1, 5))
        lo, hi = ((1, 2), (2, 9), (9, 33), (33, 129))[rs.randint(4)]
        nq = int(rs.randint(lo, hi))
        nk = int(rs.randint(1, 20000))
        causal = bool(rs.rand() < 0.5)
        scale = float(SCALES[rs.randint(len(SCALES))])
        splits = int((0, 1, int(rs.randint(2, 300)))[rs.randint(3)])
        out.append((i, b, h, nq, nk, causal, scale, splits))
    return out


def _split_id(c):
    i, b, h, nq, nk, causal, scale, splits = c
    return f"{i}-B{b}H{h}-q{nq}-k{nk}-{'causal' if causal else 'full'}-s{scale}-x{splits}"


def _split_id_many(c):
    i, b, h, nq, nk, causal, scale = c
    return f"{i}-B{b}H{h}-q{nq}-k{nk}-{'causal' if causal else 'full'}-s{scale}"


def torch_cus(dev):
    import torch

    return torch.cuda.get_device_properties(dev).multi_processor_count


@pytest.mark.gpu
@pytest.mark.parametrize("case", _split_cases(), ids=_split_id)
def test_random_shape_splitkv(cuda, case):
    i, b, h, nq, nk, causal, scale, splits = case
    rs = np.random.RandomState(5000 + i)
    q = rs.standard_normal((b, h, nq, 64)).astype(np.float32).astype(np.float16)
    k = rs.standard_normal((b, h, nk, 64)).astype(np.float32).astype(np.float16)
    v = rs.standard_normal((b, h, nk, 64)).astype(np.float32).astype(np.float16)
    print(f"random split-KV {_split_id(case)}", flush=True)
    tq, tk, tv = (to_dev(x, cuda) for x in (q, k, v))
    peaked = abs(scale) >= 1.0
    o, ls, _ = run_splitkv(tq, tk, tv, scale, causal, splits)
    assert_close_oracle(o.float().cpu().numpy(), q, k, v, scale, causal, peaked=True)
    if not peaked:
        ref = attention_lse(q, k, scale, causal)
        lse = ls.cpu().numpy()
        assert np.array_equal(np.isneginf(lse), np.isneginf(ref)), "lse -inf pattern"
        fin = np.isfinite(ref)
        if fin.any():
            mx, mean = error_stats(lse[fin], ref[fin])
            assert mx <= LSE_MAX_ABS["fp16"] and mean <= LSE_MEAN_ABS["fp16"], (
                f"lse max-abs {mx:.3e} mean-abs {mean:.3e}")


def _many_head_cases(n=8, seed=20261209):
    rs = np.random.RandomState(seed)
    out = []
    for i in range(n):
        b = int(rs.choice([4, 8, 16]))
        h = int(rs.choice([16, 32]))
        nq = int(rs.choice([1, 4, 16, 32, 64]))
        nk = int(rs.randint(600, 4097))
        causal = bool(rs.rand() < 0.5)
        scale = float(SCALES[rs.randint(3)])
        out.append((i, b, h, nq, nk, causal, scale))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("case", _many_head_cases(), ids=_split_id_many)
def test_random_shape_splitkv_many_heads(cuda, case):
    """The library's own plan over 64-512 heads: one pass from half as many
    query-row groups as CUs (the 4-wave groups for at most 32 rows over at
    least as many heads as CUs), key chunks below."""
    i, b, h, nq, nk, causal, scale = case
    rs = np.random.RandomState(7000 + i)
    q = rs.standard_normal((b, h, nq, 64)).astype(np.float32).astype(np.float16)
    k = rs.standard_normal((b, h, nk, 64)).astype(np.float32).astype(np.float16)
    v = rs.standard_normal((b, h, nk, 64)).astype(np.float32).astype(np.float16)
    print(f"random split-KV many heads {_split_id_many(case)}", flush=True)
    tq, tk, tv = (to_dev(x, cuda) for x in (q, k, v))
    o, ls, need = run_splitkv(tq, tk, tv, scale, causal, 0)
    waves = 1 if nq <= 32 else (2 if nq <= 64 else 4)
    groups = b * h * -(-nq // (32 * waves))
    if 2 * groups >= torch_cus(cuda):
        assert need == 0, "one pass expected"
    assert_close_oracle(o.float().cpu().numpy(), q, k, v, scale, causal, peaked=True)
    ref = attention_lse(q, k, scale, causal)
    fin = np.isfinite(ref)
    mx, mean = error_stats(ls.cpu().numpy()[fin], ref[fin])
    assert mx <= LSE_MAX_ABS["fp16"] and mean <= LSE_MEAN_ABS["fp16"], (
        f"lse max-abs {mx:.3e} mean-abs {mean:.3e}")


def _naive_cases(n=16, seed=20261205):
    rs = np.random.RandomState(seed)
    out = []
    for i in range(n):
        b = int(rs.randint(1, 3))
        h = int(rs.randint(1, 4))
        d = int(rs.randint(1, 201))
        nq = int(rs.randint(1, 1500))
        nk = nq if rs.rand() < 0.5 else int(rs.randint(1, 1500))
        causal = bool(rs.rand() < 0.5)
        scale = float(SCALES[rs.randint(len(SCALES))])
        out.append((i, b, h, d, nq, nk, causal, scale))
    return out


def _naive_id(c):
    i, b, h, d, nq, nk, causal, scale = c
    return f"{i}-B{b}H{h}-D{d}-q{nq}-k{nk}-{'causal' if causal else 'full'}-s{scale}"


@pytest.mark.gpu
@pytest.mark.parametrize("case", _naive_cases(), ids=_naive_id)
def test_random_shape_naive(cuda, case):
    i, b, h, d, nq, nk, causal, scale = case
    rs = np.random.RandomState(6000 + i)
    q = rs.standard_normal((b, h, nq, d)).astype(np.float32).astype(np.float16)
    k = rs.standard_normal((b, h, nk, d)).astype(np.float32).astype(np.float16)
    v = rs.standard_normal((b, h, nk, d)).astype(np.float32).astype(np.float16)
    print(f"random naive {_naive_id(case)}", flush=True)
    out = run_capi(q, k, v, scale, causal, cuda, naive=True)
    assert_close_oracle(out, q, k, v, scale, causal, peaked=True)
