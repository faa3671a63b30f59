"""Pins the CPU oracle (runs without a GPU).

Each check is chosen so that a plausible slip in the oracle -- a transposed
operand, a mask in the wrong direction, a missing or doubled scale, softmax
over the wrong axis, a dropped max subtraction -- fails at least one of them.
"""

import json
import math
import os

import numpy as np
import pytest

from flashlite_amd.workloads import WORKLOADS, digest, make_qkv, workload_inputs
from oracle import (attention_bruteforce, attention_bytes, attention_flops, attention_fp32,
                    attention_fp64, attention_lse, causal_visible, error_stats, resolve_sm_scale,
                    sm_scale_log2)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _qkv(b, h, n, d, seed, scale=1.0):
    return make_qkv(b, h, n, d, seed, scale)


# --- brute force (independent scalar loops) --------------------------------

@pytest.mark.parametrize("n", [1, 2, 3, 17])
@pytest.mark.parametrize("causal", [False, True])
def test_fp32_matches_bruteforce(n, causal):
    q, k, v = _qkv(1, 2, n, 8, seed=10 + n)
    ref = attention_bruteforce(q, k, v, 0.37, causal)
    mx, mean = error_stats(attention_fp32(q, k, v, 0.37, causal), ref)
    assert mx < 2e-6 and mean < 5e-7
    mx64, _ = error_stats(attention_fp64(q, k, v, 0.37, causal), ref)
    assert mx64 < 1e-12


def test_bruteforce_is_not_symmetric_in_q_and_k():
    # Guards the transposed-operand slip: swapping q and k changes the result.
    q, k, v = _qkv(1, 1, 5, 4, seed=3)
    a = attention_bruteforce(q, k, v, 0.5, False)
    b = attention_bruteforce(k, q, v, 0.5, False)
    assert error_stats(a, b)[0] > 1e-2


# --- golden fixture ---------------------------------------------------------

def test_c0_golden_fixture():
    z = np.load(os.path.join(GOLDEN, "c0_golden.npz"))
    w = WORKLOADS["C0_plumbing_B1H1N128"]
    q, k, v = workload_inputs(w)
    assert np.array_equal(z["q"], q) and np.array_equal(z["k"], k) and np.array_equal(z["v"], v)
    for causal, key in ((False, "out_noncausal"), (True, "out_causal")):
        mx, mean = error_stats(attention_fp32(q, k, v, w.sm_scale, causal), z[key])
        assert mx < 1e-5 and mean < 1e-6, (causal, mx, mean)


def test_input_hashes_frozen():
    with open(os.path.join(GOLDEN, "input_hashes.json")) as f:
        hashes = json.load(f)
    assert set(hashes) == set(WORKLOADS)
    for name, w in WORKLOADS.items():
        if w.batch * w.heads * w.seq > (1 << 20):
            continue  # the large configs are hashed on the GPU box
        assert digest(*workload_inputs(w)) == hashes[name]["sha256"], name


def test_generator_casts_through_fp32():
    rs = np.random.RandomState(7)
    x = rs.standard_normal(size=(1, 1, 4, 8))
    q, _, _ = make_qkv(1, 1, 4, 8, seed=7)
    assert np.array_equal(q, x.astype(np.float32).astype(np.float16))


# --- torch CPU SDPA (the reference tests' own comparator) -------------------

@pytest.mark.parametrize("causal", [False, True])
def test_matches_torch_sdpa_cpu(causal):
    from oracle.cpu_sdpa import sdpa_cpu_f32, to_cpu_f32

    q, k, v = _qkv(2, 3, 97, 64, seed=21)
    tq, tk, tv = to_cpu_f32(q, k, v)
    ref = sdpa_cpu_f32(tq, tk, tv, 0.0, causal).numpy()
    mx, mean = error_stats(attention_fp32(q, k, v, 0.0, causal), ref)
    assert mx < 1e-5 and mean < 1e-6


# --- closed forms and invariants --------------------------------------------

def test_causal_row0_is_v0():
    q, k, v = _qkv(2, 2, 33, 16, seed=4)
    out = attention_fp32(q, k, v, 0.125, True)
    assert np.allclose(out[:, :, 0, :], v[:, :, 0, :].astype(np.float32), atol=0, rtol=0)


def test_constant_keys_give_mean_of_values():
    q, _, v = _qkv(1, 2, 20, 8, seed=5)
    k = np.ones_like(q)
    nc = attention_fp64(q, k, v, 0.7, False)
    assert np.allclose(nc, v.astype(np.float64).mean(axis=2, keepdims=True), atol=1e-12)
    c = attention_fp64(q, k, v, 0.7, True)
    prefix = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, 21)[None, None, :, None]
    assert np.allclose(c, prefix, atol=1e-12)


def test_peaked_scores_select_one_row():
    n, d = 16, 8
    _, _, v = _qkv(1, 1, n, d, seed=6)
    k = np.zeros((1, 1, n, d), np.float16)
    k[0, 0, np.arange(n), np.arange(n) % d] = 1.0
    q = np.zeros((1, 1, n, d), np.float16)
    target = (np.arange(n) * 5) % d  # query i points at key with one-hot column target
    q[0, 0, np.arange(n), target] = 1.0
    out = attention_fp64(q, k, v, 200.0, False)
    # keys j with j % d == target tie; weights split evenly among them
    for i in range(n):
        ties = [j for j in range(n) if j % d == target[i]]
        assert np.allclose(out[0, 0, i], v[0, 0, ties].astype(np.float64).mean(0), atol=1e-9)


def test_score_shift_invariance():
    # Adding one vector u to every key row shifts row i's logits by the
    # constant q_i.u, which softmax must ignore (inputs kept in float64).
    q, k, v = _qkv(1, 2, 24, 8, seed=8)
    u = np.linspace(-2.0, 3.0, 8)[None, None, None, :]
    for causal in (False, True):
        a = attention_fp64(q, k, v, 0.3, causal)
        b = attention_fp64(q, k.astype(np.float64) + u, v, 0.3, causal)
        assert np.allclose(a, b, atol=1e-12)


def test_joint_permutation_invariance_noncausal():
    q, k, v = _qkv(1, 2, 31, 16, seed=9)
    perm = np.random.RandomState(1).permutation(31)
    a = attention_fp64(q, k, v, 0.2, False)
    b = attention_fp64(q, k[:, :, perm], v[:, :, perm], 0.2, False)
    assert np.allclose(a, b, atol=1e-12)


def test_causal_ignores_later_keys():
    q, k, v = _qkv(1, 1, 40, 16, seed=11)
    a = attention_fp64(q, k, v, 0.2, True)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 25:] = 3.0
    v2[:, :, 25:] = -7.0
    b = attention_fp64(q, k2, v2, 0.2, True)
    assert np.array_equal(a[:, :, :25], b[:, :, :25])
    assert not np.allclose(a[:, :, 25:], b[:, :, 25:])


def test_linearity_in_values():
    q, k, v = _qkv(1, 1, 19, 8, seed=12)
    _, _, w = _qkv(1, 1, 19, 8, seed=13)
    a = attention_fp64(q, k, v.astype(np.float64) * 2 + w.astype(np.float64), 0.4, True)
    b = 2 * attention_fp64(q, k, v, 0.4, True) + attention_fp64(q, k, w, 0.4, True)
    assert np.allclose(a, b, atol=1e-12)


def test_rows_subset_matches_full():
    q, k, v = _qkv(1, 2, 70, 16, seed=14)
    rows = [0, 5, 69, 33]
    full = attention_fp32(q, k, v, 0.125, True)
    part = attention_fp32(q, k, v, 0.125, True, rows=rows)
    assert np.allclose(part, full[:, :, rows], atol=1e-7)


# --- scale sentinel, prescale, work formulas --------------------------------

def test_scale_sentinel():
    assert resolve_sm_scale(0.0, 64) == 0.125
    assert resolve_sm_scale(0.0, 80) == float(np.float32(1) / np.sqrt(np.float32(80)))
    assert resolve_sm_scale(0.3, 64) == 0.3
    q, k, v = _qkv(1, 1, 9, 64, seed=15)
    assert np.array_equal(attention_fp32(q, k, v, 0.0, True), attention_fp32(q, k, v, 0.125, True))


def test_scale_log2_prescale():
    # kernel_flash2.cu:772 with LOG2_E a float constant
    assert sm_scale_log2(0.125) == np.float32(0.125 * float(np.float32(1.4426950408889634)))
    assert abs(float(sm_scale_log2(0.125)) - 0.125 / math.log(2)) < 1e-7


def test_work_formulas():
    # benchmark_throughput.py:23-31 at the headline config
    assert attention_flops(2, 8, 4096, 64, False) == 4 * 2 * 8 * 4096 ** 2 * 64
    assert attention_flops(2, 8, 4096, 64, True) == 2 * 2 * 8 * 4096 ** 2 * 64
    assert attention_bytes(2, 8, 4096, 64) == 32 * 2 ** 20


# --- N_k != N_q (bottom-right causal) and the log-sum-exp --------------------

def _qkv2(b, h, nq, nk, d, seed):
    rs = np.random.RandomState(seed)
    mk = lambda n: rs.standard_normal((b, h, n, d)).astype(np.float32).astype(np.float16)
    return mk(nq), mk(nk), mk(nk)


@pytest.mark.parametrize("nq,nk", [(1, 5), (3, 7), (7, 3), (5, 1), (4, 4), (2, 9)])
@pytest.mark.parametrize("causal", [False, True])
def test_rectangular_matches_bruteforce(nq, nk, causal):
    q, k, v = _qkv2(1, 2, nq, nk, 8, seed=40 + nq * 10 + nk)
    ref = attention_bruteforce(q, k, v, 0.37, causal)
    assert error_stats(attention_fp64(q, k, v, 0.37, causal), ref)[0] < 1e-12
    assert error_stats(attention_fp32(q, k, v, 0.37, causal), ref)[0] < 2e-6


@pytest.mark.parametrize("nq,nk", [(37, 100), (100, 37), (64, 200), (1, 130)])
def test_rectangular_causal_matches_torch_lower_right(nq, nk):
    """Bottom-right alignment pinned by PyTorch's own causal_lower_right
    bias (a library routine, independent of this oracle's mask code)."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention.bias import causal_lower_right

    q, k, v = _qkv2(2, 3, nq, nk, 64, seed=nq + nk)
    tq, tk, tv = (torch.from_numpy(x.astype(np.float64)) for x in (q, k, v))
    if nq <= nk:
        ref = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=causal_lower_right(nq, nk),
                                             scale=0.125).numpy()
        assert error_stats(attention_fp64(q, k, v, 0.125, True), ref)[0] < 1e-12
    else:
        # rows with no visible key: torch yields NaN there, the reference's rule 0
        ref = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=causal_lower_right(nq, nk),
                                             scale=0.125).numpy()
        out = attention_fp64(q, k, v, 0.125, True)
        empty = nq - nk
        assert np.all(out[:, :, :empty, :] == 0.0)
        assert error_stats(out[:, :, empty:, :], ref[:, :, empty:, :])[0] < 1e-12


def test_rectangular_closed_forms():
    q, _, v = _qkv2(1, 2, 6, 10, 8, seed=50)
    k = np.ones((1, 2, 10, 8), np.float16)
    # constant keys: query i averages V[0 .. i + (10 - 6)]
    c = attention_fp64(q, k, v, 0.7, True)
    vf = v.astype(np.float64)
    for i in range(6):
        assert np.allclose(c[:, :, i, :], vf[:, :, :i + 5, :].mean(axis=2), atol=1e-12)
    # the last query row sees every key: equals the non-causal last row
    q, k, v = _qkv2(1, 2, 6, 10, 8, seed=51)
    assert np.array_equal(attention_fp64(q, k, v, 0.3, True)[:, :, -1],
                          attention_fp64(q, k, v, 0.3, False)[:, :, -1])
    # more queries than keys: the first nq - nk rows see nothing and are 0
    q, k, v = _qkv2(1, 1, 9, 4, 8, seed=52)
    out = attention_fp64(q, k, v, 0.3, True)
    assert np.all(out[:, :, :5] == 0.0) and np.all(np.abs(out[:, :, 5:]).sum(-1) > 0)
    assert np.all(causal_visible(np.arange(9), 9, 4).sum(1) == [0, 0, 0, 0, 0, 1, 2, 3, 4])


def test_lse_closed_forms():
    q, _, _ = _qkv2(1, 2, 7, 11, 16, seed=53)
    zero_k = np.zeros((1, 2, 11, 16), np.float16)
    # all scores 0: lse = ln(#visible keys)
    assert np.allclose(attention_lse(q, zero_k, 0.5, False), math.log(11), atol=1e-15)
    vis = causal_visible(np.arange(7), 7, 11).sum(1)
    assert np.allclose(attention_lse(q, zero_k, 0.5, True), np.log(vis)[None, None, :],
                       atol=1e-15)
    # a row with no visible key: -inf
    lse = attention_lse(*_qkv2(1, 1, 5, 2, 8, seed=54)[:2], 0.5, True)
    assert np.all(np.isneginf(lse[..., :3])) and np.all(np.isfinite(lse[..., 3:]))


def test_lse_matches_torch_logsumexp_and_reproduces_output():
    import torch

    q, k, v = _qkv2(2, 2, 40, 70, 32, seed=55)
    scale = 0.21
    s = torch.from_numpy(q.astype(np.float64)) @ torch.from_numpy(k.astype(np.float64)).transpose(-1, -2)
    s = s * scale
    mask = torch.from_numpy(causal_visible(np.arange(40), 40, 70))
    ref = torch.logsumexp(s.masked_fill(~mask, float("-inf")), dim=-1).numpy()
    lse = attention_lse(q, k, scale, True)
    assert np.allclose(lse, ref, atol=1e-12)
    # softmax weights exp(s - lse) reproduce the oracle's output
    w = np.where(mask.numpy(), np.exp(s.numpy() - lse[..., None]), 0.0)
    assert np.allclose(w.sum(-1), 1.0, atol=1e-12)
    assert np.allclose(w @ v.astype(np.float64), attention_fp64(q, k, v, scale, True), atol=1e-12)
