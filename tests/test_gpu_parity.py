"""Parity of the HIP path (through the C ABI) with the CPU oracle on the GPU.

Tolerance (north_star): max-abs <= 2e-3 and mean-abs <= 2e-4 of the fp16
output against softmax(Q K^T * sm_scale) V in fp32 on the same seeded inputs.
Outputs start as NaN so a row the kernel fails to write fails the check.
"""

import os

import numpy as np
import pytest

from flashlite_amd import capi
from flashlite_amd.workloads import WORKLOADS, make_qkv, workload_inputs
from gpu_util import (PAIR64_CFG, PAIR_CFG, SLOT_W4_CFG, SLOT_W8_CFG, SPLIT2_CFG, SPLIT2W2_CFG,
                      assert_close_oracle,
                      config_fits, redo_expected, run_capi, to_dev)
from oracle import attention_fp32, error_stats

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
NCFG = 10  # tile configurations exported by the library
# the key-range-split configurations
SPLIT_CFGS = [SPLIT2_CFG, SPLIT2W2_CFG, PAIR_CFG, PAIR64_CFG]


def test_num_configs():
    assert capi.num_configs() == NCFG
    assert [capi.config_name(i) for i in range(NCFG)] == [
        "br32_bc64_w1", "br64_bc64_w2", "br128_bc64_w4x2_slot", "br256_bc64_w8_slot",
        "br128_bc64_w4_slot", "br256_kv256_w8_stream", "br32_kv512_w4_quarters",
        "br64_bc64_w2x2_slot", "br128_bc64_w4x2_pair", "br64_bc64_w2x2_pair"]


@pytest.mark.parametrize("config", list(range(NCFG)))
@pytest.mark.parametrize("causal", [False, True])
def test_c0_golden(cuda, config, causal):
    z = np.load(os.path.join(GOLDEN, "c0_golden.npz"))
    out = run_capi(z["q"], z["k"], z["v"], 0.125, causal, cuda, config=config)
    ref = z["out_causal" if causal else "out_noncausal"]
    assert_close_oracle(out, z["q"], z["k"], z["v"], 0.125, causal, ref=ref)


@pytest.mark.parametrize("name", ["C1_short_B2H8N512", "sweep_B2H8N1024", "sweep_B2H8N2048",
                                  "C2_headline_B2H8N4096"])
@pytest.mark.parametrize("causal", [False, True])
def test_benchmark_configs(cuda, name, causal):
    # every output row, the headline shape included
    w = WORKLOADS[name]
    q, k, v = workload_inputs(w)
    out = run_capi(q, k, v, w.sm_scale, causal, cuda)
    mx, mean = assert_close_oracle(out, q, k, v, w.sm_scale, causal)
    print(f"{name} causal={causal}: max-abs {mx:.2e} mean-abs {mean:.2e}")


_C2_REF = {}


def _c2_ref(causal):
    """The fp32 oracle of the whole C2 headline output (cached per mask)."""
    if causal not in _C2_REF:
        w = WORKLOADS["C2_headline_B2H8N4096"]
        q, k, v = workload_inputs(w)
        _C2_REF[causal] = attention_fp32(q, k, v, w.sm_scale, causal)
    return _C2_REF[causal]


@pytest.mark.parametrize("config", [SLOT_W8_CFG, SLOT_W4_CFG] + SPLIT_CFGS)
@pytest.mark.parametrize("causal", [False, True])
def test_headline_each_config(cuda, config, causal):
    # every output row of the headline shape, on every configuration that can
    # serve it
    w = WORKLOADS["C2_headline_B2H8N4096"]
    q, k, v = workload_inputs(w)
    out = run_capi(q, k, v, w.sm_scale, causal, cuda, config=config)
    mx, mean = assert_close_oracle(out, q, k, v, w.sm_scale, causal, ref=_c2_ref(causal))
    print(f"C2 config {config} causal={causal}, every row: max-abs {mx:.2e} mean-abs {mean:.2e}")


@pytest.mark.parametrize("config", SPLIT_CFGS)
@pytest.mark.parametrize("scale", [-0.2, 1.0, 3.0])
@pytest.mark.parametrize("causal", [False, True])
def test_split_scales(cuda, config, scale, causal):
    # peaked softmax: the stabiliser moves in both key ranges before the merge
    q, k, v = make_qkv(1, 4, 700, 64, seed=43)
    out = run_capi(q, k, v, scale, causal, cuda, config=config)
    assert_close_oracle(out, q, k, v, scale, causal, peaked=scale >= 1)


def test_c3_long_causal(cuda):
    w = WORKLOADS["C3_long_B1H16N16384"]
    q, k, v = workload_inputs(w)
    out = run_capi(q, k, v, w.sm_scale, True, cuda)
    mx, mean = assert_close_oracle(out, q, k, v, w.sm_scale, True)  # all 16384 rows
    print(f"C3 all rows: max-abs {mx:.2e} mean-abs {mean:.2e}")
    # causal row 0 sees only key 0: the output is V[0] exactly
    assert np.array_equal(out[:, :, 0], v[:, :, 0])


def test_pairs64_dispatch(cuda):
    # a square causal problem the dispatcher gives the 64-row block pairs
    # (192 pairs: an odd head count, heads split across work-groups' XCDs);
    # every output row
    q, k, v = make_qkv(1, 3, 8192, 64, seed=97)
    tq, tk, tv = (to_dev(x, cuda) for x in (q, k, v))
    assert capi.select_config(capi.tensor_params(tq, tk, tv, tq, 0.125, True)) == PAIR64_CFG
    out = run_capi(q, k, v, 0.125, True, cuda)
    mx, mean = assert_close_oracle(out, q, k, v, 0.125, True)
    print(f"B1 H3 N8192 causal, 64-row pairs, every row: max-abs {mx:.2e} mean-abs {mean:.2e}")
    assert np.array_equal(out[:, :, 0], v[:, :, 0])


def test_c4_many_small_heads(cuda):
    w = WORKLOADS["C4_many_B32H32N256"]
    q, k, v = workload_inputs(w)
    out = run_capi(q, k, v, w.sm_scale, True, cuda)
    assert_close_oracle(out, q, k, v, w.sm_scale, True)


# More than 256 blocks of 32 query rows: the key-quarter kernel runs 8-wave
# groups of two row blocks (a ragged last group, N_q != N_k both ways).
QUARTER_RB2 = [(4, 8, 512, 512), (5, 7, 300, 300), (4, 20, 130, 400), (3, 11, 400, 130)]


@pytest.mark.parametrize("b,h,nq,nk", QUARTER_RB2)
@pytest.mark.parametrize("causal", [False, True])
def test_quarter_two_row_blocks(cuda, b, h, nq, nk, causal):
    assert b * h * ((nq + 31) // 32) > 256
    rs = np.random.RandomState(b * 1000 + h * 10 + nq + nk)
    mk = lambda n: rs.standard_normal((b, h, n, 64)).astype(np.float32).astype(np.float16)  # noqa: E731
    q, k, v = mk(nq), mk(nk), mk(nk)
    cfg = capi.config_id("br32_kv512_w4_quarters")
    print(f"quarter RB2 B{b} H{h} Nq{nq} Nk{nk} causal={causal}", flush=True)
    out = run_capi(q, k, v, 0.125, causal, cuda, config=cfg)
    assert_close_oracle(out, q, k, v, 0.125, causal)
    # peaked scores take the checked softmax in every quarter
    out = run_capi(q, k, v, 3.0, causal, cuda, config=cfg)
    assert_close_oracle(out, q, k, v, 3.0, causal, peaked=True)


RAGGED = [1, 2, 3, 17, 31, 32, 33, 63, 64, 65, 100, 127, 128, 129, 191, 255, 256, 257, 300, 513]


@pytest.mark.parametrize("config", list(range(NCFG)))
@pytest.mark.parametrize("causal", [False, True])
def test_ragged_all_configs(cuda, config, causal):
    for n in RAGGED:
        q, k, v = make_qkv(2, 3, n, 64, seed=1000 + n)
        if not config_fits(config, n):
            with pytest.raises(RuntimeError, match="needs N_k <= "):
                run_capi(q, k, v, 0.125, causal, cuda, config=config)
            continue
        out = run_capi(q, k, v, 0.125, causal, cuda, config=config)
        try:
            assert_close_oracle(out, q, k, v, 0.125, causal)
        except AssertionError as e:
            raise AssertionError(f"N={n}: {e}") from None


def test_scale_sentinel_bitwise(cuda):
    q, k, v = make_qkv(1, 4, 300, 64, seed=31)
    a = run_capi(q, k, v, 0.0, True, cuda)
    b = run_capi(q, k, v, 0.125, True, cuda)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("scale", [-0.2, 0.05, 1.0, 3.0])
@pytest.mark.parametrize("causal", [False, True])
def test_other_scales(cuda, scale, causal):
    # 1.0 and 3.0 make the softmax nearly one-hot (logits with std 8 and 24);
    # the negative scale exercises the sign flip of Q.
    # For scale >= 1 the output is nearly a single V row, so |O| reaches 4-5
    # where one fp16 ulp of the output alone is 3.9e-3; the bound there is,
    # per element, the output's own half-ulp on top of the 2e-3 budget.
    q, k, v = make_qkv(1, 4, 257, 64, seed=41)
    # the peaked cases must take the kernel's checked (rescaling) pass
    assert redo_expected(q, k, scale, causal) == (scale >= 1.0)
    out = run_capi(q, k, v, scale, causal, cuda)
    assert_close_oracle(out, q, k, v, scale, causal, peaked=scale >= 1)


@pytest.mark.parametrize("config", range(NCFG))
@pytest.mark.parametrize("scale", [1.0, 3.0])
@pytest.mark.parametrize("causal", [False, True])
def test_peaked_every_config(cuda, config, scale, causal):
    # Every configuration's work-group-wide redo decision: the peaked inputs
    # send blocks to the checked pass, whose flag each kernel keeps in its
    # idle ring memory.  300 query rows give 1-10 work-groups per head, so
    # groups that redo run beside groups that do not.
    n = 256 if not config_fits(config, 300) else 300
    q, k, v = make_qkv(1, 4, n, 64, seed=47)
    assert redo_expected(q, k, scale, causal)
    out = run_capi(q, k, v, scale, causal, cuda, config=config)
    assert_close_oracle(out, q, k, v, scale, causal, peaked=True)


def _second_block_dominates(gap, seed):
    """B1 H4 N1024 inputs whose keys 32-63 of every 64-key tile score `gap`
    base-2 logits above keys 0-31 for every row: the slot-scheduled kernels
    take their stabiliser from keys 0-31 of a walk's first tile, so p of the
    other half reaches 2^gap in the first pass."""
    rs = np.random.RandomState(seed)
    n, d = 1024, 64
    q = (rs.standard_normal((1, 4, n, d)) * 0.3).astype(np.float32)
    k = (rs.standard_normal((1, 4, n, d)) * 0.3).astype(np.float32)
    v = rs.standard_normal((1, 4, n, d)).astype(np.float32)
    # score gap = a * b * sm_scale * log2 e with sm_scale 1/8
    ab = gap / (0.125 * 1.4426950408889634)
    q[..., 0] = np.sqrt(ab)
    k[..., 0] = np.where((np.arange(n) % 64) >= 32, np.sqrt(ab), 0.0)
    return q.astype(np.float16), k.astype(np.float16), v.astype(np.float16)


@pytest.mark.parametrize("config", range(NCFG))
@pytest.mark.parametrize("gap", [8.0, 24.0])
@pytest.mark.parametrize("causal", [False, True])
def test_first_tile_second_half_dominates(cuda, config, gap, causal):
    # gap 8: p up to 2^8 beside the stabiliser, no checked pass; gap 24: p
    # past fp16's range (2^24), which the range check sends to the checked
    # pass.  Either way the result is the oracle's.
    q, k, v = _second_block_dominates(gap, seed=71)
    if not config_fits(config, k.shape[2]):
        q, k, v = q[:, :, :256], k[:, :, :256], v[:, :, :256]
    out = run_capi(q, k, v, 0.125, causal, cuda, config=config)
    assert_close_oracle(out, q, k, v, 0.125, causal, peaked=True)


def test_deterministic(cuda):
    q, k, v = make_qkv(2, 8, 1000, 64, seed=51)
    for causal in (False, True):
        a = run_capi(q, k, v, 0.125, causal, cuda)
        b = run_capi(q, k, v, 0.125, causal, cuda)
        assert np.array_equal(a, b)


@pytest.mark.parametrize("config", list(range(NCFG)))
def test_no_writes_outside_output(cuda, config):
    # o sits inside a larger buffer with guard regions on both sides.
    import torch

    b, h, n, d = 2, 3, 130, 64
    q, k, v = make_qkv(b, h, n, d, seed=61)
    tq, tk, tv = (to_dev(x, cuda) for x in (q, k, v))
    guard = 4096
    numel = b * h * n * d
    buf = torch.full((guard + numel + guard,), 7.0, dtype=torch.float16, device=cuda)
    o = buf[guard:guard + numel].view(b, h, n, d)
    p = capi.tensor_params(tq, tk, tv, o, 0.125, True)
    capi.check(capi.fwd(p, torch.cuda.current_stream().cuda_stream, config))
    torch.cuda.synchronize()
    host = buf.cpu().numpy()
    assert (host[:guard] == 7.0).all() and (host[guard + numel:] == 7.0).all()
    assert_close_oracle(o.cpu().numpy(), q, k, v, 0.125, True)


def test_out_aliases_q(cuda):
    import torch

    q, k, v = make_qkv(2, 4, 200, 64, seed=71)
    ref = run_capi(q, k, v, 0.125, False, cuda)
    tq, tk, tv = (to_dev(x, cuda) for x in (q, k, v))
    p = capi.tensor_params(tq, tk, tv, tq, 0.125, False)
    capi.check(capi.fwd(p, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert np.array_equal(tq.cpu().numpy(), ref)


def test_empty_problem_is_noop(cuda):
    p = capi.make_params(0, 0, 0, 0, 2, 8, 0, 0, 64, 0.125, True)
    assert capi.fwd(p) == capi.FL_OK


# --- naive baseline kernel ---------------------------------------------------

@pytest.mark.parametrize("causal", [False, True])
def test_naive_c1(cuda, causal):
    w = WORKLOADS["C1_short_B2H8N512"]
    q, k, v = workload_inputs(w)
    out = run_capi(q, k, v, w.sm_scale, causal, cuda, naive=True)
    assert_close_oracle(out, q, k, v, w.sm_scale, causal)


@pytest.mark.parametrize("d", [1, 8, 32, 64, 80, 128, 200])
@pytest.mark.parametrize("causal", [False, True])
def test_naive_head_dims_and_ragged(cuda, d, causal):
    for n in (1, 5, 64, 257):
        q, k, v = make_qkv(1, 3, n, d, seed=2000 + d + n)
        out = run_capi(q, k, v, 0.0, causal, cuda, naive=True)
        assert_close_oracle(out, q, k, v, 0.0, causal)


def test_naive_matches_flash2(cuda):
    q, k, v = make_qkv(2, 2, 384, 64, seed=81)
    for causal in (False, True):
        a = run_capi(q, k, v, 0.125, causal, cuda, naive=True)
        b = run_capi(q, k, v, 0.125, causal, cuda)
        assert error_stats(a, b)[0] < 2e-3


# The block-pair schedule (a work-group walks blocks p and nqb-1-p): even and
# odd block counts (an odd count leaves the middle block alone), ragged
# last blocks, N_k != N_q both ways (bottom-right diagonal), every row.
PAIR_SHAPES = [(2, 8, 4096, 4096), (1, 3, 640, 640), (2, 2, 1000, 1000), (1, 4, 384, 1500),
               (1, 2, 1500, 384), (3, 5, 129, 129)]


@pytest.mark.parametrize("b,h,nq,nk", PAIR_SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_pair_schedule(cuda, b, h, nq, nk, causal):
    rs = np.random.RandomState(b * 7919 + h * 104729 + nq * 31 + nk)
    mk = lambda n: rs.standard_normal((b, h, n, 64)).astype(np.float32).astype(np.float16)  # noqa: E731
    q, k, v = mk(nq), mk(nk), mk(nk)
    print(f"pair schedule B{b} H{h} Nq{nq} Nk{nk} causal={causal}", flush=True)
    out = run_capi(q, k, v, 0.125, causal, cuda, config=PAIR_CFG)
    assert_close_oracle(out, q, k, v, 0.125, causal)
    # peaked scores send blocks to the checked pass in both blocks of a pair
    out = run_capi(q, k, v, 3.0, causal, cuda, config=PAIR_CFG)
    assert_close_oracle(out, q, k, v, 3.0, causal, peaked=True)
