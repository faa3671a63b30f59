"""CPU checks of the paths beyond the reference's element type and head dim:
the bf16 input rounding, and the C ABI's argument checks for bf16 and
head_dim 128 (rejections happen before any launch, so no GPU is needed)."""

import numpy as np
import torch

from flashlite_amd import capi
from flashlite_amd.workloads import make_qkv, make_qkv_bf16, round_bf16

A = 0x7F0000000000  # fake, aligned device addresses: never dereferenced here


def test_round_bf16_matches_torch():
    """round_bf16 is torch's own float32 -> bfloat16 conversion (round to
    nearest even), over magnitudes from subnormal to 1e30."""
    rs = np.random.RandomState(0)
    x = (rs.standard_normal(200_000) * np.exp(rs.uniform(-90, 70, 200_000))).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(round_bf16(x), ref)


def test_round_bf16_closed_forms():
    """Ties go to the even neighbour; exact values are kept."""
    one_ulp = 2.0 ** -7  # bf16 ulp at 1
    cases = {
        1.0: 1.0,
        1.0 + one_ulp / 2: 1.0,                     # tie, 1.0 is even
        1.0 + 3 * one_ulp / 2: 1.0 + 2 * one_ulp,   # tie, 1 + 2 ulp is even
        1.0 + one_ulp / 2 + 2.0 ** -20: 1.0 + one_ulp,
        -(1.0 + one_ulp / 2): -1.0,
        3.140625: 3.140625,                         # exactly representable
    }
    x = np.array(list(cases), dtype=np.float32)
    assert np.array_equal(round_bf16(x), np.array(list(cases.values()), dtype=np.float32))


def test_make_qkv_bf16_rounds_the_make_qkv_stream():
    q, k, v = make_qkv_bf16(1, 2, 64, 64, seed=4)
    q16, k16, v16 = make_qkv(1, 2, 64, 64, seed=4)
    for b, h in ((q, q16), (k, k16), (v, v16)):
        assert np.array_equal(round_bf16(b), b)  # bf16-exact
        # the same draws: the bf16 and fp16 roundings differ by < 2^-8 relative
        assert (np.abs(b - h.astype(np.float32)) <= 2.0 ** -8 * np.abs(b) + 1e-6).all()


def _ex(head_dim=128, **kw):
    base = dict(q=A, k=A + 0x1000000, v=A + 0x2000000, o=A + 0x3000000, batch=2, heads=8,
                seq_q=4096, head_dim=head_dim, sm_scale=0.125, causal=False)
    base.update(kw)
    p = capi.make_params(**base)
    c = (8 * 4096 * head_dim, 4096 * head_dim, head_dim)
    return capi.make_params_ex(p, c, c, c, c, 0)


def test_wide_config_checks():
    for fn, who in ((capi.fwd_ex, "fl_attn_fwd_f16_ex"), (capi.fwd_bf16_ex, "fl_attn_fwd_bf16_ex")):
        for d in (64, 128):
            if fn is capi.fwd_ex and d == 64:
                continue  # fp16 at D = 64 has every configuration
            slots = (capi.config_id("br256_bc64_w8_slot"), capi.config_id("br128_bc64_w4_slot"))
            stream_cfg = capi.config_id("br256_kv256_w8_stream")
            quarter_cfg = capi.config_id("br32_kv512_w4_quarters")
            # bf16 at D = 64 also has both key-range splits and both block pairs
            # (and the streaming and key-quarter kernels, checked below)
            splits = (capi.config_id("br128_bc64_w4x2_slot"), capi.config_id("br64_bc64_w2x2_slot"),
                      capi.config_id("br128_bc64_w4x2_pair"), capi.config_id("br64_bc64_w2x2_pair"))
            for cfg in range(capi.num_configs()):
                if cfg in slots or cfg in (stream_cfg, quarter_cfg):
                    continue
                if d == 64 and cfg in splits:
                    assert fn(_ex(head_dim=d), config=cfg) != capi.FL_ERR_BAD_CONFIG
                    continue
                assert fn(_ex(head_dim=d), config=cfg) == capi.FL_ERR_BAD_CONFIG
                assert "not built" in capi.last_error() and who in capi.last_error()
            # N_k 4096: past both short-key kernels' limits (not built at D = 128)
            assert fn(_ex(head_dim=d), config=stream_cfg) == capi.FL_ERR_BAD_CONFIG
            assert fn(_ex(head_dim=d), config=quarter_cfg) == capi.FL_ERR_BAD_CONFIG
            if d == 64:
                assert "needs N_k" in capi.last_error()
        for d in (32, 96, 256):
            assert fn(_ex(head_dim=d)) == capi.FL_ERR_UNSUPPORTED
            assert "head_dim must be 64 or 128" in capi.last_error()


def test_reference_entries_keep_head_dim_64():
    p = capi.make_params(A, A + 0x1000000, A + 0x2000000, A + 0x3000000, 2, 8, 4096, 4096, 128,
                         0.125, False)
    assert capi.fwd(p) == capi.FL_ERR_UNSUPPORTED
    assert capi.last_error() == "FlashLite WMMA kernel currently requires head_dim == 64"
    assert capi.select_config(p) == -1


def test_splitkv_stays_fp16_head_dim_64():
    assert capi.splitkv_workspace_bytes(_ex(head_dim=128, seq_q=1), 4) == -1
    assert "requires head_dim == 64" in capi.last_error()


def test_wide_stride_limits():
    # rows of a head_dim-128 tensor must be at least 128 elements apart
    p = capi.make_params(A, A + 0x1000000, A + 0x2000000, A + 0x3000000, 1, 1, 64, 64, 128,
                         0.125, False)
    bad = capi.make_params_ex(p, (64 * 128, 64 * 128, 64), (64 * 128, 64 * 128, 128),
                              (64 * 128, 64 * 128, 128), (64 * 128, 64 * 128, 128), 0)
    assert capi.fwd_bf16_ex(bad) == capi.FL_ERR_UNSUPPORTED
    assert "row stride 64 must be in [128" in capi.last_error()
