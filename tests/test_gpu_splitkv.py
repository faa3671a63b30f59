"""GPU parity of split-KV ("flash-decoding"): the key range cut into chunks,
partial results merged by a second kernel.  Same tolerances as the one-pass
kernel against the fp32 oracle (max-abs 2e-3, mean-abs 2e-4; log-sum-exp
2e-3 / 3e-4, see test_gpu_rect_strided.py), on decode-like shapes (one or a
few query rows over many keys), both masks (causal aligned bottom-right),
forced and automatic chunk counts, empty chunks past the causal limit."""

import numpy as np
import pytest

from flashlite_amd import capi
from gpu_util import assert_close_oracle, to_dev
from gpu_util import run_splitkv as _run_split
from oracle import attention_fp32, attention_lse, error_stats

pytestmark = pytest.mark.gpu

LSE_MAX_ABS = 2e-3
LSE_MEAN_ABS = 3e-4


def _qkv(b, h, nq, nk, seed):
    rs = np.random.RandomState(seed)
    mk = lambda n: rs.standard_normal((b, h, n, 64)).astype(np.float32).astype(np.float16)
    return mk(nq), mk(nk), mk(nk)


# (2, 9000) with 1000 requested: 141 chunks, more than one wave's 64 lanes
# in the combine
SHAPES = [(1, 4096), (1, 1000), (4, 777), (32, 4096), (33, 2048), (100, 3000), (1, 64),
          (100, 130), (2, 9000)]


@pytest.mark.parametrize("nq,nk", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("splits", [1, 3, 0, 1000])
def test_splitkv_matches_oracle(cuda, nq, nk, causal, splits):
    q16, k16, v16 = _qkv(2, 4, nq, nk, seed=nq * 13 + nk)
    tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
    o, ls, need = _run_split(tq, tk, tv, 0.125, causal, splits)
    if splits > 0:
        tiles = (nk + 63) // 64
        assert need == min(splits, tiles, 256) * 2 * 4 * nq * 68 * 4
    out = o.float().cpu().numpy()
    assert_close_oracle(out, q16, k16, v16, 0.125, causal,
                        ref=attention_fp32(q16, k16, v16, 0.125, causal))
    lse = ls.cpu().numpy()
    ref = attention_lse(q16, k16, 0.125, causal)
    assert np.array_equal(np.isneginf(lse), np.isneginf(ref))
    fin = np.isfinite(ref)
    mx, mean = error_stats(lse[fin], ref[fin])
    assert mx <= LSE_MAX_ABS and mean <= LSE_MEAN_ABS, f"lse max-abs {mx:.3e} mean-abs {mean:.3e}"


@pytest.mark.parametrize("nq", [1, 40, 100])  # 1-, 2- and 4-wave chunks
@pytest.mark.parametrize("causal", [False, True])
def test_splitkv_peaked(cuda, nq, causal):
    # sm_scale 3 (logits with std ~24) and, in the second tile of every
    # chunk (5 chunks of 5 tiles), a copy of query row 0 as a key: every
    # chunk measures that key far above its first tile and takes the checked
    # pass; the combine kernel merges partials whose maxima differ by hundreds
    from gpu_util import redo_expected

    q16, k16, v16 = _qkv(1, 4, nq, 1500, seed=nq + 5)
    per = 5 * 64
    for c0 in range(0, 1500, per):
        k16[:, :, c0 + 64 + 7] = q16[:, :, 0]
        # chunk starts are tile-aligned: the chunk alone shows the condition
        assert redo_expected(q16, k16[:, :, c0:c0 + per], 3.0, False)
    tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
    o, ls, _ = _run_split(tq, tk, tv, 3.0, causal, 5)
    assert_close_oracle(o.float().cpu().numpy(), q16, k16, v16, 3.0, causal, peaked=True,
                        ref=attention_fp32(q16, k16, v16, 3.0, causal))
    lse, ref = ls.cpu().numpy(), attention_lse(q16, k16, 3.0, causal)
    mx, mean = error_stats(lse, ref)
    assert mx <= LSE_MAX_ABS and mean <= LSE_MEAN_ABS, f"lse max-abs {mx:.3e} mean-abs {mean:.3e}"


def test_splitkv_auto_choice(cuda):
    # a decode step on a small batch splits; the headline shape does not
    q16, k16, v16 = _qkv(2, 8, 1, 4096, seed=1)
    tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
    _, _, need = _run_split(tq, tk, tv, 0.125, False, 0)
    assert need == 8 * 16 * 68 * 4  # 8 key-quarter chunks of 8 tiles


def test_splitkv_strided_and_deterministic(cuda):
    import torch

    q16, k16, v16 = _qkv(2, 3, 5, 2000, seed=2)
    tq, tk, tv = (to_dev(x, cuda) for x in (q16, k16, v16))
    a, la, _ = _run_split(tq, tk, tv, 0.125, True, 7)
    b, lb, _ = _run_split(tq, tk, tv, 0.125, True, 7)
    assert torch.equal(a, b) and torch.equal(la, lb)
    # [B, N, H, D] storage gives the same bits
    qb, kb, vb = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (tq, tk, tv))
    c, lc, _ = _run_split(qb, kb, vb, 0.125, True, 7)
    assert torch.equal(c, a) and torch.equal(lc, la)


def test_binding_splitkv(cuda):
    import torch

    import flashlite_amd as fl

    q16, k16, v16 = _qkv(2, 8, 1, 4096, seed=3)
    q, k, v = (to_dev(x, cuda) for x in (q16, k16, v16))
    need = fl.splitkv_workspace_bytes(q, k, False, 0)
    assert need > 0
    ws = torch.empty(need // 4, dtype=torch.float32, device=cuda)
    out = torch.empty_like(q)
    got, lse = fl.forward_flash2_ex(q, k, v, 0.125, False, out=out, return_lse=True, workspace=ws)
    torch.cuda.synchronize()
    assert got.data_ptr() == out.data_ptr()
    assert_close_oracle(got.float().cpu().numpy(), q16, k16, v16, 0.125, False)
    ref_lse = attention_lse(q16, k16, 0.125, False)
    assert error_stats(lse.cpu().numpy(), ref_lse)[0] <= LSE_MAX_ABS
    # num_splits=1: the one-pass kernel, bit-identical to forward_flash2
    one = fl.forward_flash2_ex(q, k, v, 0.125, False, num_splits=1)
    assert torch.equal(one, fl.forward_flash2(q, k, v, 0.125, False))
    assert fl.splitkv_workspace_bytes(q, k, False, 1) == 0
