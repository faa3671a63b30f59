"""GPU parity of the causal pair schedule (fl_attn_fwd_f16_ws): query blocks
hi = n-1-p and lo = p of a head share two work-groups, block hi's key range
split between them and merged through the caller's workspace.

Same tolerance as every other path (north_star: max-abs <= 2e-3, mean-abs
<= 2e-4 against the fp32 oracle; the elementwise half-ulp bound on peaked
inputs).  Beyond parity: the result has the same bits on every call (the
merge is fixed in order whichever work-group arrives last), the workspace
comes back zero-filled, the log-sum-exp agrees with the one-pass launch,
strided views give the contiguous result bit for bit, and a workspace
that is too small or misaligned is refused before anything runs.
"""

import numpy as np
import pytest

from flashlite_amd import capi
from gpu_util import SLOT_W4_CFG, assert_close_oracle, sample_rows, to_dev
from oracle import attention_lse, error_stats

pytestmark = pytest.mark.gpu

LSE_MAX_ABS = 2e-3
LSE_MEAN_ABS = 3e-4


def _qkv(b, h, n, seed, qk_scale=1.0):
    rs = np.random.RandomState(seed)
    mk = lambda c: (rs.standard_normal((b, h, n, 64)) * c).astype(np.float32).astype(np.float16)
    return mk(qk_scale), mk(qk_scale), mk(1.0)


class _Pair:
    """One problem on the device with a zero-filled workspace."""

    def __init__(self, q16, k16, v16, sm_scale, dev, lse=False):
        import torch

        self.torch, self.dev = torch, dev
        self.q, self.k, self.v = (to_dev(x, dev) for x in (q16, k16, v16))
        self.o = torch.full_like(self.q, float("nan"))
        self.lse = (torch.full(self.q.shape[:3], float("nan"), dtype=torch.float32, device=dev)
                    if lse else None)
        self.p = capi.tensor_params_ex(self.q, self.k, self.v, self.o, sm_scale, True,
                                       lse=self.lse)
        self.need = capi.fwd_workspace_bytes(self.p)
        self.ws = torch.zeros(max(self.need, 256), dtype=torch.uint8, device=dev)
        self.stream = torch.cuda.current_stream(dev).cuda_stream

    def run(self):
        self.o.fill_(float("nan"))
        capi.check(capi.fwd_ws(self.p, self.ws.data_ptr(), self.need, self.stream))
        self.torch.cuda.synchronize(self.dev)
        return self.o.cpu().numpy()


# (B, H, N): 128-row blocks that fill the CUs in one round (B*H*N/128 <= 512),
# B*H a multiple of 8.  The cut falls in block hi, exactly between the two
# blocks, or in block lo, depending on the pair.
SHAPES = [(2, 8, 768), (2, 8, 1024), (1, 8, 1024), (2, 8, 2048), (1, 8, 2048), (1, 8, 4096),
          (2, 8, 4096), (1, 16, 4096)]


@pytest.mark.parametrize("b,h,n", SHAPES)
def test_pair_parity(cuda, b, h, n):
    q, k, v = _qkv(b, h, n, seed=n + 11 * h + b)
    run = _Pair(q, k, v, 0.125, cuda)
    assert run.need > 0, "the pair schedule should apply to this shape"
    out = run.run()
    rows = None if b * h * n <= 16 * 1024 else sample_rows(n, seed=n)
    assert_close_oracle(out, q, k, v, 0.125, True, rows=rows)
    # every row written, not only the checked ones
    assert np.isfinite(out).all()


@pytest.mark.parametrize("qk_scale", [2.5, 4.0])
def test_pair_peaked_checked_pass(cuda, qk_scale):
    # Large logits send blocks to the checked pass in either member.
    q, k, v = _qkv(1, 8, 1024, seed=5, qk_scale=qk_scale)
    out = _Pair(q, k, v, 0.125, cuda).run()
    assert_close_oracle(out, q, k, v, 0.125, True, peaked=True)


def test_pair_same_bits_and_workspace_left_zero(cuda):
    import torch

    q, k, v = _qkv(2, 8, 2048, seed=3)
    run = _Pair(q, k, v, 0.125, cuda)
    first = run.run()
    assert int(torch.count_nonzero(run.ws[:256])) == 0, "pair flags not reset"
    for _ in range(3):
        again = run.run()
        assert np.array_equal(first.view(np.uint16), again.view(np.uint16))


def test_pair_close_to_one_pass(cuda):
    import torch

    q, k, v = _qkv(2, 8, 4096, seed=9)
    out = _Pair(q, k, v, 0.125, cuda).run()
    tq, tk, tv = (to_dev(x, cuda) for x in (q, k, v))
    o1 = torch.empty_like(tq)
    p1 = capi.tensor_params_ex(tq, tk, tv, o1, 0.125, True)
    capi.check(capi.fwd_ex(p1, torch.cuda.current_stream(cuda).cuda_stream, SLOT_W4_CFG))
    torch.cuda.synchronize(cuda)
    mx, mean = error_stats(out, o1.cpu().numpy())
    assert mx <= 2e-3 and mean <= 1e-5, (mx, mean)


def test_pair_lse(cuda):
    q, k, v = _qkv(1, 8, 2048, seed=21)
    run = _Pair(q, k, v, 0.125, cuda, lse=True)
    out = run.run()
    assert_close_oracle(out, q, k, v, 0.125, True)
    ref = attention_lse(q, k, 0.125, True)
    mx, mean = error_stats(run.lse.cpu().numpy(), ref)
    assert mx <= LSE_MAX_ABS and mean <= LSE_MEAN_ABS, (mx, mean)


def test_pair_strided_equals_contiguous(cuda):
    import torch

    b, h, n = 2, 8, 1024
    q, k, v = _qkv(b, h, n, seed=17)
    contiguous = _Pair(q, k, v, 0.125, cuda).run()
    # [B, N, H, D] storage viewed as [B, H, N, D]
    tq, tk, tv = (to_dev(np.ascontiguousarray(x.transpose(0, 2, 1, 3)), cuda).transpose(1, 2)
                  for x in (q, k, v))
    o = torch.full((b, n, h, 64), float("nan"), dtype=torch.float16, device=cuda).transpose(1, 2)
    p = capi.tensor_params_ex(tq, tk, tv, o, 0.125, True)
    need = capi.fwd_workspace_bytes(p)
    ws = torch.zeros(need, dtype=torch.uint8, device=cuda)
    capi.check(capi.fwd_ws(p, ws.data_ptr(), need, torch.cuda.current_stream(cuda).cuda_stream))
    torch.cuda.synchronize(cuda)
    got = o.contiguous().cpu().numpy()
    assert np.array_equal(got.view(np.uint16), contiguous.view(np.uint16))


def test_pair_workspace_checks(cuda):
    import torch

    q, k, v = _qkv(1, 8, 1024, seed=2)
    run = _Pair(q, k, v, 0.125, cuda)
    rc = capi.fwd_ws(run.p, run.ws.data_ptr(), run.need - 4, run.stream)
    assert rc == capi.FL_ERR_INVALID_ARGUMENT and "workspace of" in capi.last_error()
    rc = capi.fwd_ws(run.p, 0, run.need, run.stream)
    assert rc == capi.FL_ERR_INVALID_ARGUMENT
    big = torch.zeros(run.need + 512, dtype=torch.uint8, device=cuda)
    rc = capi.fwd_ws(run.p, big.data_ptr() + 16, run.need, run.stream)
    assert rc == capi.FL_ERR_MISALIGNED
    torch.cuda.synchronize(cuda)
    assert bool(torch.isnan(run.o).all()), "a refused call must not launch"
