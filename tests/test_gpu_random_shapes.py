"""Seeded random shapes against the CPU oracle, through the C ABI: every tile
configuration that takes the key range, plus the dispatcher's choice, on the
same inputs.  A broad sweep beside the targeted tests: batch and head counts,
query and key lengths drawn independently (N_k != N_q both ways, so causal
rows with no visible key occur), both masks, and the scale sentinel (0.0),
negative, small and peaked (1.0) scales.  Inputs are N(0,1) in fp16, as the
reference's tests draw them (tests/test_correctness.py:38-41)."""

import numpy as np
import pytest

from flashlite_amd import capi
from gpu_util import assert_close_oracle, config_fits, run_capi
from oracle import attention_fp32

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
    peaked = abs(scale) >= 1.0
    for config in [-1] + list(range(NCFG)):
        if config >= 0 and not config_fits(config, nk):
            continue
        print(f"random shape {_case_id(case)} config={config}", flush=True)
        out = run_capi(q, k, v, scale, causal, cuda, config=config)
        assert_close_oracle(out, q, k, v, scale, causal, ref=ref, peaked=peaked)
