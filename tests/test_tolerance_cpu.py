"""The elementwise tolerance of the peaked-scale GPU tests: half_ulp must be
half of numpy's fp16 (and bf16-width) spacing, so a peaked output is allowed
exactly its own rounding on top of the 2e-3 budget."""

import numpy as np

from gpu_util import half_ulp


def test_half_ulp_fp16_matches_numpy_spacing():
    rs = np.random.RandomState(0)
    x = np.concatenate([rs.standard_normal(4096) * 3, [1.0, 2.0, 4.0, 0.5, 30000.0, 6.1e-5]])
    x16 = x.astype(np.float16)
    want = np.spacing(np.abs(x16)).astype(np.float64) / 2
    assert np.array_equal(half_ulp(x16.astype(np.float32)), want)


def test_half_ulp_bf16_width_and_edges():
    # bf16 keeps 7 stored bits: ulp(1) = 2^-7, ulp(4.5) = 2^-5
    assert half_ulp(np.array([1.0, 4.5, -3.0]), 7).tolist() == [2.0 ** -8, 2.0 ** -6, 2.0 ** -7]
    # zero and fp16 subnormals: half of the subnormal step
    assert half_ulp(np.array([0.0, 2.0 ** -20])).tolist() == [2.0 ** -25, 2.0 ** -25]
