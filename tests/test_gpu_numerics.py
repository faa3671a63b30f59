"""Full-output error of the shipped arithmetic against the reference's.

For every BASELINE configuration (C1-C4, both masks where the configuration
has them), every output row is compared with the fp32 oracle for:

* the library's choice (``config=-1``): fp16 Q prescaled by
  ``|sm_scale| * log2 e``, packed-fp16 row-sum tree on unmasked tiles;
* the ``*_exact`` slot configuration: the reference's arithmetic -- Q
  unscaled, fp32 scores multiplied by ``sm_scale * log2 e``
  (``kernel_flash2.cu:188-195``, ``:529-536``), fp32 sums of the unrounded
  p (``:268-276``, ``:339``);
* ``br256_bc64_w4_pair``: fp16 Q prescaled as the library's choice, fp32
  sums of the unrounded p (the reference's row sums only);
* the floor: the oracle's own fp32 output rounded to fp16, i.e. the error
  any fp16 output has at best.

Each row of the printed table is ``workload mask variant max-abs mean-abs``
(run with ``-s`` to see it).  Every variant must meet the north_star bound
(max-abs 2e-3, mean-abs 2e-4).
"""

import numpy as np
import pytest

from flashlite_amd import capi
from flashlite_amd.workloads import WORKLOADS, workload_inputs
from gpu_util import MAX_ABS, MEAN_ABS, run_capi
from oracle import attention_fp32, error_stats

pytestmark = pytest.mark.gpu

CASES = [
    ("C1_short_B2H8N512", False), ("C1_short_B2H8N512", True),
    ("C2_headline_B2H8N4096", False), ("C2_headline_B2H8N4096", True),
    ("C3_long_B1H16N16384", True),
    ("C4_many_B32H32N256", True),
]


def _exact_config(causal):
    return capi.config_id("br128_bc64_w4_slot_exact" if causal else "br256_bc64_w8_slot_exact")


@pytest.mark.parametrize("name,causal", CASES)
def test_full_output_error_table(cuda, name, causal):
    w = WORKLOADS[name]
    q, k, v = workload_inputs(w)
    ref = attention_fp32(q, k, v, w.sm_scale, causal)
    floor = error_stats(ref.astype(np.float16).astype(np.float32), ref)
    rows = [("fp16 rounding of the fp32 oracle", floor)]
    variants = (("library choice", -1), ("exact (reference arithmetic)", _exact_config(causal)),
                ("fp32 row sums, fp16 prescaled Q", capi.config_id("br256_bc64_w4_pair")))
    for label, cfg in variants:
        out = run_capi(q, k, v, w.sm_scale, causal, cuda, config=cfg)
        assert np.isfinite(out).all(), label
        stats = error_stats(out, ref)
        rows.append((label, stats))
        assert stats[0] <= MAX_ABS and stats[1] <= MEAN_ABS, (label, stats)
    print()
    for label, (mx, mean) in rows:
        print(f"| {name} | {'causal' if causal else 'non-causal'} | {label} | {mx:.3e} | {mean:.3e} |")
