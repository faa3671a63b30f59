"""Regenerates the committed fixtures in this directory.

    python tests/golden/make_golden.py

* ``c0_golden.npz`` -- the CPU plumbing config C0 (B1 H1 N128 D64, seed 0,
  sm_scale 1/8): fp16 q, k, v and the float64 output of the scalar
  brute-force loops (``oracle.attention_bruteforce``) for both masks.
* ``input_hashes.json`` -- sha256 of the fp16 q, k, v bytes of every
  benchmark configuration, from ``flashlite_amd.workloads``.

The reference ships no golden vectors (its tests compare against
torch SDPA at run time, ``tests/test_correctness.py:43-45, 75-77``), so these
are this build's own fixtures.
"""

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from flashlite_amd.workloads import WORKLOADS, digest, workload_inputs  # noqa: E402
from oracle import attention_bruteforce  # noqa: E402


def main():
    w = WORKLOADS["C0_plumbing_B1H1N128"]
    q, k, v = workload_inputs(w)
    o_nc = attention_bruteforce(q, k, v, w.sm_scale, False)
    o_c = attention_bruteforce(q, k, v, w.sm_scale, True)
    np.savez_compressed(os.path.join(HERE, "c0_golden.npz"), q=q, k=k, v=v,
                        out_noncausal=o_nc, out_causal=o_c, sm_scale=np.float64(w.sm_scale))
    hashes = {}
    for name, wl in WORKLOADS.items():
        hashes[name] = {"shape": list(wl.shape), "seed": wl.seed, "input_scale": wl.input_scale,
                        "sha256": digest(*workload_inputs(wl))}
    with open(os.path.join(HERE, "input_hashes.json"), "w") as f:
        json.dump(hashes, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
