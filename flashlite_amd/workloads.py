"""Synthetic workloads of the benchmark configurations and their inputs.

The configurations are the ones the reference benchmarks and tests run at
(``benchmarks/benchmark_throughput.py:205-222``: B=2, H=8, D=64,
N in {512, 1024, 2048, 4096}, both masks, sm_scale = 1/8) plus two stress
shapes: a very long causal sequence and many small heads reused through the
``out=`` buffer.

Inputs: the reference draws them with the CUDA Philox stream
(``tests/test_correctness.py:20-26``) or unseeded
(``benchmark_throughput.py:94-96``); neither can be reproduced on a CPU.
Here one ``numpy.random.RandomState(seed)`` draws q, k, v in that order as
float64 standard normals, optionally scaled, cast to float32 and then to
float16.  numpy keeps that legacy stream frozen, so the same fp16 bytes come
out on every machine; their sha256 digests are committed as test fixtures.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    heads: int
    seq: int
    head_dim: int
    causal: tuple          # masks the config is run with
    seed: int
    input_scale: float = 1.0
    sm_scale: float = 0.125
    reuse_out: bool = False  # timed through forward_flash2(..., out=buf)

    @property
    def shape(self):
        return (self.batch, self.heads, self.seq, self.head_dim)


WORKLOADS = {
    "C0_plumbing_B1H1N128": Workload("C0_plumbing_B1H1N128", 1, 1, 128, 64, (False, True), 0),
    "C1_short_B2H8N512": Workload("C1_short_B2H8N512", 2, 8, 512, 64, (False, True), 1),
    "C2_headline_B2H8N4096": Workload("C2_headline_B2H8N4096", 2, 8, 4096, 64, (False, True), 2),
    "sweep_B2H8N1024": Workload("sweep_B2H8N1024", 2, 8, 1024, 64, (False, True), 3),
    "sweep_B2H8N2048": Workload("sweep_B2H8N2048", 2, 8, 2048, 64, (False, True), 4),
    "C3_long_B1H16N16384": Workload("C3_long_B1H16N16384", 1, 16, 16384, 64, (True,), 5,
                                    input_scale=0.5),
    "C4_many_B32H32N256": Workload("C4_many_B32H32N256", 32, 32, 256, 64, (True,), 6,
                                   reuse_out=True),
}

HEADLINE = "C2_headline_B2H8N4096"


def make_qkv(batch: int, heads: int, seq: int, head_dim: int, seed: int = 0,
             scale: float = 1.0):
    """Seeded fp16 Q, K, V (numpy, [B, H, N, D], contiguous)."""
    rs = np.random.RandomState(seed)
    shape = (batch, heads, seq, head_dim)
    out = []
    for _ in range(3):
        x = rs.standard_normal(size=shape)
        if scale != 1.0:
            x = x * scale
        out.append(np.ascontiguousarray(x.astype(np.float32).astype(np.float16)))
    return tuple(out)


def round_bf16(x) -> np.ndarray:
    """float32 array -> the nearest bfloat16 values (round to nearest, ties to
    even), returned as float32.  bf16 is the upper half of an IEEE float32,
    so rounding adds half an ulp of the dropped 16 bits (minus one when the
    kept low bit is 0, which sends ties to even) and clears them.  NaN and
    inf are not expected here (inputs are finite normals)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def make_qkv_bf16(batch: int, heads: int, seq: int, head_dim: int, seed: int = 0,
                  scale: float = 1.0):
    """Seeded bf16-valued Q, K, V: the make_qkv draws rounded to bfloat16,
    held in float32 arrays (numpy has no bfloat16; every value is exactly
    representable, so ``torch.from_numpy(x).to(torch.bfloat16)`` is exact)."""
    rs = np.random.RandomState(seed)
    shape = (batch, heads, seq, head_dim)
    out = []
    for _ in range(3):
        x = rs.standard_normal(size=shape)
        if scale != 1.0:
            x = x * scale
        out.append(round_bf16(x.astype(np.float32)))
    return tuple(out)


def workload_inputs(w: Workload):
    return make_qkv(w.batch, w.heads, w.seq, w.head_dim, w.seed, w.input_scale)


def digest(q, k, v) -> str:
    """sha256 over the fp16 bytes of q, k and v in that order."""
    h = hashlib.sha256()
    for x in (q, k, v):
        h.update(np.ascontiguousarray(x).tobytes())
    return h.hexdigest()
