"""The benchmark harness (flashlite_amd/benchmark_throughput.py), the
reference's benchmarks/benchmark_throughput.py restated for MI355X.

CPU: the FLOP formula against values fixed by hand from 4*B*H*N^2*D
(benchmark_throughput.py:23-31) and against the BASELINE workloads.
GPU: one small run of both tables; SDPA's output and forward_flash2's
agree to the parity tolerance, and the fused path allocates far less than
the unfused one."""

import pytest

from flashlite_amd import benchmark_throughput as bt


def test_flops_closed_form():
    # B2 H8 N4096 D64: 4 * 2 * 8 * 4096^2 * 64 = 68,719,476,736
    assert bt.calculate_flops(2, 8, 4096, 64) == 68_719_476_736.0
    assert bt.calculate_flops(2, 8, 4096, 64, is_causal=True) == 34_359_738_368.0
    # B1 H1 N1 D1: one multiply-add per GEMM
    assert bt.calculate_flops(1, 1, 1, 1) == 4.0
    # quadratic in N, linear in B, H and D
    assert bt.calculate_flops(3, 5, 20, 7) == 4.0 * 3 * 5 * 400 * 7


def test_row_format_marks_missing_columns():
    row = {"seq_len": 512, "causal": False, "flops": 1.0, "flashlite_ms": 0.01,
           "flashlite_tflops": 1e-10, "sdpa_backend": "unavailable"}
    text = bt.format_throughput_row(row)
    assert text.split("|")[0].strip() == "512"
    assert text.count("N/A") == 7  # sdpa x2, official x2, naive x2, FL-SDPA
    assert len(text.split("|")) == len(bt.THROUGHPUT_HEADER.split("|"))


@pytest.mark.gpu
@pytest.mark.parametrize("causal", [False, True])
def test_throughput_rows_small(cuda, causal):
    rows = bt.throughput_rows(1, 2, 64, (128, 320), causal, runs=3, warmup=1, log=None)
    assert [r["seq_len"] for r in rows] == [128, 320]
    for r in rows:
        assert r["flashlite_ms"] > 0 and r["naive_ms"] > 0
        assert r["flashlite_tflops"] == pytest.approx(r["flops"] / (r["flashlite_ms"] * 1e-3) / 1e12)
        if r["sdpa_backend"] != "unavailable":
            assert r["sdpa_ms"] > 0
            assert r["max_abs_vs_sdpa"] <= 2e-3, r


@pytest.mark.gpu
def test_memory_rows_fused_is_smaller(cuda):
    rows = bt.memory_rows(1, 4, 64, (1024,), False, log=None)
    r = rows[0]
    # unfused holds the 1*4*1024*1024 fp16 scores (8 MiB) and its softmax;
    # the fused call allocates only its 0.5 MiB output.  (The absolute peaks
    # also hold the inputs and whatever the BLAS library keeps allocated.)
    assert r["unfused_extra_mib"] >= 8.0
    assert 0.5 <= r["flashlite_extra_mib"] < 0.6
    assert r["unfused_mib"] >= r["unfused_extra_mib"]
    assert r["flashlite_mib"] >= r["flashlite_extra_mib"]
