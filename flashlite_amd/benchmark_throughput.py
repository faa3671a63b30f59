"""Throughput and peak-memory tables of the reference benchmark, on MI355X.

    python -m flashlite_amd.benchmark_throughput [--seq 512 1024 2048 4096]
                                                 [--batch 2] [--heads 8]
                                                 [--json results.json]

Mirrors ``benchmarks/benchmark_throughput.py`` of thebigblender/FlashLite:

* throughput table (``:57-161``), one row per sequence length, for both
  masks: PyTorch SDPA, the official ``flash_attn`` package (reported
  "N/A (not installed)" when absent, as in the reference), this build's
  ``forward_naive`` and this build's ``forward_flash2(..., out=buf)``;
  latency is the median of hip-event pairs around each call
  (``measure_latency_ms``, ``:34-54``: 25 warm-ups and 100 runs; the naive
  kernel 5/20 below N = 2048 and 2/5 above, ``:129-131``), and
  TFLOP/s = FLOPs / latency with FLOPs = 4*B*H*N^2*D, halved when causal
  (``calculate_flops``, ``:23-31``);
* peak-memory table (``:163-202``): ``torch.cuda.max_memory_allocated`` of
  an unfused matmul-softmax-matmul attention (which materialises the
  B*H*N*N scores) against ``forward_flash2`` without ``out``.  Those peaks
  include every live allocation (the inputs, and the BLAS workspace that
  PyTorch keeps after the unfused products), as in the reference; two more
  columns give each call's own growth over what was allocated before it.

The reference pins SDPA to its FlashAttention backend (``:99-103``).  On
ROCm that backend is provided by PyTorch's own kernels for some
architectures only; when it cannot run here the harness falls back to the
memory-efficient backend and then to PyTorch's default choice, and names
the backend it used in every row.  SDPA is a comparator only: nothing in
this package calls it.  Every row also records the largest absolute
difference between SDPA's output and ``forward_flash2``'s, so a fast but
wrong row is visible.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
from typing import Callable, Optional


def calculate_flops(batch_size: int, num_heads: int, seq_len: int, head_dim: int,
                    is_causal: bool = False) -> float:
    """4*B*H*N^2*D for QK^T plus PV, halved for the causal mask
    (``benchmark_throughput.py:23-31``)."""
    multiplier = 2.0 if is_causal else 4.0
    return multiplier * batch_size * num_heads * (seq_len ** 2) * head_dim


def measure_latency_ms(fn: Callable, warmup: int = 25, runs: int = 100) -> float:
    """Median latency in ms of ``fn`` from one event pair per run on the
    current stream (``benchmark_throughput.py:34-54``)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(runs)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(runs)]
    for i in range(runs):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    lat = sorted(s.elapsed_time(e) for s, e in zip(starts, ends))
    return lat[len(lat) // 2]


def _official_flash():
    try:
        from flash_attn import flash_attn_func  # noqa: F401  (third-party, optional)
    except Exception:
        return None
    return flash_attn_func


def _sdpa_runner(q, k, v, is_causal: bool, sm_scale: float):
    """(callable, backend name) for SDPA, trying the reference's FlashAttention
    backend first, then memory-efficient, then PyTorch's default choice."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    def make(backend):
        def run():
            if backend is None:
                return F.scaled_dot_product_attention(q, k, v, dropout_p=0.0, is_causal=is_causal,
                                                      scale=sm_scale)
            with sdpa_kernel([backend]):
                return F.scaled_dot_product_attention(q, k, v, dropout_p=0.0,
                                                      is_causal=is_causal, scale=sm_scale)
        return run

    for backend, name in ((SDPBackend.FLASH_ATTENTION, "flash"),
                          (SDPBackend.EFFICIENT_ATTENTION, "efficient"), (None, "default")):
        fn = make(backend)
        try:
            fn()
            torch.cuda.synchronize()
        except RuntimeError:
            continue
        return fn, name
    return None, "unavailable"


def throughput_rows(batch_size: int = 2, num_heads: int = 8, head_dim: int = 64,
                    seq_lengths=(512, 1024, 2048, 4096), is_causal: bool = False,
                    runs: int = 100, warmup: int = 25, naive: bool = True,
                    log: Optional[Callable[[str], None]] = print):
    """One dict per sequence length: latencies (ms) and TFLOP/s of each
    implementation, as the reference's throughput table."""
    import torch

    import flashlite_amd as fl

    device = torch.device("cuda:0")
    sm_scale = 1.0 / math.sqrt(head_dim)
    official = _official_flash()
    rows = []
    for seq_len in seq_lengths:
        flops = calculate_flops(batch_size, num_heads, seq_len, head_dim, is_causal)
        shape = (batch_size, num_heads, seq_len, head_dim)
        q = torch.randn(shape, dtype=torch.float16, device=device)
        k = torch.randn(shape, dtype=torch.float16, device=device)
        v = torch.randn(shape, dtype=torch.float16, device=device)
        row = {"seq_len": seq_len, "causal": is_causal, "flops": flops}

        sdpa_fn, backend = _sdpa_runner(q, k, v, is_causal, sm_scale)
        row["sdpa_backend"] = backend
        if sdpa_fn is not None:
            row["sdpa_ms"] = measure_latency_ms(sdpa_fn, warmup, runs)
        if official is not None:
            qf, kf, vf = (x.transpose(1, 2).contiguous() for x in (q, k, v))
            try:
                row["official_ms"] = measure_latency_ms(
                    lambda: official(qf, kf, vf, softmax_scale=sm_scale, causal=is_causal),
                    warmup, runs)
            except Exception as exc:  # reported, as the reference does
                row["official_error"] = str(exc)
        if naive:
            n_warm, n_runs = (5, 20) if seq_len <= 1024 else (2, 5)
            row["naive_ms"] = measure_latency_ms(
                lambda: fl.forward_naive(q, k, v, sm_scale, is_causal), n_warm, n_runs)
        out_buf = torch.empty_like(q)
        row["flashlite_ms"] = measure_latency_ms(
            lambda: fl.forward_flash2(q, k, v, sm_scale, is_causal, out=out_buf), warmup, runs)
        if sdpa_fn is not None:
            ref = sdpa_fn()
            fl.forward_flash2(q, k, v, sm_scale, is_causal, out=out_buf)
            torch.cuda.synchronize()
            row["max_abs_vs_sdpa"] = float((ref.float() - out_buf.float()).abs().max())
        for key in ("sdpa", "official", "naive", "flashlite"):
            if key + "_ms" in row:
                row[key + "_tflops"] = flops / (row[key + "_ms"] * 1e-3) / 1e12
        rows.append(row)
        if log is not None:
            log(format_throughput_row(row))
        del q, k, v, out_buf
    return rows


def format_throughput_row(row) -> str:
    def cell(key, width, fmt):
        return f"{row[key]:{width}{fmt}}" if key in row else f"{'N/A':>{width}}"
    return (f"{row['seq_len']:>8} | {cell('sdpa_ms', 17, '.3f')} | {cell('sdpa_tflops', 13, '.2f')} | "
            f"{cell('official_ms', 17, '.3f')} | {cell('official_tflops', 11, '.2f')} | "
            f"{cell('naive_ms', 15, '.3f')} | {cell('naive_tflops', 12, '.2f')} | "
            f"{cell('flashlite_ms', 16, '.3f')} | {cell('flashlite_tflops', 12, '.2f')} | "
            f"{row.get('sdpa_backend', ''):>9} | {cell('max_abs_vs_sdpa', 9, '.2e')}")


THROUGHPUT_HEADER = (
    f"{'SeqLen':>8} | {'PyTorch SDPA (ms)':>17} | {'SDPA TFLOPS':>13} | "
    f"{'Official FA2 (ms)':>17} | {'FA2 TFLOPS':>11} | {'Naive HIP (ms)':>15} | "
    f"{'Naive TFLOPS':>12} | {'FlashLite (ms)':>16} | {'FL TFLOPS':>12} | "
    f"{'SDPA path':>9} | {'FL-SDPA':>9}")


def memory_rows(batch_size: int = 2, num_heads: int = 8, head_dim: int = 64,
                seq_lengths=(512, 1024, 2048, 4096), is_causal: bool = False,
                log: Optional[Callable[[str], None]] = print):
    """Peak allocated MiB of unfused attention and of ``forward_flash2``
    (``benchmark_throughput.py:163-202``)."""
    import torch

    import flashlite_amd as fl

    device = torch.device("cuda:0")
    sm_scale = 1.0 / math.sqrt(head_dim)

    def unfused(qi, ki, vi):
        # The transposed operand is made contiguous before the batched
        # product (a transposed right operand is avoided on this platform).
        scores = torch.matmul(qi, ki.transpose(-2, -1).contiguous()) * sm_scale
        if is_causal:
            n = qi.shape[-2]
            keep = torch.ones(n, n, dtype=torch.bool, device=qi.device).tril()
            scores = scores.masked_fill(~keep, float("-inf"))
        return torch.matmul(torch.softmax(scores, dim=-1), vi)

    rows = []
    for seq_len in seq_lengths:
        shape = (batch_size, num_heads, seq_len, head_dim)
        q = torch.randn(shape, dtype=torch.float16, device=device)
        k = torch.randn(shape, dtype=torch.float16, device=device)
        v = torch.randn(shape, dtype=torch.float16, device=device)
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        _ = unfused(q, k, v)
        torch.cuda.synchronize()
        peak_unfused = torch.cuda.max_memory_allocated()
        del _
        torch.cuda.empty_cache()
        base_flash = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        _ = fl.forward_flash2(q, k, v, sm_scale, is_causal)
        torch.cuda.synchronize()
        peak_flash = torch.cuda.max_memory_allocated()
        del _
        mib = 1024.0 ** 2
        row = {"seq_len": seq_len, "causal": is_causal,
               "unfused_mib": peak_unfused / mib, "flashlite_mib": peak_flash / mib,
               "reduction": peak_unfused / peak_flash if peak_flash > 0 else None,
               "unfused_extra_mib": (peak_unfused - base) / mib,
               "flashlite_extra_mib": (peak_flash - base_flash) / mib}
        rows.append(row)
        if log is not None:
            ratio = f"{row['reduction']:.1f}x" if row["reduction"] else "N/A"
            log(f"{seq_len:>8} | {row['unfused_mib']:>20.2f} MB | {row['flashlite_mib']:>18.2f} MB | "
                f"{ratio:>18} | {row['unfused_extra_mib']:>16.2f} MB | "
                f"{row['flashlite_extra_mib']:>16.2f} MB")
        del q, k, v
    return rows


def run_benchmarks(batch_size: int = 2, num_heads: int = 8, head_dim: int = 64,
                   seq_lengths=(512, 1024, 2048, 4096), is_causal: bool = False,
                   runs: int = 100, warmup: int = 25, naive: bool = True):
    """Prints both tables for one mask; returns their rows."""
    import torch

    if not torch.cuda.is_available():
        print("A GPU is required for the benchmark.")
        return None
    props = torch.cuda.get_device_properties(0)
    arch = getattr(props, "gcnArchName", "")
    print("=" * 150)
    print(" FlashAttention-2 forward throughput (FlashLite on MI355X)")
    print(f" Target Device: {props.name} ({arch})")
    print(f" Config: Batch={batch_size}, Heads={num_heads}, HeadDim={head_dim}, Causal={is_causal}")
    print("=" * 150)
    print(THROUGHPUT_HEADER)
    print("-" * len(THROUGHPUT_HEADER))
    tput = throughput_rows(batch_size, num_heads, head_dim, seq_lengths, is_causal, runs, warmup,
                           naive)
    print("=" * 150)
    print(" - TFLOPS = (FLOPs / (latency_ms * 1e-3)) / 1e12, FLOPs = 4 * B * H * N^2 * D "
          "(halved when causal)")
    print("\n" + "=" * 85)
    print(" Peak Memory Allocation Benchmark (Intermediate Activation Overhead)")
    print("=" * 85)
    print(f"{'SeqLen':>8} | {'Un-fused PyTorch (MB)':>22} | {'FlashLite (MB)':>20} | "
          f"{'Memory Reduction':>18} | {'Un-fused extra':>19} | {'FlashLite extra':>19}")
    print("-" * 130)
    mem = memory_rows(batch_size, num_heads, head_dim, seq_lengths, is_causal)
    print("=" * 85, flush=True)
    return {"throughput": tput, "memory": mem}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--batch", type=int, default=2)
    ap.add_argument("--heads", type=int, default=8)
    ap.add_argument("--seq", type=int, nargs="+", default=[512, 1024, 2048, 4096])
    ap.add_argument("--causal", choices=["both", "0", "1"], default="both")
    ap.add_argument("--runs", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=25)
    ap.add_argument("--no-naive", action="store_true", help="skip the naive kernel")
    ap.add_argument("--json", default=None, help="also write every row to this file")
    args = ap.parse_args(argv)
    masks = {"both": (False, True), "0": (False,), "1": (True,)}[args.causal]
    results = {}
    for causal in masks:
        r = run_benchmarks(args.batch, args.heads, 64, tuple(args.seq), causal, args.runs,
                           args.warmup, not args.no_naive)
        if r is None:
            return 1
        results["causal" if causal else "noncausal"] = r
    if args.json:
        os.makedirs(os.path.dirname(os.path.abspath(args.json)), exist_ok=True)
        with open(args.json, "w") as f:
            json.dump(results, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
