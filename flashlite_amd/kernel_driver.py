"""Runs one forward configuration a fixed number of times, for profilers.

    python -m flashlite_amd.kernel_driver --workload C2_headline_B2H8N4096 \
        --causal 0 --config -1 --iters 20

Inputs are the workload's seeded synthetic tensors, resident on the GPU
before the first launch; each launch goes through the C ABI
(``fl_attn_fwd_f16_cfg``, or ``fl_attn_naive_f16`` with ``--naive``) on the
current stream.  Under ``rocprofv3 --kernel-trace --stats`` or ``--pmc`` the
kernel's dispatches are the only ones besides the input uploads.  Prints the
mean launch time measured with HIP events on that stream.

``--copy-mib M`` instead runs an elementwise fp16 kernel that reads M MiB and
writes M MiB (``torch.mul(src, 1, out=dst)``): the reference point that
scales the HBM byte counters (FETCH_SIZE / WRITE_SIZE) of a profile.

``--dtype bf16`` and/or ``--head-dim 128`` run the workload's shape at that
element type / head dim through ``fl_attn_fwd_bf16_ex`` or
``fl_attn_fwd_f16_ex`` (seeded inputs from ``make_qkv`` / ``make_qkv_bf16``;
``--config`` -1 or what the entry point accepts: at head_dim 128 3 or 4, bf16 at
head_dim 64 any configuration but 0 and 1).

``--cold-mib M`` (workloads and ``--decode``) reads and writes an M MiB
buffer before every launch, evicting the inputs from the L2 caches and the
256 MiB Infinity Cache (M > 256), and times each launch alone with its own
HIP event pair; the mean over ``--iters`` launches is printed.

``--timeline MODE`` (MODE 8, 4, 2, 7 or 9: br256_bc64_w8_slot, br128_bc64_w4_slot,
br128_bc64_w4x2_slot, br64_bc64_w2x2_slot or br128_bc64_w4x2_pair; fp16 D = 64 workloads or
``--shape``, ``--causal``)
runs the diagnostic build of the slot kernels whose waves stamp their entry,
loop start and end, and exit (``fl_diag_slot_timeline``), launched
``--iters`` times back to back, and summarises the last launch: launch span,
start skew, prologue / loop / epilogue times, the loop clock per XCD
(s_memtime cycles over s_memrealtime time), and the per-CU work-group
pairing (iterations and loop time of the groups that shared each CU).

``--empty-kernel G W`` times the launch floor the same way: a kernel that
does nothing, G work-groups of W waves (``fl_diag_empty`` in the diagnostic
library), launched back to back through ctypes like the forward calls.

``--shape B H N`` replaces the workload's shape (fp16, D = 64, N_q = N_k = N,
sm_scale 1/8, ``make_qkv`` inputs with seed 1): sweeps over shapes the
workloads do not name.

``--decode B H NQ NK`` runs a decode-shaped call (NQ query rows over NK
keys, seeded N(0,1) inputs) through ``fl_attn_fwd_f16_splitkv`` with
``--splits S`` (1 = one pass, 0 = the library's choice, n = n key chunks;
a one pass runs ``--config``'s configuration, by default the dispatcher's;
``--dtype bf16`` runs one pass only)
and reports the K/V read rate against 8 TB/s: bytes = 2 * B*H*NK*64*2
(K and V once) + Q and O.

``--mfma-clock ROUNDS`` runs the clock calibration of the diagnostic
library (``libflashlite_diag.so``, ``csrc/diag.hip``): every wave issues
ROUNDS x 16 independent ``v_mfma_f32_32x32x16_f16`` (``--groups`` work-groups
of ``--waves`` waves, ``--lds-kib`` of dynamic LDS each, ``--random`` for
random operands).  With one wave per SIMD the matrix core is busy for
ROUNDS * 512 shader cycles per wave, so the HIP-event time gives the clock
the chip sustained; the per-wave ``s_memtime`` / ``s_memrealtime`` deltas
check that ``s_memtime`` counts those cycles.

``--mfma-mix MODE`` with ``--mfma-clock ROUNDS`` runs the issue-rate probe
instead (``fl_diag_mfma_mix``): each of the 16 MFMAs of a round is followed
by a fixed sequence of independent VALU instructions (MODE 0-8, listed in
``csrc/diag.hip``), and the s_memtime cycles per MFMA show what issues under
a running MFMA.
"""

from __future__ import annotations

import argparse
import sys


def main(argv=None):
    ap = argparse.ArgumentParser(description="run one forward configuration repeatedly")
    ap.add_argument("--workload", default="C2_headline_B2H8N4096")
    ap.add_argument("--causal", type=int, default=0)
    ap.add_argument("--config", type=int, default=-1, help="tile configuration (-1 = dispatcher)")
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--naive", action="store_true")
    ap.add_argument("--copy-mib", type=int, default=0, help="run the calibration copy instead")
    ap.add_argument("--decode", type=int, nargs=4, metavar=("B", "H", "NQ", "NK"), default=None)
    ap.add_argument("--splits", type=int, default=0)
    ap.add_argument("--causal-decode", type=int, default=0)
    ap.add_argument("--dtype", choices=("fp16", "bf16"), default="fp16")
    ap.add_argument("--head-dim", type=int, default=0, help="override the workload's head dim")
    ap.add_argument("--shape", type=int, nargs=3, metavar=("B", "H", "N"), default=None)
    ap.add_argument("--mfma-clock", type=int, default=0, metavar="ROUNDS")
    ap.add_argument("--groups", type=int, default=256)
    ap.add_argument("--waves", type=int, default=4)
    ap.add_argument("--lds-kib", type=int, default=96)
    ap.add_argument("--random", type=int, default=1)
    ap.add_argument("--mfma-mix", type=int, default=-1, metavar="MODE")
    ap.add_argument("--cold-mib", type=int, default=0, metavar="M")
    ap.add_argument("--empty-kernel", type=int, nargs=2, metavar=("G", "W"), default=None)
    ap.add_argument("--timeline", type=int, default=0, metavar="MODE")
    ap.add_argument("--stream-timeline", action="store_true",
                    help="per-unit marks of the streaming kernel (N <= 256)")
    ap.add_argument("--quarter-timeline", action="store_true",
                    help="per-wave marks of the key-quarter kernel (N <= 512)")
    args = ap.parse_args(argv)

    import torch

    if args.mfma_clock:
        return _mfma_clock(args, torch)
    if args.empty_kernel:
        return _empty(args, torch)
    if args.timeline:
        return _timeline(args, torch)
    if args.stream_timeline:
        return _stream_timeline(args, torch)
    if args.quarter_timeline:
        return _quarter_timeline(args, torch)
    if args.decode:
        return _decode(args, torch)

    if args.copy_mib:
        n = args.copy_mib * (1 << 20) // 2
        src = torch.ones(n, dtype=torch.float16, device="cuda:0")
        dst = torch.empty_like(src)
        torch.mul(src, 1, out=dst)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.iters):
            torch.mul(src, 1, out=dst)
        end.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(end) * 1e3 / args.iters
        print(f"copy {args.copy_mib} MiB read + {args.copy_mib} MiB write: {us:.2f} us/launch, "
              f"{2 * args.copy_mib * (1 << 20) / us / 1e3:.1f} GB/s", flush=True)
        return 0

    from flashlite_amd import capi
    from flashlite_amd.workloads import WORKLOADS, make_qkv, make_qkv_bf16, workload_inputs

    w = WORKLOADS[args.workload]
    if args.shape:
        from flashlite_amd.workloads import Workload

        b, h, n = args.shape
        w = Workload(f"B{b}H{h}N{n}", b, h, n, 64, (False, True), 1)
    dev = torch.device("cuda:0")
    head_dim = args.head_dim or w.head_dim
    wide = args.dtype == "bf16" or head_dim != 64
    if wide:
        gen = make_qkv_bf16 if args.dtype == "bf16" else make_qkv
        dt = torch.bfloat16 if args.dtype == "bf16" else torch.float16
        q, k, v = (torch.from_numpy(x).to(dev).to(dt)
                   for x in gen(w.batch, w.heads, w.seq, head_dim, w.seed, w.input_scale))
    else:
        q, k, v = (torch.from_numpy(x).to(dev) for x in workload_inputs(w))
    o = torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream
    if wide:
        p = capi.tensor_params_ex(q, k, v, o, w.sm_scale, bool(args.causal))
        fwd_ex = capi.fwd_bf16_ex if args.dtype == "bf16" else capi.fwd_ex
        cfg = args.config
    else:
        p = capi.tensor_params(q, k, v, o, w.sm_scale, bool(args.causal))
        cfg = capi.select_config(p) if args.config < 0 else args.config

    def launch():
        if wide:
            rc = fwd_ex(p, stream, cfg)
        else:
            rc = capi.naive(p, stream) if args.naive else capi.fwd(p, stream, cfg)
        capi.check(rc)

    us = _time_launches(launch, args, torch)
    flops = (2.0 if args.causal else 4.0) * w.batch * w.heads * w.seq ** 2 * head_dim
    nbytes = 4 * w.batch * w.heads * w.seq * head_dim * q.element_size()
    name = "naive" if args.naive else ("auto" if cfg < 0 else capi.config_name(cfg))
    print(f"{w.name} {args.dtype} D={head_dim} causal={args.causal} {name}"
          f"{' cold' if args.cold_mib else ''}: {us:.2f} us/launch, "
          f"{flops / us / 1e6:.1f} TFLOP/s, {nbytes / us / 1e3:.1f} GB/s", flush=True)


def _decode(args, torch):
    import numpy as np

    from flashlite_amd import capi

    b, h, nq, nk = args.decode
    bf16 = args.dtype == "bf16"
    if bf16 and args.splits != 1:
        raise SystemExit("--decode with --dtype bf16 runs one pass only (--splits 1)")
    dev = torch.device("cuda:0")
    rs = np.random.RandomState(7)
    dt = torch.bfloat16 if bf16 else torch.float16
    mk = lambda n: torch.from_numpy(  # noqa: E731
        rs.standard_normal((b, h, n, 64)).astype(np.float32)).to(dev).to(dt)
    q, k, v = mk(nq), mk(nk), mk(nk)
    o = torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream
    p = capi.tensor_params_ex(q, k, v, o, 0.125, bool(args.causal_decode))
    need = 0 if args.splits == 1 else capi.splitkv_workspace_bytes(p, args.splits)
    ws = torch.empty(max(need, 16) // 4, dtype=torch.float32, device=dev)

    # one pass (no chunks): the dispatcher's configuration, or --config's
    cfg = args.config if need == 0 else -1

    def launch():
        if need == 0:
            capi.check((capi.fwd_bf16_ex if bf16 else capi.fwd_ex)(p, stream, cfg))
        else:
            capi.check(capi.fwd_splitkv(p, ws.data_ptr(), need, stream, args.splits))

    us = _time_launches(launch, args, torch)
    nbytes = 2 * b * h * nk * 64 * 2 + 2 * b * h * nq * 64 * 2
    chunks = need // (b * h * nq * 68 * 4) if need else 1
    name = f" {capi.config_name(cfg)}" if need == 0 and cfg >= 0 else ""
    print(f"decode B{b} H{h} NQ{nq} NK{nk}{' bf16' if bf16 else ''} causal={args.causal_decode} "
          f"chunks={chunks}{name}"
          f"{' cold' if args.cold_mib else ''}: "
          f"{us:.2f} us/call, {nbytes / us / 1e3:.1f} GB/s ({nbytes / us / 1e3 / 8000:.1%} of 8 TB/s)",
          flush=True)
    return 0


def _time_launches(launch, args, torch):
    """Mean microseconds per launch: one warm-up, then ``args.iters``
    launches between two events (warm), or, with ``--cold-mib``, each launch
    between its own event pair after a pass over the eviction buffer."""
    launch()
    torch.cuda.synchronize()
    if not args.cold_mib:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.iters):
            launch()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1e3 / args.iters
    flush = torch.zeros(args.cold_mib * (1 << 20) // 4, dtype=torch.float32, device="cuda:0")
    pairs = []
    for _ in range(args.iters):
        flush.add_(1.0)
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        launch()
        e.record()
        pairs.append((s, e))
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in pairs) * 1e3 / len(pairs)


def _diag_lib():
    import ctypes
    import os

    return ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                    "libflashlite_diag.so"))


def _empty(args, torch):
    import ctypes

    lib = _diag_lib()
    lib.fl_diag_empty.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.fl_diag_empty.restype = ctypes.c_int
    groups, waves = args.empty_kernel
    stream = torch.cuda.current_stream().cuda_stream

    def launch():
        rc = lib.fl_diag_empty(groups, waves, stream)
        if rc != 0:
            raise RuntimeError(f"diagnostic launch failed: hipError {rc}")

    us = _time_launches(launch, args, torch)
    print(f"empty kernel {groups} groups x {waves} waves{' cold' if args.cold_mib else ''}: "
          f"{us:.2f} us/launch", flush=True)
    return 0


def _timeline(args, torch):
    import collections
    import ctypes

    import numpy as np

    from flashlite_amd.workloads import WORKLOADS, Workload, workload_inputs

    w = WORKLOADS[args.workload]
    if args.shape:
        b, h, n = args.shape
        w = Workload(f"B{b}H{h}N{n}", b, h, n, 64, (False, True), 1)
    if w.head_dim != 64:
        raise SystemExit("--timeline runs fp16 at head_dim 64")
    lib = _diag_lib()
    lib.fl_diag_slot_timeline.argtypes = ([ctypes.c_int] * 2 + [ctypes.c_void_p] * 4 +
                                          [ctypes.c_int] * 3 + [ctypes.c_void_p, ctypes.c_longlong,
                                                                ctypes.c_void_p])
    lib.fl_diag_slot_timeline.restype = ctypes.c_int
    lib.fl_diag_wall_clock_khz.argtypes = [ctypes.c_int]
    lib.fl_diag_wall_clock_khz.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    q, k, v = (torch.from_numpy(x).to(dev) for x in workload_inputs(w))
    o = torch.empty_like(q)
    mode = args.timeline
    rows, wpg = {8: (256, 8), 4: (128, 4), 7: (64, 4)}.get(mode, (128, 8))
    blocks = (w.seq + rows - 1) // rows
    groups = w.batch * w.heads * blocks
    if mode == 9:  # one group per block pair, one record per wave and block
        groups, wpg = w.batch * w.heads * ((blocks + 1) // 2), 16
    out = torch.zeros(groups * wpg * 8, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def launch():
        rc = lib.fl_diag_slot_timeline(mode, args.causal, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                       o.data_ptr(), w.batch, w.heads, w.seq, out.data_ptr(),
                                       out.numel(), stream)
        if rc != 0:
            raise RuntimeError(f"diagnostic launch failed: hipError {rc}")

    us = _time_launches(launch, args, torch)
    d = out.cpu().numpy().reshape(-1, 8).astype(np.int64)
    blk = (np.arange(len(d)) % wpg) // 8 if mode == 9 else np.zeros(len(d), np.int64)
    keep = d[:, 7] != 0  # every wave (and block) that stamped
    d, blk = d[keep], blk[keep]
    tick_us = 1e3 / lib.fl_diag_wall_clock_khz(0)
    t = (d[:, :6] - d[:, 0].min()) * tick_us
    iters = d[:, 7] >> 48
    xcc = (d[:, 7] >> 32) & 0xFF
    hw = d[:, 7] & 0xFFFFFFFF
    loop = t[:, 3] - t[:, 2]
    clk = d[:, 6] / np.maximum(loop, 1e-9) / 1e3  # GHz
    names = {8: "br256_bc64_w8_slot", 4: "br128_bc64_w4_slot", 2: "br128_bc64_w4x2_slot",
             7: "br64_bc64_w2x2_slot", 9: "br128_bc64_w4x2_pair"}
    print(f"timeline {w.name} causal={args.causal} {names[mode]}: {us:.2f} us/launch over "
          f"{args.iters} launches (events); last launch: {len(d)} wave records, span "
          f"{t[:, 5].max():.2f} us (first entry to last exit), start skew {t[:, 0].max():.2f} us",
          flush=True)
    pct = lambda x: (f"min {x.min():7.2f}  p50 {np.median(x):7.2f}  p90 "  # noqa: E731
                     f"{np.percentile(x, 90):7.2f}  max {x.max():7.2f} us")
    for b in sorted(set(blk.tolist())):
        m = blk == b
        if mode == 9:
            print(f"  block {b} of each pair ({'the heavier, first' if b == 0 else 'the lighter'}; "
                  f"times from {'the group entry' if b == 0 else 'its own start'}):")
        print(f"  entry -> loop start (prologue)  {pct(t[m, 2] - t[m, 0])}")
        print(f"  loop                            {pct(loop[m])}")
        print(f"  loop end -> exit (epilogue)     {pct(t[m, 5] - t[m, 3])}")
        it = iters[m]
        print(f"  iterations p50 {np.median(it):.0f} (min {it.min()}, max {it.max()}); loop time "
              f"per iteration p50 {np.median(loop[m] / it) * 1e3:.0f} ns")
    print(f"  loop cycles per iteration p50 {np.median(d[:, 6] / iters):.0f}; loop clock "
          f"min {clk.min():.3f} p50 {np.median(clk):.3f} max {clk.max():.3f} GHz")
    for x in range(8):
        m = xcc == x
        if m.any():
            print(f"  XCD {x}: {m.sum():4d} waves, exits {t[m, 5].min():6.2f}-{t[m, 5].max():6.2f} us, "
                  f"loop p50 {np.median(loop[m]):6.2f} us at {np.median(clk[m]):.3f} GHz")
    # work-groups per CU (XCC_ID; SE, SH and CU ids, HW_ID bits 8-15) and their loop work
    cu_key = xcc * 256 + ((hw >> 8) & 0xFF)
    if len(d) % wpg == 0:
        per_cu = collections.defaultdict(list)
        for g in range(len(d) // wpg):
            sl = slice(g * wpg, (g + 1) * wpg)
            bs = [blk[sl] == b for b in sorted(set(blk[sl].tolist()))]  # a pair's two blocks
            per_cu[cu_key[sl][0]].append((int(sum(iters[sl][m].max() for m in bs)),
                                          float(sum(loop[sl][m].max() for m in bs)),
                                          float(t[sl, 5].max())))
        ends = np.array([max(x[2] for x in v) for v in per_cu.values()])
        print(f"  {len(per_cu)} CUs; CU finish min {ends.min():.2f} p50 {np.median(ends):.2f} "
              f"max {ends.max():.2f} us")
        for key in sorted(per_cu, key=lambda c: -max(x[2] for x in per_cu[c]))[:3]:
            print("  latest CU: " + ", ".join(f"{n} it / loop {lt:.1f} us / exit {e:.1f} us"
                                              for n, lt, e in sorted(per_cu[key])))
    return 0


def _stream_timeline(args, torch):
    """Where the streaming kernel's time goes: per unit of each work-group,
    the wait at its barrier (its loads landing), the issue of the next
    unit's loads and its compute."""
    import ctypes

    import numpy as np

    from flashlite_amd.workloads import WORKLOADS, Workload, workload_inputs

    w = WORKLOADS[args.workload]
    if args.shape:
        b, h, n = args.shape
        w = Workload(f"B{b}H{h}N{n}", b, h, n, 64, (False, True), 1)
    lib = _diag_lib()
    lib.fl_diag_stream_timeline.argtypes = ([ctypes.c_int] + [ctypes.c_void_p] * 4 +
                                            [ctypes.c_int] * 3 +
                                            [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p])
    lib.fl_diag_stream_timeline.restype = ctypes.c_int
    lib.fl_diag_wall_clock_khz.argtypes = [ctypes.c_int]
    lib.fl_diag_wall_clock_khz.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    q, k, v = (torch.from_numpy(x).to(dev) for x in workload_inputs(w))
    o = torch.empty_like(q)
    groups = min(w.batch * w.heads * ((w.seq + 255) // 256), 256)
    out = torch.zeros(groups * 8 * 64, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def launch():
        rc = lib.fl_diag_stream_timeline(args.causal, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                         o.data_ptr(), w.batch, w.heads, w.seq, out.data_ptr(),
                                         out.numel(), stream)
        if rc != 0:
            raise RuntimeError(f"diagnostic launch failed: hipError {rc}")

    us = _time_launches(launch, args, torch)
    d = out.cpu().numpy().reshape(groups, 8, 64).astype(np.int64)
    tick_us = 1e3 / lib.fl_diag_wall_clock_khz(0)
    t = (d - d[:, :, 0].min()) * tick_us
    units = (np.count_nonzero(d[0, 0, 1:63]) - 1) // 3 + 1 if d[0, 0, 1] else 0
    pct = lambda x: (f"p50 {np.median(x):6.2f}  p90 {np.percentile(x, 90):6.2f}  "  # noqa: E731
                     f"max {x.max():6.2f} us")
    print(f"stream timeline {w.name} causal={args.causal}: {us:.2f} us/launch over {args.iters} "
          f"launches (events); last launch: {groups} groups x 8 waves, {units} units each, span "
          f"{t[:, :, 63].max():.2f} us", flush=True)
    print(f"  entry -> first unit's loads landed  {pct(t[:, :, 1] - t[:, :, 0])}")
    for i in range(units):
        start = t[:, :, 1 + 3 * i].max(axis=1)  # barrier passed (all waves)
        issued = t[:, :, 2 + 3 * i].max(axis=1)
        stored = t[:, :, 3 + 3 * i].max(axis=1)
        line = f"  unit {i}: starts {pct(start)}; issue {pct(issued - start)}; compute {pct(stored - issued)}"
        if i > 0:
            prev = t[:, :, 3 * i].max(axis=1)
            line += f"; wait for loads {pct(start - prev)}"
        print(line)
    print(f"  last stores issued -> exit  {pct(t[:, :, 63].max(axis=1) - t[:, :, 3 * units].max(axis=1))}")
    return 0


def _quarter_timeline(args, torch):
    """Where the key-quarter kernel's time goes: per wave, its loads' issue
    and landing, its two tiles, the merge with its chunk's stores, and the
    wait for them to land."""
    import ctypes

    import numpy as np

    from flashlite_amd.workloads import WORKLOADS, Workload, workload_inputs

    w = WORKLOADS[args.workload]
    if args.shape:
        b, h, n = args.shape
        w = Workload(f"B{b}H{h}N{n}", b, h, n, 64, (False, True), 1)
    lib = _diag_lib()
    lib.fl_diag_quarter_timeline.argtypes = ([ctypes.c_int] + [ctypes.c_void_p] * 4 +
                                             [ctypes.c_int] * 3 +
                                             [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p])
    lib.fl_diag_quarter_timeline.restype = ctypes.c_int
    lib.fl_diag_wall_clock_khz.argtypes = [ctypes.c_int]
    lib.fl_diag_wall_clock_khz.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    q, k, v = (torch.from_numpy(x).to(dev) for x in workload_inputs(w))
    o = torch.empty_like(q)
    groups = w.batch * w.heads * ((w.seq + 31) // 32)
    out = torch.zeros(groups * 8 * 64, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def launch():
        rc = lib.fl_diag_quarter_timeline(args.causal, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                          o.data_ptr(), w.batch, w.heads, w.seq, out.data_ptr(),
                                          out.numel(), stream)
        if rc != 0:
            raise RuntimeError(f"diagnostic launch failed: hipError {rc}")

    us = _time_launches(launch, args, torch)
    d = out.cpu().numpy().reshape(groups, 8, 64)[:, :4, :].astype(np.int64)
    tick_us = 1e3 / lib.fl_diag_wall_clock_khz(0)
    t = (d - d[:, :, 0].min()) * tick_us
    pct = lambda x: (f"p50 {np.median(x):6.2f}  p90 {np.percentile(x, 90):6.2f}  "  # noqa: E731
                     f"max {x.max():6.2f} us")
    print(f"quarter timeline {w.name} causal={args.causal}: {us:.2f} us/launch over {args.iters} "
          f"launches (events); last launch: {groups} groups x 4 waves, span "
          f"{t[:, :, 63].max():.2f} us", flush=True)
    busy = d[:, :, 2] != 0  # waves with key tiles
    print(f"  entry (after the first)          {pct(t[:, :, 0].ravel())}")
    print(f"  entry -> loads issued, Q loaded  {pct((t[:, :, 1] - t[:, :, 0]).ravel())}")
    print(f"  -> loads landed                  {pct((t[:, :, 2] - t[:, :, 1])[busy])}")
    print(f"  -> tiles done                    {pct((t[:, :, 3] - t[:, :, 2])[busy])}")
    print(f"  -> merged, own chunk's stores issued {pct((t[:, :, 4] - t[:, :, 3]).ravel())}")
    print(f"  -> exit (stores landed)          {pct((t[:, :, 63] - t[:, :, 4]).ravel())}")
    print(f"  group span (first entry -> last exit) "
          f"{pct(t[:, :, 63].max(axis=1) - t[:, :, 0].min(axis=1))}")
    return 0


def _mfma_clock(args, torch):
    import ctypes

    import numpy as np

    lib = _diag_lib()
    lib.fl_diag_mfma_clock.argtypes = [ctypes.c_int] * 5 + [ctypes.c_void_p] * 3
    lib.fl_diag_mfma_clock.restype = ctypes.c_int
    lib.fl_diag_mfma_mix.argtypes = [ctypes.c_int] * 5 + [ctypes.c_void_p] * 3
    lib.fl_diag_mfma_mix.restype = ctypes.c_int
    lib.fl_diag_wall_clock_khz.argtypes = [ctypes.c_int]
    lib.fl_diag_wall_clock_khz.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    nwaves = args.groups * args.waves
    out = torch.zeros(2 * nwaves, dtype=torch.int64, device=dev)
    sink = torch.empty(nwaves * 64, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def launch():
        if args.mfma_mix >= 0:
            rc = lib.fl_diag_mfma_mix(args.groups, args.waves, args.mfma_clock, args.mfma_mix,
                                      args.lds_kib * 1024, out.data_ptr(), sink.data_ptr(), stream)
        else:
            rc = lib.fl_diag_mfma_clock(args.groups, args.waves, args.mfma_clock, args.random,
                                        args.lds_kib * 1024, out.data_ptr(), sink.data_ptr(),
                                        stream)
        if rc != 0:
            raise RuntimeError(f"diagnostic launch failed: hipError {rc}")

    launch()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.iters):
        launch()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / args.iters
    d = out.cpu().numpy().reshape(-1, 2).astype(np.float64)
    khz = lib.fl_diag_wall_clock_khz(0)
    cyc, real = d[:, 0], d[:, 1]
    clk = cyc / (real / (khz * 1e3)) / 1e9
    known = args.mfma_clock * 16 * 32
    flops = nwaves * args.mfma_clock * 16 * 32768
    if args.mfma_mix >= 0:
        per_simd = max(1, args.waves // 4)
        print(f"mfma mix mode {args.mfma_mix}: {args.groups} groups x {args.waves} waves "
              f"({per_simd}/SIMD), rounds {args.mfma_clock}: {us:.2f} us/launch; s_memtime cycles "
              f"per MFMA per SIMD median {np.median(cyc) / (args.mfma_clock * 16 * per_simd):.2f} "
              f"(min {cyc.min() / (args.mfma_clock * 16 * per_simd):.2f}); clock "
              f"{np.median(clk):.3f} GHz", flush=True)
        return 0
    print(f"mfma clock: {args.groups} groups x {args.waves} waves, {args.lds_kib} KiB LDS, "
          f"rounds {args.mfma_clock}, random {args.random}: {us:.2f} us/launch, "
          f"{flops / us / 1e6:.1f} TFLOP/s; known MFMA cycles per wave {known}; "
          f"s_memtime per wave min/median/max {cyc.min():.0f}/{np.median(cyc):.0f}/{cyc.max():.0f} "
          f"(median/known {np.median(cyc) / known:.4f}); s_memrealtime rate {khz} kHz; "
          f"s_memtime/s_memrealtime clock min/median/max {clk.min():.3f}/{np.median(clk):.3f}/"
          f"{clk.max():.3f} GHz; known cycles / event time {known / us / 1e3:.3f} GHz",
          flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
