"""Benchmark of the MI355X fused residual-add + RMSNorm + group-quant operator.

Default workload: the headline configuration (BASELINE.json metric),
16384 x 7168 bf16 -> fp8 e4m3fn, group 128, fp32 column-major scales, 1 %
outlier channels.  A "step" is one call of the operator over the whole
[16384, 7168] batch.  Inputs are resident in HBM before the timed region; K
steps are timed between device synchronisations, rotating over enough
input/output sets that no step reads data left in L2/MALL by the previous
one.

Prints one JSON line.  One timing underlies value, ms_per_step, pct_of_peak
and roofline: one HIP event pair recorded on the launch stream around the K
timed back-to-back steps (the host clock over the same region is reported as
us_per_call_host_wall).
  value       whole-job achieved bandwidth: algorithmic bytes / (event time / K)
  roofline    the same figure against 8 TB/s; traffic = measured HBM bytes per
              launch from the committed rocprofv3 counter summary for this
              workload (null if none)
  us_per_call_graph_replay  device time per call of consecutive launches
              captured in a HIP graph (workloads under 64 MB only)
  cpu_baseline  the eager-PyTorch CPU restatement timed on a bounded row sample
              of the same workload on this host's CPU share (and checked against
              the GPU's rows); cpu_baseline_config1 = BASELINE config 1
              (128 x 4096) in full, with the GPU's output checked against it

--config f16_* / bf16_r32_*: the typed form (fp16 tensors; fp32 residual stream).
--config ref4_*: the reference operator's own output mode: norm_out written
(4 outputs), int8 codes by truncation, fp32 row-major scales.

--config tp*_shard_*: the multi-input form (fagq_launch_parts) at one rank's
shard of a tensor-parallel layer: nparts partial sums reduced, normalized and
quantized (fp8, fp32 column-major scales); cpu_baseline = the C oracle.

--config dsa_*: the Task 02 DSA top-k page-table transform
(fagq_dsa_topk_launch); value = algorithmic GB/s (valid score prefixes read
once, outputs and page gathers), also rows/s; cpu_baseline = the C oracle.

--config gemm_*: the fp8 block-scaled GEMM that consumes the operator's
output (fagq_gemm_launch); value and roofline in TFLOP/s against MI355X's
5.0 PFLOP/s dense fp8 peak, cpu_baseline = the C oracle (oracle/gemm_oracle.c)
on a row sample.

--copy BYTES and --mfma-peak time the ceiling probes instead (libfagq_probe.so,
include/fagq_probe.h, not part of the drop-in library): HBM
copy, read-only and write-only streams with the operator's cache policies
(achievable bandwidth, counter calibration), and the GEMM's matrix instruction
issued from registers (achievable MFMA rate).  --lds-probe times the LDS read
patterns of fagq_diag_lds_read (run it under rocprofv3 --pmc for the bank
conflicts of each).  For a quantizer config, --rows-sweep times it over row
counts and --route-sweep under each explicit launch mapping (fagq_launch_mapped)
against the route table's choice.

Usage: python bench.py [--steps K] [--warmup W] [--config NAME] [--gpus 1]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

REPO_DIR = Path(__file__).resolve().parent
PEAK_HBM_GBS = 8000.0
PEAK_FP8_TFLOPS = 5000.0   # MI355X dense fp8 MFMA
METRIC = "achieved HBM GB/s (% of 8 TB/s peak) + µs/call, 16384×7168 bf16→fp8 g128"
ROTATE_BYTES = 1 << 30     # rotate buffer sets until > 1 GiB (4x the 256 MB MALL)


def measured_traffic(name: str):
    """HBM bytes per launch (per call for multi-kernel operators) from the committed
    profiles/traffic_<name>.json, measured with rocprofv3 FETCH_SIZE / WRITE_SIZE runs and
    calibrated against a copy kernel; None when no such file exists."""
    tfile = REPO_DIR / "profiles" / f"traffic_{name}.json"
    if not tfile.exists():
        return None
    try:
        return json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
    except (ValueError, OSError):
        return None


def timed_region(torch, dev, stream, step, steps: int):
    """The timed region: K steps between device synchronisations, bracketed by one
    HIP event pair recorded on the launch stream and by the host clock.  Returns
    (device ms per step from the events, host wall ms per step).  Nothing but the
    launches runs between the events, so back-to-back kernels are measured as the
    stream executes them."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize(dev)
    t1 = time.perf_counter()
    return e0.elapsed_time(e1) / steps, (t1 - t0) * 1e3 / steps


def heat(torch, dev, step, ms: float) -> None:
    """Runs step back to back for ms milliseconds (synchronising every 64 calls)."""
    t_end = time.perf_counter() + ms * 1e-3
    i = 0
    while time.perf_counter() < t_end:
        step(i)
        i += 1
        if i % 64 == 0:
            torch.cuda.synchronize(dev)
    torch.cuda.synchronize(dev)


def steady_region(args, torch, dev, stream, step):
    """Device ms per step of K more steps after --steady-ms of load (None when
    disabled).  Reported beside value, never as it: the device's clocks settle
    over the first tens of milliseconds of load, which a short warm-up does not
    cover."""
    if args.steady_ms <= 0:
        return None
    heat(torch, dev, step, args.steady_ms)
    return timed_region(torch, dev, stream, step, args.steps)[0]


def steady_fields(steady_ms, nbytes):
    if steady_ms is None:
        return {"us_per_call_steady_state": None, "steady_state_pct_of_peak": None}
    return {"us_per_call_steady_state": round(steady_ms * 1e3, 2),
            "steady_state_pct_of_peak": round(100.0 * nbytes / (steady_ms * 1e-3) / 1e9 /
                                              PEAK_HBM_GBS, 2)}


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads() -> int:
    """Threads for the CPU baseline: the CPUs this process may run on, capped by
    OMP_NUM_THREADS when it is set (a GPU box gives each GPU's jobs a 16-CPU share and
    sets OMP_NUM_THREADS to it; nproc there counts the whole host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


def host_info(threads: int) -> dict:
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = None
    return {"cpu_model": cpu_model(), "nproc": os.cpu_count(), "affinity_cpus": aff,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "threads_used": threads}


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--config", default=None, help="workload name (default: the headline one)")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="target CPU time of the cpu_baseline leg (0 disables it)")
    p.add_argument("--cpu-rows", type=int, default=512, help="rows in the cpu_baseline sample")
    p.add_argument("--copy", type=int, default=0, metavar="BYTES",
                   help="instead: time the library's HBM copy / read / write probes over BYTES "
                        "(achievable bandwidth, HBM counter calibration)")
    p.add_argument("--mfma-peak", action="store_true",
                   help="instead: time the library's register-only issue-rate probe of the fp8 "
                        "GEMM's matrix instruction (the compute ceiling its rate is compared with)")
    p.add_argument("--lds-probe", action="store_true",
                   help="instead: time the library's LDS read probe for each address pattern")
    p.add_argument("--steady-ms", type=float, default=300.0,
                   help="after the timed region: run the operator this long, then time K more "
                        "steps (us_per_call_steady_state; 0 disables)")
    p.add_argument("--rows-sweep", default="",
                   help="instead: comma-separated row counts; the config's operator at each, after "
                        "a warm-up of the device, with a least-squares line of time against bytes")
    p.add_argument("--route-sweep", action="store_true",
                   help="instead: the config's operator under each explicit launch mapping "
                        "(fagq_launch_mapped), against the route table's own choice")
    return p.parse_args()


def copy_bench(args, torch, pkg) -> int:
    """Times the library's HBM ceiling probes (fagq_diag_stream) over BYTES, with the
    operator's cache policies: copy (BYTES read + BYTES written), read-only,
    write-only, and the operator's byte mix without its arithmetic (two input
    streams of BYTES/2 read, residual_out and one-byte codes written: 3.5 x BYTES/2
    moved), buffer sets rotated past the MALL, one event pair around the K launches
    of each.  One JSON line per probe."""
    import ctypes
    from fagq_mi355x import _lib
    dev = torch.device("cuda:0")
    lib = pkg.load_probe_library()
    n = args.copy // 16 * 16
    nsets = max(2, math.ceil(ROTATE_BYTES / (2 * n)) + 1)
    bufs = [(torch.empty(n, dtype=torch.uint8, device=dev).fill_(1),
             torch.empty(n, dtype=torch.uint8, device=dev)) for _ in range(nsets)]
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    # opmix: the operator's byte mix (x, residual in; residual_out, one-byte codes out)
    # over n/2 bytes per input stream, carved from the same buffers.
    nop = n // 2 // 32 * 32
    for mode, name, moved, nb in ((_lib.STREAM_COPY, "copy", 2 * n, n),
                                  (_lib.STREAM_READ, "read", n, n),
                                  (_lib.STREAM_WRITE, "write", n, n),
                                  (_lib.STREAM_OPMIX, "opmix", 7 * nop // 2, nop)):
        def step(i, mode=mode, nb=nb):
            s, d = bufs[i % nsets]
            pkg._lib.check(lib.fagq_diag_stream(ctypes.c_void_p(s.data_ptr()),
                                                ctypes.c_void_p(d.data_ptr()), nb, mode, sp),
                           "fagq_diag_stream")

        for i in range(args.warmup):
            step(i)
        ms, _ = timed_region(torch, dev, stream, step, args.steps)
        print(json.dumps({"probe": name, "bytes_per_launch": moved, "buffer_bytes": nb,
                          "us_per_call": round(ms * 1e3, 2),
                          "GBps": round(moved / (ms * 1e-3) / 1e9, 1),
                          "frac_of_8000": round(moved / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                          "buffer_sets": nsets, "steps": args.steps}), flush=True)
    return 0


def mfma_peak_bench(args, torch, pkg) -> int:
    """Times fagq_diag_mfma_rate for both fp8 instruction shapes: 2048 workgroups of
    4 waves, each wave issuing 1000 x 8 v_mfma_scale_f32_16x16x128_f8f6f4 (8
    accumulators) or 1000 x 4 v_mfma_scale_f32_32x32x64_f8f6f4 (4 accumulators) on
    register operands, the same flops per launch.  One JSON line per shape."""
    import ctypes
    dev = torch.device("cuda:0")
    lib = pkg.load_probe_library()
    blocks, iters = 2048, 1000
    out = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    for shape, name, flops in ((0, "v_mfma_scale_f32_16x16x128_f8f6f4", blocks * 4 * iters * 8 * 65536),
                               (1, "v_mfma_scale_f32_32x32x64_f8f6f4", blocks * 4 * iters * 4 * 131072)):
        def step(shape=shape):
            pkg._lib.check(lib.fagq_diag_mfma_rate(ctypes.c_void_p(out.data_ptr()), blocks, iters,
                                                   shape, sp), "fagq_diag_mfma_rate")

        for _ in range(args.warmup):
            step()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(dev)
        e0.record(stream)
        for _ in range(args.steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize(dev)
        ms = e0.elapsed_time(e1) / args.steps
        tflops = flops / (ms * 1e-3) / 1e12
        print(json.dumps({"instruction": name, "flops_per_call": flops,
                          "us_per_call": round(ms * 1e3, 2), "TFLOPs": round(tflops, 1),
                          "frac_of_5000_TFLOPs": round(tflops / 5000.0, 4),
                          "steps": args.steps, "warmup": args.warmup}), flush=True)
    return 0


def lds_probe_bench(args, torch, pkg) -> int:
    """Times fagq_diag_lds_read for each address pattern (1024 workgroups of 4 waves,
    8 x 256 ds_read_b128 per wave), one launch per pattern and step, in pattern order,
    so a rocprofv3 counter run sees the patterns as consecutive dispatches.  One JSON
    line per pattern."""
    import ctypes
    dev = torch.device("cuda:0")
    lib = pkg.load_probe_library()
    blocks, iters = 1024, 256
    out = torch.empty(blocks * 256 * 4, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    names = ["lane order", "GEMM fragment, low half", "GEMM fragment, high half",
             "fragment, chunk c ^ ((r / 2) % 8)", "fragment, chunk c ^ (r % 8)",
             "fragment, no swizzle"]
    for pattern, name in enumerate(names):
        def step(pattern=pattern):
            pkg._lib.check(lib.fagq_diag_lds_read(ctypes.c_void_p(out.data_ptr()), blocks, iters,
                                                  pattern, sp), "fagq_diag_lds_read")

        for _ in range(args.warmup):
            step()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(dev)
        e0.record(stream)
        for _ in range(args.steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize(dev)
        ms = e0.elapsed_time(e1) / args.steps
        print(json.dumps({"probe": "fagq_diag_lds_read", "pattern": pattern, "name": name,
                          "ds_read_b128_per_call": blocks * 4 * iters * 8,
                          "us_per_call": round(ms * 1e3, 2),
                          "steps": args.steps, "warmup": args.warmup}), flush=True)
    return 0


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(rows shard with no exchange: one process per GPU runs its own row block)",
              file=sys.stderr)
        return 2
    sys.path.insert(0, str(REPO_DIR))
    import torch
    import __graft_entry__ as ge

    pkg = ge.load_package()
    from fagq_mi355x.workloads import CONFIGS, HEADLINE, make_inputs

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    if args.copy:
        return copy_bench(args, torch, pkg)
    if args.mfma_peak:
        return mfma_peak_bench(args, torch, pkg)
    if args.lds_probe:
        return lds_probe_bench(args, torch, pkg)
    name = args.config or HEADLINE
    from fagq_mi355x.workloads import DSA_CONFIGS, GEMM_CONFIGS, MLA_CONFIGS, PARTS_CONFIGS
    if name in DSA_CONFIGS:
        return dsa_bench(args, torch, pkg, DSA_CONFIGS[name])
    if name in MLA_CONFIGS:
        return mla_bench(args, torch, pkg, MLA_CONFIGS[name])
    if name in GEMM_CONFIGS:
        return gemm_bench(args, torch, pkg, GEMM_CONFIGS[name])
    if name in PARTS_CONFIGS:
        return parts_bench(args, torch, pkg, PARTS_CONFIGS[name])
    from fagq_mi355x.workloads import REFERENCE_MODE_CONFIGS, TYPED_CONFIGS
    w = {**CONFIGS, **TYPED_CONFIGS, **REFERENCE_MODE_CONFIGS}[name]
    if args.rows_sweep:
        return rows_sweep(args, torch, pkg, w)
    if args.route_sweep:
        return route_sweep(args, torch, pkg, w)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = pkg.load_library()

    x, res, gamma = make_inputs(w)
    set_bytes = w.algorithmic_bytes()
    nsets = max(2, math.ceil(ROTATE_BYTES / set_bytes) + 1)
    nsets = min(nsets, 64)
    xd, rd, gd = x.to(dev), res.to(dev), gamma.to(dev)
    sets = []
    for i in range(nsets):
        xs, rs = (xd, rd) if i == 0 else (xd.clone(), rd.clone())
        ro = torch.empty_like(rs)
        q = torch.empty((w.M, w.D), dtype=w.out_dtype, device=dev)
        sc = pkg.empty_scales(w.M, w.groups, ue8m0=w.scale_ue8m0, col_major=w.scale_col_major,
                              device=dev)
        no = torch.empty_like(xs) if w.norm else None
        sets.append((xs, rs, ro, q, sc, no))

    def step(i: int):
        xs, rs, ro, q, sc, no = sets[i % nsets]
        pkg.fused_add_rmsnorm_group_quant(
            xs, rs, gd, ro, no, q, sc, w.eps, w.group_size,
            rounding=w.rounding if w.out_dtype == torch.int8 else None)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)

    # Timed region: K back-to-back steps; device time from one HIP event pair on the
    # launch stream, host wall time over the same region.
    kern_ms, wall_ms = timed_region(torch, dev, stream, step, args.steps)

    steady_ms = steady_region(args, torch, dev, stream, step)

    # Device time per call without host launch gaps: a HIP graph of
    # consecutive launches, replayed (matters when a call is shorter than its
    # Python + launch overhead, i.e. decode-sized batches).
    graph_us = None
    if set_bytes < (64 << 20):
        per_graph = min(64, args.steps)
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            step(0)                                  # warm the side stream
            torch.cuda.synchronize(dev)
            with torch.cuda.graph(g, stream=side):
                for i in range(per_graph):
                    step(i)
        torch.cuda.synchronize(dev)
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize(dev)
        ge0, ge1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        ge0.record(stream)
        for _ in range(reps):
            g.replay()
        ge1.record(stream)
        torch.cuda.synchronize(dev)
        graph_us = ge0.elapsed_time(ge1) * 1e3 / (reps * per_graph)

    value = set_bytes / (kern_ms * 1e-3) / 1e9

    traffic = measured_traffic(name)

    route = pkg.route_for(w.M, w.D, w.group_size, scale_ue8m0=w.scale_ue8m0,
                          scale_col_major=w.scale_col_major, x_dtype=w.act, residual_dtype=w.res)
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(kern_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "timing": "value, ms_per_step, pct_of_peak and roofline.achieved all come from one "
                  "HIP event pair on the launch stream around the K timed steps",
        "config": {"workload": name, "M": w.M, "D": w.D, "group_size": w.group_size,
                   "q": str(w.out_dtype).replace("torch.", ""),
                   "scale": ("ue8m0" if w.scale_ue8m0 else "f32") +
                            (" col-major" if w.scale_col_major else " row-major"),
                   "inputs": w.dist, "x_dtype": str(w.act).replace("torch.", ""),
                   "residual_dtype": str(w.res).replace("torch.", ""),
                   "algorithmic_bytes": set_bytes, "buffer_sets": nsets,
                   "route": route},
        "us_per_call": round(kern_ms * 1e3, 2),
        "us_per_call_host_wall": round(wall_ms * 1e3, 2),
        "us_per_call_graph_replay": None if graph_us is None else round(graph_us, 2),
        **steady_fields(steady_ms, set_bytes),
        "pct_of_peak": round(100.0 * value / PEAK_HBM_GBS, 2),
        "rows_per_s": round(w.M / (kern_ms * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(value / PEAK_HBM_GBS, 4),
                     "traffic": traffic},
        "cpu_baseline": None,
    }

    if args.cpu_seconds > 0:
        out["cpu_baseline"] = cpu_baseline(w, x, res, gamma, sets[0], args, torch)
        if name != CPU_CONFIG:
            out["cpu_baseline_config1"] = cpu_config1(pkg, dev, args, torch)
    print(json.dumps(out), flush=True)
    return 0


CPU_CONFIG = "cpu_ref_128x4096"   # the CPU PyTorch reference path


def rows_sweep(args, torch, pkg, w0) -> int:
    """The config's operator at each row count of --rows-sweep (same D, formats
    and distribution), in one process: 300 ms of warm-up on the largest size,
    then, in 5 interleaved rounds, K steps per size timed by one event pair
    (buffer sets rotated past the MALL); median per size.  One JSON line per
    size, then a least-squares line t = t0 + bytes / bw over the sizes whose
    time is above 4 x the smallest (the launch-bound sizes excluded)."""
    import dataclasses
    from fagq_mi355x.workloads import make_inputs
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    sizes = sorted(int(v) for v in args.rows_sweep.split(","))
    runs = []
    for M in sizes:
        w = dataclasses.replace(w0, name=f"{w0.name}@M={M}", M=M)
        x, res, gamma = make_inputs(w)
        nb = w.algorithmic_bytes()
        nsets = max(2, min(64, math.ceil(ROTATE_BYTES / nb) + 1))
        xd, rd, gd = x.to(dev), res.to(dev), gamma.to(dev)
        sets = []
        for i in range(nsets):
            xs, rs = (xd, rd) if i == 0 else (xd.clone(), rd.clone())
            sets.append((xs, rs, torch.empty_like(rs),
                         torch.empty((M, w.D), dtype=w.out_dtype, device=dev),
                         pkg.empty_scales(M, w.groups, ue8m0=w.scale_ue8m0,
                                          col_major=w.scale_col_major, device=dev),
                         torch.empty_like(xs) if w.norm else None))

        def step(i, sets=sets, w=w):
            xs, rs, ro, q, sc, no = sets[i % len(sets)]
            pkg.fused_add_rmsnorm_group_quant(
                xs, rs, gd, ro, no, q, sc, w.eps, w.group_size,
                rounding=w.rounding if w.out_dtype == torch.int8 else None)
        runs.append((M, nb, step, sets, gd))
    heat(torch, dev, runs[-1][2], 300.0)
    times = {M: [] for M, *_ in runs}
    for _ in range(5):
        for M, nb, step, *_ in runs:
            times[M].append(timed_region(torch, dev, stream, step, args.steps)[0])
    pts = []
    for M, nb, *_ in runs:
        t = sorted(times[M])[2] * 1e3
        pts.append((M, nb, t))
        print(json.dumps({"workload": w0.name, "M": M, "D": w0.D, "algorithmic_bytes": nb,
                          "us_per_call_median": round(t, 2),
                          "GBps": round(nb / (t * 1e-6) / 1e9, 1),
                          "pct_of_peak": round(100.0 * nb / (t * 1e-6) / 1e9 / PEAK_HBM_GBS, 2)}),
              flush=True)
    tmin = min(t for _, _, t in pts)
    fit = [(nb, t) for _, nb, t in pts if t > 4 * tmin]
    if len(fit) >= 2:
        n = len(fit)
        mx = sum(b for b, _ in fit) / n
        my = sum(t for _, t in fit) / n
        slope = sum((b - mx) * (t - my) for b, t in fit) / sum((b - mx) ** 2 for b, _ in fit)
        print(json.dumps({"fit": "t = t0 + bytes / bw", "points": n,
                          "t0_us": round(my - slope * mx, 2),
                          "bw_GBps": round(1.0 / slope / 1e3, 1)}), flush=True)
    return 0


def route_sweep(args, torch, pkg, w) -> int:
    """The config's operator under explicit launch mappings (fagq_launch_mapped,
    include/fagq_diag.h; every mapping gives the same bits), in one process: for
    1-4 steps of 512 columns per wave, the waves per row that gives, times 1, 2
    or 4 rows per workgroup (at most 16 waves) and each row-group mode that
    applies, with the route's own XCD order and LDS reservation.  300 ms of
    warm-up, then 3 interleaved rounds of K steps per mapping, one event pair
    each; median.  One JSON line per mapping, fastest first; `route` marks the
    route table's own choice (fagq_query_route), timed the same way."""
    import ctypes
    from fagq_mi355x import _lib
    from fagq_mi355x.workloads import make_inputs
    if w.act != torch.bfloat16 or w.res != torch.bfloat16:
        print("bench.py: --route-sweep times fagq_launch_mapped, which takes bf16 tensors only",
              file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    lib = pkg.load_library()
    x, res, gamma = make_inputs(w)
    nb = w.algorithmic_bytes()
    nsets = max(2, min(64, math.ceil(ROTATE_BYTES / nb) + 1))
    xd, rd, gd = x.to(dev), res.to(dev), gamma.to(dev)
    sets = []
    for i in range(nsets):
        xs, rs = (xd, rd) if i == 0 else (xd.clone(), rd.clone())
        sets.append((xs, rs, torch.empty_like(rs), torch.empty((w.M, w.D), dtype=w.out_dtype, device=dev),
                     pkg.empty_scales(w.M, w.groups, ue8m0=w.scale_ue8m0, col_major=w.scale_col_major,
                                      device=dev),
                     torch.empty_like(xs) if w.norm else None))
    qf = _lib.Q_INT8 if w.out_dtype == torch.int8 else _lib.Q_FP8_E4M3FN
    sf = _lib.SCALE_UE8M0 if w.scale_ue8m0 else _lib.SCALE_F32
    lay = _lib.LAYOUT_COL_MAJOR if w.scale_col_major else _lib.LAYOUT_ROW_MAJOR
    rnd = _lib.ROUND_TRUNC if (w.out_dtype == torch.int8 and w.rounding == "trunc") else _lib.ROUND_RNE
    route = pkg.route_for(w.M, w.D, w.group_size, scale_ue8m0=w.scale_ue8m0,
                          scale_col_major=w.scale_col_major)
    remap, lds = route["xcd_remap"], route["lds_bytes"]
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(stream.cuda_stream)

    def stepper(wpr, rpb, mode):
        def step(i):
            xs, rs, ro, q, sc, no = sets[i % nsets]
            e = lib.fagq_launch_mapped(P(xs), P(rs), P(gd), P(ro), None if no is None else P(no),
                                       P(q), P(sc), w.M, w.D,
                                       w.group_size, w.eps, qf, sf, lay, rnd, wpr, rpb, mode,
                                       remap, lds, st)
            if e:
                raise RuntimeError(f"fagq_launch_mapped: status {e}")
        return step

    def route_step(i):
        xs, rs, ro, q, sc, no = sets[i % nsets]
        pkg.fused_add_rmsnorm_group_quant(xs, rs, gd, ro, no, q, sc, w.eps, w.group_size,
                                          rounding=w.rounding if w.out_dtype == torch.int8 else None)

    steps_total = -(-w.D // 512)
    cands = [("route", route["waves_per_row"], route["rows_per_block"], route["row_group_mode"],
              route_step)]
    for ns in (1, 2, 3, 4):
        wpr = -(-steps_total // ns)
        if wpr > 16 or (ns > 1 and -(-steps_total // (ns - 1)) == wpr):
            continue
        for rpb in (1, 2, 4):
            if wpr * rpb > 16:
                continue
            for mode in (0, 1, 2):
                if mode >= 1 and wpr * ns > 16:
                    continue
                if mode == 2 and (not w.scale_col_major or rpb == 1):
                    continue
                step = stepper(wpr, rpb, mode)
                try:
                    step(0)
                except RuntimeError:
                    continue
                cands.append(("mapped", wpr, rpb, mode, step))
    torch.cuda.synchronize(dev)
    heat(torch, dev, route_step, 300.0)
    times = [[] for _ in cands]
    for _ in range(3):
        for k, c in enumerate(cands):
            times[k].append(timed_region(torch, dev, stream, c[4], args.steps)[0])
    rows = []
    for (kind, wpr, rpb, mode, _), ts in zip(cands, times):
        t = sorted(ts)[1] * 1e3
        rows.append({"workload": w.name, "route": kind == "route", "waves_per_row": wpr,
                     "steps_per_wave": -(-steps_total // wpr), "rows_per_block": rpb,
                     "row_group_mode": mode, "xcd_remap": remap, "lds_bytes": lds,
                     "us_per_call_median": round(t, 2),
                     "pct_of_peak": round(100.0 * nb / (t * 1e-6) / 1e9 / PEAK_HBM_GBS, 2)})
    for r in sorted(rows, key=lambda r: r["us_per_call_median"]):
        print(json.dumps(r), flush=True)
    return 0


def _time_cpu(run, min_runs: int, seconds: float, max_runs: int = 1000):
    """Median seconds per call over at least min_runs calls (after 2 warm-ups),
    continuing for up to `seconds`."""
    run()
    run()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < seconds and len(times) < max_runs):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def _gpu_rows_parity(w, gpu_set, ref, rows, torch):
    import numpy as np
    from oracle.compare import compare
    _, _, ro, q, sc, no = gpu_set
    torch.cuda.synchronize()
    scale_rows = sc[:rows]
    scale_phys = scale_rows.t() if w.scale_col_major else scale_rows
    gpu = {"residual_out": ro[:rows].cpu().view(torch.uint16).numpy(),
           "q": q[:rows].cpu().view(torch.uint8).numpy(),
           "scale": np.ascontiguousarray(scale_phys.cpu().numpy())}
    refd = {"residual_out": ref[0].view(torch.uint16).numpy(),
            "q": ref[1].view(torch.uint8).numpy(), "scale": ref[2].numpy()}
    if no is not None:
        gpu["norm_out"] = no[:rows].cpu().view(torch.uint16).numpy()
        refd["norm_out"] = ref[3].view(torch.uint16).numpy()
    try:
        st = compare(gpu, refd, fp8=w.out_dtype == torch.float8_e4m3fn, ue8m0=w.scale_ue8m0)
        return {"ok": True, "exact": st["exact"], "q_mismatch": st["q_mismatch"]}
    except AssertionError as e:
        return {"ok": False, "error": str(e)[:200]}


def cpu_baseline(w, x, res, gamma, gpu_set, args, torch) -> dict:
    """Times the eager-PyTorch CPU restatement (oracle/torch_eager.py) on the
    first rows of the same workload, on this host's CPU share, and checks those
    rows of the GPU's output against it."""
    from oracle.torch_eager import fagq_torch

    threads = cpu_threads()
    torch.set_num_threads(threads)
    rows = max(1, min(args.cpu_rows, w.M))
    xs, rs = x[:rows].contiguous(), res[:rows].contiguous()

    def run():
        return fagq_torch(xs, rs, gamma, w.eps, w.group_size, w.out_dtype, w.scale_ue8m0,
                          w.scale_col_major, w.rounding, with_norm=w.norm)

    ref = run()
    t, n = _time_cpu(run, 3, args.cpu_seconds)
    nbytes = w.algorithmic_bytes() * rows // w.M
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "us_per_call": round(t * 1e6, 1),
            "sample": f"first {rows} of {w.M} rows of {w.name}, eager PyTorch CPU "
                      f"restatement (oracle/torch_eager.py), {threads} threads, median of {n} runs",
            "host": host_info(threads),
            "parity_vs_gpu_rows": _gpu_rows_parity(w, gpu_set, ref, rows, torch)}


def cpu_config1(pkg, dev, args, torch) -> dict:
    """BASELINE config 1 in full (128 x 4096 -> fp8, fp32 row-major scales): the
    eager-PyTorch CPU path timed on this host's CPU share (median of >= 10 runs
    after 2 warm-ups), and the GPU operator's output on the same inputs checked
    against it."""
    from fagq_mi355x.workloads import CONFIGS, make_inputs
    from oracle.torch_eager import fagq_torch
    w = CONFIGS[CPU_CONFIG]
    threads = cpu_threads()
    torch.set_num_threads(threads)
    x, res, gamma = make_inputs(w)

    def run():
        return fagq_torch(x, res, gamma, w.eps, w.group_size, w.out_dtype, w.scale_ue8m0,
                          w.scale_col_major, w.rounding)

    ref = run()
    t, n = _time_cpu(run, 10, min(args.cpu_seconds, 5.0))
    xd, rd, gd = x.to(dev), res.to(dev), gamma.to(dev)
    ro = torch.empty_like(rd)
    q = torch.empty((w.M, w.D), dtype=w.out_dtype, device=dev)
    sc = pkg.empty_scales(w.M, w.groups, device=dev)
    pkg.fused_add_rmsnorm_group_quant(xd, rd, gd, ro, None, q, sc, w.eps, w.group_size)
    nbytes = w.algorithmic_bytes()
    return {"workload": w.name, "value": round(nbytes / t / 1e9, 3), "unit": "GB/s",
            "us_per_call": round(t * 1e6, 1), "cores": threads, "kind": "port",
            "sample": f"all {w.M} rows, eager PyTorch CPU restatement (oracle/torch_eager.py), "
                      f"{threads} threads, median of {n} runs",
            "host": host_info(threads),
            "parity_vs_gpu": _gpu_rows_parity(w, (xd, rd, ro, q, sc, None), ref, w.M, torch)}


def parts_bench(args, torch, pkg, w) -> int:
    """Times fagq_launch_parts on a shard workload (inputs resident in HBM,
    buffer sets rotated past the MALL), kernel time by HIP events."""
    import ctypes
    from fagq_mi355x import _lib
    from fagq_mi355x.workloads import make_parts_inputs
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _lib.load()
    parts, res, gamma = make_parts_inputs(w)
    set_bytes = w.algorithmic_bytes()
    nsets = max(2, min(16, math.ceil(ROTATE_BYTES / set_bytes) + 1))
    gd = gamma.to(dev)
    pd0 = [p.to(dev) for p in parts]
    rd0 = res.to(dev)
    sets = []
    for i in range(nsets):
        pd = pd0 if i == 0 else [p.clone() for p in pd0]
        rd = rd0 if i == 0 else rd0.clone()
        ro = torch.empty_like(rd)
        q = torch.empty(w.M, w.D, dtype=torch.float8_e4m3fn, device=dev)
        sc = pkg.empty_scales(w.M, w.D // w.group_size, col_major=True, device=dev)
        arr = (ctypes.c_void_p * w.nparts)(*[t.data_ptr() for t in pd])
        sets.append((pd, arr, rd, ro, q, sc))
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())

    def step(i: int):
        _, arr, rd, ro, q, sc = sets[i % nsets]
        st = lib.fagq_launch_parts(ctypes.cast(arr, ctypes.c_void_p), w.nparts, P(rd), P(gd),
                                   P(ro), P(q), P(sc), w.M, w.D, w.group_size, 1e-6,
                                   _lib.Q_FP8_E4M3FN, _lib.SCALE_F32, _lib.LAYOUT_COL_MAJOR,
                                   _lib.ROUND_RNE, sp)
        if st:
            _lib.check(st, "fagq_launch_parts")

    for i in range(args.warmup):
        step(i)
    kern_ms, wall_ms = timed_region(torch, dev, stream, step, args.steps)
    steady_ms = steady_region(args, torch, dev, stream, step)
    value = set_bytes / (kern_ms * 1e-3) / 1e9
    achieved = value
    out = {
        "metric": "achieved HBM GB/s (% of 8 TB/s), multi-input form at one rank's shard",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(kern_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": w.name, "M": w.M, "D": w.D, "nparts": w.nparts,
                   "group_size": w.group_size, "q": "float8_e4m3fn", "scale": "f32 col-major",
                   "algorithmic_bytes": set_bytes, "buffer_sets": nsets,
                   "route": _lib.query_route_parts(w.M, w.D, w.group_size, w.nparts,
                                                   _lib.SCALE_F32, _lib.LAYOUT_COL_MAJOR)},
        "us_per_call": round(kern_ms * 1e3, 2),
        "us_per_call_host_wall": round(wall_ms * 1e3, 2),
        **steady_fields(steady_ms, set_bytes),
        "pct_of_peak": round(100.0 * achieved / PEAK_HBM_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": measured_traffic(w.name)},
        "cpu_baseline": None,
    }
    if args.cpu_seconds > 0:
        out["cpu_baseline"] = parts_cpu_baseline(w, parts, res, gamma, sets[0], args, torch)
    print(json.dumps(out), flush=True)
    return 0


def parts_cpu_baseline(w, parts, res, gamma, gpu_set, args, torch) -> dict:
    """Times the C oracle (oracle.fagq_parts, OpenMP) on the first rows of the
    shard and checks those rows of the GPU's output against it."""
    import numpy as np
    import oracle
    from oracle.compare import compare
    threads = cpu_threads()
    rows = max(1, min(args.cpu_rows, w.M))
    u16 = lambda t: t[:rows].contiguous().view(torch.uint16).numpy()
    pr = [u16(p) for p in parts]
    rr, gg = u16(res), gamma.contiguous().view(torch.uint16).numpy()

    def run():
        return oracle.fagq_parts(pr, rr, gg, 1e-6, w.group_size, oracle.Q_FP8, oracle.S_F32,
                                 oracle.L_COL, oracle.R_RNE, nthreads=threads)

    ref = run()
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < args.cpu_seconds and len(times) < 1000):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    times.sort()
    t = times[len(times) // 2]
    _, _, _, ro, q, sc = gpu_set
    torch.cuda.synchronize()
    gpu = {"residual_out": ro[:rows].cpu().view(torch.uint16).numpy(),
           "q": q[:rows].cpu().view(torch.uint8).numpy(),
           "scale": np.ascontiguousarray(sc[:rows].t().cpu().numpy())}
    try:
        st = compare(gpu, ref, fp8=True, ue8m0=False)
        parity = {"ok": True, "exact": st["exact"], "q_mismatch": st["q_mismatch"]}
    except AssertionError as e:
        parity = {"ok": False, "error": str(e)[:200]}
    nbytes = w.algorithmic_bytes() * rows // w.M
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_call": round(t * 1e6, 1),
            "sample": f"first {rows} of {w.M} rows of {w.name}, C oracle (oracle.fagq_parts, "
                      f"OpenMP), median of {len(times)} runs",
            "parity_vs_gpu_rows": parity}


def dsa_bench(args, torch, pkg, w) -> int:
    """Times fagq_dsa_topk_launch (inputs resident in HBM, sets rotated past the
    MALL), kernel time by HIP events on the launch stream."""
    import ctypes
    from fagq_mi355x import _lib
    from fagq_mi355x.workloads import dsa_valid_blocks, make_dsa_inputs
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _lib.load()
    scores, pt, pos, kv = make_dsa_inputs(w)
    nbytes = w.algorithmic_bytes(dsa_valid_blocks(w, pos, kv))
    full = scores.numel() * scores.element_size()
    nsets = max(2, min(16, math.ceil(ROTATE_BYTES / full) + 1))
    s0, pt_d, pos_d, kv_d = scores.to(dev), pt.to(dev), pos.to(dev), kv.to(dev)
    sets = []
    for i in range(nsets):
        s = s0 if i == 0 else s0.clone()
        ob = torch.empty(w.B, w.H, w.Q, w.top_k, dtype=torch.int32, device=dev)
        sets.append((s, ob, torch.empty_like(ob)))
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    sdt = 1 if w.dtype == torch.bfloat16 else 0

    def step(i: int):
        s, ob, op = sets[i % nsets]
        st = lib.fagq_dsa_topk_launch(P(s), sdt, P(pt_d), P(pos_d), P(kv_d), 0, P(ob), P(op),
                                      w.B, w.H, w.Q, w.NB, w.block_size, w.top_k, sp)
        if st:
            _lib.check(st, "fagq_dsa_topk_launch")

    for i in range(args.warmup):
        step(i)
    kern_ms, wall_ms = timed_region(torch, dev, stream, step, args.steps)
    steady_ms = steady_region(args, torch, dev, stream, step)
    value = nbytes / (kern_ms * 1e-3) / 1e9
    achieved = value
    out = {
        "metric": "DSA top-k page-table transform: algorithmic GB/s (% of 8 TB/s) + us/call",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(kern_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if w.dtype == torch.float32 else "bf16 (compared as f32)",
        "data": "synthetic",
        "config": {"workload": w.name, "B": w.B, "H": w.H, "Q": w.Q, "NB": w.NB,
                   "top_k": w.top_k, "block_size": w.block_size, "rows": w.rows,
                   "algorithmic_bytes": nbytes, "buffer_sets": nsets},
        "us_per_call": round(kern_ms * 1e3, 2),
        "us_per_call_host_wall": round(wall_ms * 1e3, 2),
        **steady_fields(steady_ms, nbytes),
        "rows_per_s": round(w.rows / (kern_ms * 1e-3), 1),
        "pct_of_peak": round(100.0 * achieved / PEAK_HBM_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": measured_traffic(w.name)},
        "cpu_baseline": None,
    }
    if args.cpu_seconds > 0:
        out["cpu_baseline"] = dsa_cpu_baseline(w, scores, pt, pos, kv, sets[0], nbytes, args, torch)
    print(json.dumps(out), flush=True)
    return 0


def mla_bench(args, torch, pkg, w) -> int:
    """Times fagq_mla_bwd_launch (Task 03; three kernels per call) with inputs
    resident in HBM, do / dq / dc sets rotated past the MALL; per-call time by
    HIP events on the launch stream."""
    import ctypes
    from fagq_mi355x import _lib
    from fagq_mi355x.workloads import make_mla_inputs
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _lib.load()
    q, c, out, do0, lse = make_mla_inputs(w, device=dev)
    nbytes = w.algorithmic_bytes()
    set_bytes = do0.numel() * 2 + do0.numel() * (2 if w.grad_dtype == torch.bfloat16 else 4)
    nsets = max(1, min(16, math.ceil(ROTATE_BYTES / set_bytes) + 1)) if set_bytes < ROTATE_BYTES else 1
    ws_bytes = lib.fagq_mla_bwd_workspace_bytes(w.B, w.S, w.D)
    sets = []
    for i in range(nsets):
        d = do0 if i == 0 else do0.clone()
        sets.append((d, torch.empty(w.B, w.H, w.S, w.D, dtype=w.grad_dtype, device=dev),
                     torch.empty(w.B, w.S, w.D, dtype=w.grad_dtype, device=dev),
                     torch.empty(ws_bytes, dtype=torch.uint8, device=dev)))
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    gcode = 1 if w.grad_dtype == torch.bfloat16 else 0

    def step(i: int):
        d, dq, dc, ws = sets[i % nsets]
        st = lib.fagq_mla_bwd_launch(P(q), P(c), P(out), P(d), P(lse), P(dq), P(dc), P(ws), ws_bytes,
                                     w.B, w.H, w.S, w.D, w.sm_scale, gcode, gcode, sp)
        if st:
            _lib.check(st, "fagq_mla_bwd_launch")

    for i in range(args.warmup):
        step(i)
    kern_ms, wall_ms = timed_region(torch, dev, stream, step, args.steps)
    steady_ms = steady_region(args, torch, dev, stream, step)
    value = nbytes / (kern_ms * 1e-3) / 1e9
    achieved = value
    out_json = {
        "metric": "MLA backward (Task 03) dQ+dC: algorithmic GB/s (% of 8 TB/s) + us/call",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(kern_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 in, fp32 accumulate, " + ("bf16" if gcode else "fp32") + " gradients",
        "data": "synthetic",
        "config": {"workload": w.name, "B": w.B, "H": w.H, "S": w.S, "D": w.D,
                   "sm_scale": w.sm_scale, "algorithmic_bytes": nbytes, "buffer_sets": nsets},
        "us_per_call": round(kern_ms * 1e3, 2),
        "us_per_call_host_wall": round(wall_ms * 1e3, 2),
        **steady_fields(steady_ms, nbytes),
        "pct_of_peak": round(100.0 * achieved / PEAK_HBM_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": measured_traffic(w.name)},
        "cpu_baseline": None,
    }
    if args.cpu_seconds > 0:
        out_json["cpu_baseline"] = mla_cpu_baseline(w, q, c, out, do0, lse, pkg, args, torch)
    print(json.dumps(out_json), flush=True)
    return 0


def mla_cpu_baseline(w, q, c, out, do, lse, pkg, args, torch) -> dict:
    """Times the C oracle on batch 0, heads 0..7 (all S rows) and checks the GPU
    operator on the same sample against it (rows >= 16 of dq bit-exact)."""
    import dataclasses
    import numpy as np
    import oracle
    threads = cpu_threads()
    hs = min(8, w.H)
    sw = dataclasses.replace(w, B=1, H=hs)
    sq, sc, so, sd, sl = (q[:1, :hs].contiguous(), c[:1].contiguous(), out[:1, :hs].contiguous(),
                          do[:1, :hs].contiguous(), lse[:1, :hs].contiguous())
    bits = lambda t: t.cpu().view(torch.uint16).numpy()
    aq, ac, ao, ad, al = bits(sq), bits(sc), bits(so), bits(sd), sl.cpu().numpy()

    def run():
        return oracle.mla_bwd(aq, ac, ao, ad, al, w.sm_scale, with_bound=False, nthreads=threads)

    rdq, rdc, _ = run()
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < args.cpu_seconds and len(times) < 100):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    times.sort()
    t = times[len(times) // 2]
    gq = torch.empty_like(sq, dtype=w.grad_dtype)
    gc = torch.empty_like(sc, dtype=w.grad_dtype)
    pkg.mla_bwd_nope_dkdv(sq, sc, so, sd, sl, gq, gc, w.sm_scale)
    torch.cuda.synchronize()
    E = sw.exact_rows
    want = torch.from_numpy(rdq[:, :, E:].astype(np.float32)).to(w.grad_dtype)
    ok = bool(torch.equal(gq[:, :, E:].cpu(), want))
    dc_err = float(np.abs(gc.float().cpu().numpy() - rdc).max() / max(np.abs(rdc).max(), 1e-30))
    return {"value": round(sw.algorithmic_bytes() / t / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "us_per_call": round(t * 1e6, 1),
            "sample": f"batch 0, heads 0..{hs - 1} of {w.name} (B=1, H={hs}, S={w.S}, D={w.D}), "
                      f"C oracle (OpenMP), median of {len(times)} runs; GB/s of that sample's "
                      f"algorithmic bytes",
            "parity_vs_gpu_sample": {"dq_rows_past_prefix_bit_exact": ok,
                                     "dc_max_rel_err": dc_err}}


def dsa_cpu_baseline(w, scores, pt, pos, kv, gpu_set, nbytes, args, torch) -> dict:
    """Times the C oracle on the rows of the first (b, h) head block and
    checks those GPU rows against it."""
    import numpy as np
    import oracle
    threads = cpu_threads()
    rows = min(w.Q, w.rows)
    sub = scores[:1, :1]
    s_np = sub.contiguous().view(torch.uint16).numpy() if w.dtype == torch.bfloat16 else \
        sub.contiguous().numpy()
    pt_np, pos_np, kv_np = pt[:1].numpy(), pos[:1].numpy(), kv[:1].numpy()

    def run():
        return oracle.dsa_topk(s_np, pt_np, pos_np, kv_np, w.block_size, w.top_k, nthreads=threads)

    rb, rp = run()
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < args.cpu_seconds and len(times) < 1000):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    times.sort()
    t = times[len(times) // 2]
    _, ob, op = gpu_set
    torch.cuda.synchronize()
    ok = bool(np.array_equal(ob[:1, :1].cpu().numpy(), rb) and np.array_equal(op[:1, :1].cpu().numpy(), rp))
    sample_bytes = nbytes * rows / w.rows
    return {"value": round(sample_bytes / t / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "us_per_call": round(t * 1e6, 1),
            "sample": f"the {rows} query rows of head (0, 0) of {w.name} ({rows} of {w.rows} rows), "
                      f"C oracle (OpenMP), median of {len(times)} runs; GB/s scaled by the rows' "
                      f"share of the algorithmic bytes",
            "parity_vs_gpu_rows": {"ok": ok}}


def gemm_bench(args, torch, pkg, w) -> int:
    """Times fagq_gemm_launch on a GEMM workload (inputs resident in HBM, sets
    rotated past the MALL), kernel time by HIP events on the launch stream."""
    from fagq_mi355x.workloads import make_gemm_inputs
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    a_q, a_s, b_q, b_s = make_gemm_inputs(w)
    set_bytes = w.min_bytes()
    nsets = max(2, min(8, math.ceil(ROTATE_BYTES / set_bytes) + 1))
    A, SA, B, SB = a_q.to(dev), a_s.to(dev), b_q.to(dev), b_s.to(dev)
    sets = []
    for i in range(nsets):
        c = torch.empty(w.M, w.N, dtype=torch.bfloat16, device=dev)
        if i == 0:
            sets.append((A, SA.t(), B, SB, c))
        else:
            sets.append((A.clone(), SA.clone().t(), B.clone(), SB.clone(), c))

    def step(i: int):
        a, sa, b, sb, c = sets[i % nsets]
        pkg.fp8_block_scaled_gemm(a, sa, b, sb, out=c)

    for i in range(args.warmup):
        step(i)
    stream = torch.cuda.current_stream(dev)
    kern_ms, wall_ms = timed_region(torch, dev, stream, step, args.steps)
    steady_ms = steady_region(args, torch, dev, stream, step)
    flops = w.flops()
    value = flops / (kern_ms * 1e-3) / 1e12
    achieved = value
    traffic = measured_traffic(w.name)
    out = {
        "metric": "fp8 block-scaled GEMM TFLOP/s (% of 5.0 PFLOP/s dense fp8), consumer of "
                  "the quantizer's codes and scales",
        "value": round(value, 1),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(kern_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3 (fp32 accumulate)",
        "data": "synthetic",
        "config": {"workload": w.name, "M": w.M, "N": w.N, "K": w.K,
                   "a_scale": w.a_scale + " col-major 1x128", "b_scale": w.b_scale + " 128x128",
                   "flops": flops, "min_hbm_bytes": set_bytes, "buffer_sets": nsets,
                   "route": pkg.gemm_route(w.M, w.N, w.K)},
        "us_per_call": round(kern_ms * 1e3, 2),
        "us_per_call_host_wall": round(wall_ms * 1e3, 2),
        "us_per_call_steady_state": None if steady_ms is None else round(steady_ms * 1e3, 2),
        "pct_of_peak": round(100.0 * achieved / PEAK_FP8_TFLOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_FP8_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP8_TFLOPS, 4),
                     "traffic": traffic},
        "cpu_baseline": None,
    }
    out["vendor_hipblaslt"] = gemm_vendor_reference(args, torch, dev, stream, sets, nsets, w)
    if args.cpu_seconds > 0:
        out["cpu_baseline"] = gemm_cpu_baseline(w, a_q, a_s, b_q, b_s, sets[0][4], args, torch)
    print(json.dumps(out), flush=True)
    return 0


def gemm_vendor_reference(args, torch, dev, stream, sets, nsets, w) -> dict:
    """The vendor library on the same fp8 operands, steps and buffer rotation, for
    comparison only: torch._scaled_mm (hipBLASLt) with one scale per tensor and with
    row-wise scales (neither has 1 x 128 / 128 x 128 block scales).  Returns us/call
    and TFLOP/s per scaling mode, or the error text when the call is unavailable."""
    res = {"call": "torch._scaled_mm(a [M, K], b.t() [K, N], out_dtype=bf16)"}
    ones_t = torch.ones((), device=dev)
    row_a = torch.ones(w.M, 1, device=dev)
    row_b = torch.ones(1, w.N, device=dev)
    for mode, sa, sb in (("per_tensor", ones_t, ones_t), ("row_wise", row_a, row_b)):
        def step(i: int, sa=sa, sb=sb):
            a, _, b, _, _ = sets[i % nsets]
            torch._scaled_mm(a, b.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
        try:
            for i in range(args.warmup):
                step(i)
            ms, _ = timed_region(torch, dev, stream, step, args.steps)
        except Exception as e:  # the op or the scaling mode missing from this torch build
            res[mode] = {"error": str(e)[:200]}
            continue
        res[mode] = {"us_per_call": round(ms * 1e3, 2),
                     "TFLOPs": round(w.flops() / (ms * 1e-3) / 1e12, 1)}
    return res


def gemm_cpu_baseline(w, a_q, a_s, b_q, b_s, c_gpu, args, torch) -> dict:
    """Times the C oracle (oracle/gemm_oracle.c, float64, OpenMP) on the first
    rows of the workload and checks those rows of the GPU's output against it."""
    import numpy as np
    import oracle
    threads = cpu_threads()
    rows = max(1, min(16, w.M))
    u8 = lambda t: t.contiguous().view(torch.uint8).numpy()
    aq, bq = u8(a_q[:rows]), u8(b_q)
    sa = np.ascontiguousarray(a_s[:, :rows].numpy())
    sb = b_s.numpy()
    ref, bound = oracle.gemm(aq, sa, bq, sb, nthreads=threads)       # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - t_start < args.cpu_seconds and len(times) < 100):
        t0 = time.perf_counter()
        oracle.gemm(aq, sa, bq, sb, nthreads=threads)
        times.append(time.perf_counter() - t0)
    times.sort()
    t = times[len(times) // 2]
    torch.cuda.synchronize()
    got = c_gpu[:rows].float().cpu().numpy()
    tol = 2.0 ** -8 * np.abs(ref) + 2 * (w.K // 128 + 130) * 2.0 ** -23 * bound
    bad = int((np.abs(got - ref) > tol).sum())
    return {"value": round(2.0 * rows * w.N * w.K / t / 1e12, 6), "unit": "TFLOP/s",
            "cores": threads, "kind": "port", "us_per_call": round(t * 1e6, 1),
            "sample": f"first {rows} of {w.M} rows of {w.name}, C oracle (float64, OpenMP), "
                      f"median of {len(times)} runs",
            "parity_vs_gpu_rows": {"ok": bad == 0, "outside_tolerance": bad}}


if __name__ == "__main__":
    sys.exit(main())
