#!/usr/bin/env python3
"""Benchmark of the dense-compute hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Default workload: BASELINE config 2, the bf16 GEMM M=N=K=4096 (A row-major,
B column-major, N(0,1)/sqrt(K) from seed 1, fp32 accumulate, bf16 out).  A
"step" is one launch of the hot path over one batch of synthetic input that
is already resident in HBM (generated there by the counter-based fill
kernels).  Timing uses HIP events recorded on the stream the kernels are
launched on, bracketed by stream synchronizations; `value` is whole-job
throughput (one GPU).

Prints ONE JSON line with the driver's fields plus `roofline` (dominant
kernel's achieved rate against the MI355X peak) and `cpu_baseline` (the CPU
oracle restatement timed on this host over a bounded sample of the same
workload; a reported baseline only).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# MI355X published dense peaks (TFLOP/s) and HBM bandwidth (GB/s)
PEAK = {"bf16": 2516.6, "fp8": 5033.2, "fp32": 157.3, "hbm_gbs": 8000.0}


def _cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _traffic_from_profiles(kernel_key: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy-kernel calibration) and committed under
    profiles/ as a line `traffic_bytes_per_launch <kernel_key> <bytes>`."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel_key:
                return float(parts[2])
    return None


class Timer:
    def __init__(self, ctx, stream):
        from fe2o3_amd.runtime import Event
        self.stream = stream
        self.start, self.stop = Event(ctx), Event(ctx)

    def run(self, step, steps: int, warmup: int):
        for _ in range(warmup):
            step()
        self.stream.synchronize()
        t0 = time.perf_counter()
        self.start.record(self.stream)
        for _ in range(steps):
            step()
        self.stop.record(self.stream)
        self.stop.synchronize()
        self.stream.synchronize()
        wall = time.perf_counter() - t0
        return self.start.elapsed_ms(self.stop) / steps, wall


# ---- workloads -----------------------------------------------------------------------

def wl_gemm_bf16(ctx, stream, args):
    from fe2o3_amd import kernels
    m = n = k = 4096
    seed = 1
    scale = float(1.0 / np.sqrt(k))
    a = ctx.alloc(m * k, np.uint16)
    b = ctx.alloc(n * k, np.uint16)
    c = ctx.alloc(m * n, np.uint16)
    kernels.fill_normal_bf16(a, seed, 0xA, scale, stream=stream)
    kernels.fill_normal_bf16(b, seed, 0xB, scale, stream=stream)
    prepared = kernels.gemm_bf16_nt_gpu.Kernel.load(ctx).prepare(a, b, c, m, n, k)
    flop = 2.0 * m * n * k
    ms, wall = Timer(ctx, stream).run(lambda: prepared.launch_async(stream), args.steps, args.warmup)

    # parity spot check of the timed output against the CPU oracle (4 rows)
    from oracle import oracle as orc
    ha, hb = a.download(), b.download()
    got = (c.download().astype(np.uint32) << 16).view(np.float32).reshape(m, n)
    rows = [0, 1111, 2222, 4095]
    ref = np.stack([orc.gemm_bf16_nt_rows(m, n, k, ha, hb, r, r + 1) for r in rows])
    rel = float(np.max(np.abs(got[rows] - ref)) / np.max(np.abs(ref)))

    cpu = None
    if args.cpu_baseline:
        threads = _cpu_threads()
        probe_rows = 16
        t0 = time.perf_counter()
        orc.gemm_bf16_nt_rows(m, n, k, ha, hb, 0, probe_rows, threads=threads)
        per_row = (time.perf_counter() - t0) / probe_rows
        rows_n = int(max(probe_rows, min(m, args.cpu_seconds / max(per_row, 1e-9))))
        t0 = time.perf_counter()
        orc.gemm_bf16_nt_rows(m, n, k, ha, hb, 0, rows_n, threads=threads)
        dt = time.perf_counter() - t0
        cpu = {"value": 2.0 * rows_n * n * k / dt / 1e12, "unit": "TFLOP/s", "cores": threads,
               "kind": "port",
               "sample": f"oracle/gemm.c fe2o3o_gemm_bf16_nt_rows (sequential unfused fp32 "
                         f"recurrence, -O3 -ffp-contract=off, OpenMP over columns) on the first "
                         f"{rows_n} of {m} output rows of the same 4096^3 inputs, {dt:.1f} s"}
    return {
        "metric": "bf16 GEMM TFLOP/s (M=N=K=4096) on 1 MI355X",
        "unit": "TFLOP/s", "dtype": "bf16", "flop": flop, "ms": ms, "wall": wall,
        "peak_key": "bf16", "kernel": "gemm_bf16_nt_256_kernel",
        "config": {"workload": "bf16 GEMM C=A.B^T, M=N=K=4096, A row-major, B column-major "
                               "([N,K] K-contiguous), A,B ~ N(0,1)/sqrt(K) seed 1, fp32 "
                               "accumulate, bf16 out (BASELINE config 2)",
                   "m": m, "n": n, "k": k},
        "parity": {"rows_checked": rows, "max_rel_err": rel, "tolerance": 1e-2},
        "cpu": cpu, "traffic_key": "gemm_bf16_nt_4096",
    }


WORKLOADS = {"gemm_bf16": wl_gemm_bf16}


def main() -> int:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", default="gemm_bf16", choices=sorted(WORKLOADS))
    p.add_argument("--cpu-seconds", type=float, default=20.0)
    p.add_argument("--no-cpu-baseline", dest="cpu_baseline", action="store_false")
    args = p.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not "
              "supported (the path would shard as described in DESIGN.md)", file=sys.stderr)
        return 2

    from fe2o3_amd.runtime import GpuContext
    ctx = GpuContext.current(0)
    stream = ctx.stream()
    r = WORKLOADS[args.workload](ctx, stream, args)

    value = r["flop"] / (r["ms"] * 1e-3) / 1e12
    peak = PEAK[r["peak_key"]]
    traffic = _traffic_from_profiles(r["traffic_key"])
    line = {
        "metric": r["metric"], "value": round(value, 2), "unit": r["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(r["ms"], 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": r["dtype"],
        "data": "synthetic (counter-based N(0,1) generated in HBM; bit-identical to the CPU "
                "oracle's generator)",
        "config": r["config"],
        "roofline": {"bound": "mfma", "achieved": round(value, 2), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(value / peak, 4), "traffic": traffic,
                     "kernel": r["kernel"],
                     "device": {"arch": ctx.arch, "compute_units": ctx.compute_units,
                                "clock_mhz": ctx.clock_khz / 1000.0}},
        "cpu_baseline": r["cpu"],
        "parity": r["parity"],
        "wall_s_timed_region": round(r["wall"], 4),
    }
    print(json.dumps(line), flush=True)
    ok = r["parity"]["max_rel_err"] <= r["parity"]["tolerance"]
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
