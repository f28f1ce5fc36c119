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
        "peak_key": "bf16", "kernel": "gemm_bf16_nt_256_kernel<false>",
        "config": {"workload": "bf16 GEMM C=A.B^T, M=N=K=4096, A row-major, B column-major "
                               "([N,K] K-contiguous), A,B ~ N(0,1)/sqrt(K) seed 1, fp32 "
                               "accumulate, bf16 out (BASELINE config 2)",
                   "m": m, "n": n, "k": k},
        "parity": {"rows_checked": rows, "max_rel_err": rel, "tolerance": 1e-2},
        "cpu": cpu, "traffic_key": "gemm_bf16_nt_4096",
    }


def _timed(ctx, stream, fn, steps, warmup):
    ms, _ = Timer(ctx, stream).run(fn, steps, warmup)
    return ms


def sec_flash(ctx, stream, causal, steps, warmup):
    """Config 3a/3b: B8 H32 S4096 D128 bf16, scale 1/sqrt(128), LSE out."""
    from fe2o3_amd import kernels
    b, h, s, d = 8, 32, 4096, 128
    n = b * h * s * d
    q, k, v, o = (ctx.alloc(n, np.uint16) for _ in range(4))
    lse = ctx.alloc(b * h * s, np.float32)
    for i, t in enumerate((q, k, v)):
        kernels.fill_normal_bf16(t, 2, 0xF100 + i, 1.0, stream=stream)
    prep = kernels.flash_attention_fwd_gpu.Kernel.load(ctx).prepare(
        q, k, v, o, lse, b, h, s, d, 1 if causal else 0, float(1.0 / np.sqrt(d)))
    ms = _timed(ctx, stream, lambda: prep.launch_async(stream), steps, warmup)
    flop = 4.0 * b * h * s * s * d * (0.5 if causal else 1.0)
    tf = flop / (ms * 1e-3) / 1e12
    return {"workload": f"flash-attn fwd {'causal' if causal else 'non-causal'} B8 H32 S4096 "
                        f"D128 bf16 (config 3{'b' if causal else 'a'})",
            "kernel": f"flash_fwd_kernel<{str(bool(causal)).lower()}>", "ms": ms,
            "value": round(tf, 2), "unit": "TFLOP/s",
            "roofline": {"bound": "mfma", "peak": PEAK["bf16"], "frac": round(tf / PEAK["bf16"], 4)}}


def sec_softmax(ctx, stream, steps, warmup):
    """Config 3c: 1,048,576 rows x 4096 fp32 in/out (HBM-bound)."""
    from fe2o3_amd import kernels
    rows, cols = 8 * 32 * 4096, 4096
    x = ctx.alloc(rows * cols, np.float32)
    y = ctx.alloc(rows * cols, np.float32)
    kernels.fill_normal_f32(x, 3, 0x50F7, 1.0, stream=stream)
    prep = kernels.row_softmax_gpu.Kernel.load(ctx).prepare(x, y, None, rows, cols)
    ms = _timed(ctx, stream, lambda: prep.launch_async(stream), steps, warmup)
    gbs = rows * cols * 8 / (ms * 1e-3) / 1e9
    return {"workload": "row softmax 1048576 x 4096 fp32 (config 3c)",
            "kernel": "softmax_reg_kernel<16,false>", "ms": ms, "value": round(gbs, 1),
            "unit": "GB/s",
            "roofline": {"bound": "hbm", "peak": PEAK["hbm_gbs"],
                         "frac": round(gbs / PEAK["hbm_gbs"], 4)}}


def sec_fp8(ctx, stream, steps, warmup):
    """Config 4: fp8 e4m3 GEMM 8192^3, per-tensor amax/448 scales, bf16 out."""
    from fe2o3_amd import kernels
    m = n = k = 8192
    a32, b32 = ctx.alloc(m * k, np.float32), ctx.alloc(n * k, np.float32)
    kernels.fill_normal_f32(a32, 4, 0xA, 1.0, stream=stream)
    kernels.fill_normal_f32(b32, 4, 0xB, 1.0, stream=stream)
    sa, sb, am = ctx.alloc(1, np.float32), ctx.alloc(1, np.float32), ctx.alloc(1, np.float32)
    aq, bq = ctx.alloc(m * k, np.uint8), ctx.alloc(n * k, np.uint8)
    quant_ms = 0.0
    for src, sc, q in ((a32, sa, aq), (b32, sb, bq)):
        def quant(src=src, sc=sc, q=q):
            kernels.amax_f32(src, am, stream=stream, sync=False)
            kernels.fp8_scale_from_amax(am, sc, stream=stream, sync=False)
            kernels.quantize_e4m3(src, sc, q, stream=stream, sync=False)
        quant_ms += _timed(ctx, stream, quant, 5, 1)
    c = ctx.alloc(m * n, np.uint16)
    gemm = lambda: kernels.gemm_fp8_nt(aq, bq, sa, sb, c, m, n, k, stream=stream, sync=False)
    ms = _timed(ctx, stream, gemm, steps, warmup)
    tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    return {"workload": "fp8 e4m3 GEMM 8192^3, per-tensor scales, bf16 out (config 4)",
            "kernel": "gemm_fp8_kernel<false>", "ms": ms, "value": round(tf, 2), "unit": "TFLOP/s",
            "quantize_ms_both_operands": round(quant_ms, 4),
            "roofline": {"bound": "mfma", "peak": PEAK["fp8"], "frac": round(tf / PEAK["fp8"], 4)}}


def sec_moe(ctx, stream, steps, warmup):
    """Config 5: 4096 tokens, hidden 4096, 8 experts, FFN 14336, top-2."""
    from fe2o3_amd import kernels
    t, hdim, f, e = 4096, 4096, 14336, 8
    lg = ctx.alloc(t * e, np.uint16)
    x = ctx.alloc(t * hdim, np.uint16)
    kernels.fill_normal_bf16(lg, 5, 0x10617, 1.0, stream=stream)
    kernels.fill_normal_bf16(x, 5, 0xAC7, 1.0, stream=stream)
    w = [ctx.alloc(e * f * hdim, np.uint16) for _ in range(3)]
    for i, dom in enumerate((0x6A7E, 0x0B0B, 0xD0D0)):
        kernels.fill_normal_bf16(w[i], 5, dom, 0.02, stream=stream)
    r = {"top2": ctx.alloc(2 * t, np.uint32), "requested": ctx.alloc(e, np.uint32),
         "admitted": ctx.alloc(e, np.uint32), "offsets": ctx.alloc(e + 1, np.uint32),
         "slots": ctx.alloc(2 * t, np.uint32), "permutation": ctx.alloc(2 * t, np.uint32),
         "inverse": ctx.alloc(2 * t, np.uint32), "weights": ctx.alloc(2 * t, np.float32)}
    ws = ctx.alloc(kernels.moe_ffn_workspace_bytes(t, hdim, f, e), np.uint8)
    out = ctx.alloc(t * hdim, np.uint16)

    def layer():
        kernels.moe_top2_route(lg, r, t, e, stream=stream, sync=False)
        kernels.moe_ffn_top2(x, w[0], w[1], w[2], r, out, ws, t, hdim, f, e, stream=stream,
                             sync=False)
    ms = _timed(ctx, stream, layer, max(3, steps // 10), max(1, warmup // 10))
    flop = 3.0 * 2.0 * hdim * f * 2 * t
    tf = flop / (ms * 1e-3) / 1e12
    return {"workload": "MoE top-2 layer: 4096 tokens, hidden 4096, 8 experts, FFN 14336, "
                        "router + gather + gate/up SiLU + down + combine (config 5)",
            "kernel": "gate_up_kernel + down_kernel", "ms": ms, "value": round(tf, 2),
            "unit": "TFLOP/s",
            "roofline": {"bound": "mfma", "peak": PEAK["bf16"], "frac": round(tf / PEAK["bf16"], 4)}}


def sec_gemm_f32(ctx, stream, steps, warmup):
    """Config 1: f32 GEMM 256^3, U[-1,1] seed 0, sequential unfused recurrence."""
    from fe2o3_amd import kernels
    m = n = k = 256
    a, b, c = ctx.alloc(m * k, np.float32), ctx.alloc(k * n, np.float32), ctx.alloc(m * n, np.float32)
    kernels.fill_uniform_f32(a, 0, 0xA, stream=stream)
    kernels.fill_uniform_f32(b, 0, 0xB, stream=stream)
    prep = kernels.scalar_gemm_v1_gpu.Kernel.load(ctx).prepare(a, b, c, m, n, k)
    ms = _timed(ctx, stream, lambda: prep.launch_async(stream), steps, warmup)
    tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    return {"workload": "f32 GEMM 256^3 bit-exact sequential recurrence (config 1)",
            "kernel": "scalar_gemm_kernel", "ms": ms, "value": round(tf, 3), "unit": "TFLOP/s",
            "roofline": {"bound": "fp32 VALU", "peak": PEAK["fp32"],
                         "frac": round(tf / PEAK["fp32"], 5)}}


def sec_collectives(ctx, stream, steps, warmup):
    """Wave64 collectives over 2^20 rows of 64 f32 with one mask per row:
    4 bytes in and 12 bytes out per element plus 8 bytes per row (HBM-bound)."""
    from fe2o3_amd import kernels
    rows = 1 << 20
    x = ctx.alloc(rows * 64, np.float32)
    kernels.fill_normal_f32(x, 6, 0xC011, 1.0, stream=stream)
    masks = ctx.to_device(np.random.default_rng(6).integers(0, 2**63, rows, dtype=np.uint64))
    outs = [ctx.alloc(rows * 64, np.float32) for _ in range(3)]
    ms = _timed(ctx, stream, lambda: kernels.wave64_collectives_rows(
        x, masks, *outs, rows, stream=stream, sync=False), steps, warmup)
    nbytes = rows * (64 * 16 + 8)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": "wave64 masked reduce + inclusive/exclusive scan, 2^20 rows x 64 f32",
            "kernel": "wave64_collectives_rows_kernel", "ms": ms, "value": round(gbs, 1),
            "unit": "GB/s",
            "roofline": {"bound": "hbm", "peak": PEAK["hbm_gbs"],
                         "frac": round(gbs / PEAK["hbm_gbs"], 4)}}


def sec_routing_check(ctx, stream, steps, warmup):
    """Routing-output consistency check of config 5's router output (4096
    tokens, 8 experts, unbounded capacity): one workgroup, latency-bound."""
    from fe2o3_amd import kernels
    t, e = 4096, 8
    lg = ctx.alloc(t * e, np.uint16)
    kernels.fill_normal_bf16(lg, 5, 0x10617, 1.0, stream=stream)
    r = {"top2": ctx.alloc(2 * t, np.uint32), "requested": ctx.alloc(e, np.uint32),
         "admitted": ctx.alloc(e, np.uint32), "offsets": ctx.alloc(e + 1, np.uint32),
         "slots": ctx.alloc(2 * t, np.uint32), "permutation": ctx.alloc(2 * t, np.uint32),
         "inverse": ctx.alloc(2 * t, np.uint32), "weights": ctx.alloc(2 * t, np.float32)}
    kernels.moe_top2_route(lg, r, t, e, stream=stream)
    rec = ctx.alloc(4, np.uint32)
    ms = _timed(ctx, stream, lambda: kernels.moe_routing_check(
        r, t, e, 0xFFFFFFFF, rec, stream=stream, sync=False), steps, warmup)
    kind = int(rec.download()[0])
    return {"workload": "MoE routing-output consistency check, 4096 tokens x 8 experts",
            "kernel": "routing_check_kernel", "ms": ms, "value": round(ms * 1e3, 2),
            "unit": "us", "record_kind": kind,
            "roofline": {"bound": "latency (one workgroup)", "peak": None, "frac": None}}


SECONDARY = {
    "flash_noncausal": lambda c, s, a: sec_flash(c, s, False, a.steps, a.warmup),
    "flash_causal": lambda c, s, a: sec_flash(c, s, True, a.steps, a.warmup),
    "softmax": lambda c, s, a: sec_softmax(c, s, max(5, a.steps // 10), max(2, a.warmup // 10)),
    "fp8_gemm": lambda c, s, a: sec_fp8(c, s, a.steps, a.warmup),
    "moe": lambda c, s, a: sec_moe(c, s, a.steps, a.warmup),
    "gemm_f32": lambda c, s, a: sec_gemm_f32(c, s, a.steps, a.warmup),
    "collectives": lambda c, s, a: sec_collectives(c, s, max(5, a.steps // 10),
                                                   max(2, a.warmup // 10)),
    "routing_check": lambda c, s, a: sec_routing_check(c, s, max(5, a.steps // 10),
                                                       max(2, a.warmup // 10)),
}

WORKLOADS = {"gemm_bf16": wl_gemm_bf16}


def calibrate_copy(ctx, stream, args):
    """1 GiB device-to-device copy: 1 GiB read + 1 GiB written per launch."""
    from fe2o3_amd import _lib
    from fe2o3_amd.runtime import check
    n = 1 << 30
    src, dst = ctx.alloc(n, np.uint8), ctx.alloc(n, np.uint8)
    copy = lambda: check(_lib.lib().fe2o3_rt_memcpy_async(dst.ptr, src.ptr, n, 3, stream.handle),
                         "copy")
    ms = _timed(ctx, stream, copy, args.steps, args.warmup)
    print(json.dumps({"calibration": "d2d copy", "bytes_read": n, "bytes_written": n,
                      "ms": round(ms, 5), "gbs": round(2 * n / (ms * 1e-3) / 1e9, 1)}), flush=True)
    return 0


def main() -> int:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    # MI355X idles at a low clock and needs tens of milliseconds of load to
    # reach its steady clock: the defaults warm up for ~30 ms and time ~70 ms
    p.add_argument("--steps", type=int, default=500)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--workload", default="gemm_bf16", choices=sorted(WORKLOADS))
    p.add_argument("--cpu-seconds", type=float, default=20.0)
    p.add_argument("--no-cpu-baseline", dest="cpu_baseline", action="store_false")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only time a 1 GiB device-to-device copy (the reference kernel "
                        "whose FETCH_SIZE/WRITE_SIZE calibrate the traffic counters)")
    p.add_argument("--secondary", default="all",
                   help="comma list of other configs to time after the main one "
                        f"({','.join(SECONDARY)}), 'all' or 'none'")
    args = p.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not "
              "supported (across GPUs the GEMM would shard by output tile rows, flash "
              "attention by (batch, head), the MoE layer by expert)", file=sys.stderr)
        return 2

    from fe2o3_amd.runtime import GpuContext
    ctx = GpuContext.current(0)
    stream = ctx.stream()
    if args.calibrate_copy:
        return calibrate_copy(ctx, stream, args)
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
    names = list(SECONDARY) if args.secondary == "all" else \
        [x for x in args.secondary.split(",") if x and x != "none"]
    if names:
        line["secondary"] = {}
        for name in names:
            res = SECONDARY[name](ctx, stream, args)
            res["ms"] = round(res["ms"], 5)
            line["secondary"][name] = res
    print(json.dumps(line), flush=True)
    ok = r["parity"]["max_rel_err"] <= r["parity"]["tolerance"]
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
