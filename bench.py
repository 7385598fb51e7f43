"""Benchmark of the quantized-linear hot path on one MI355X.

Workload ("c2"): fused SwiGLU -> MXFP8 producer + MXFP8
down projection, gate_up bf16 [M, 2 x 9216] ~ N(0, 1), weights [2560, 9216] ~ N(0, 0.02)
pre-quantized to MXFP8 (E4M3 + E8M0 per 32), bf16 out, for M in {1, 16, 128, 512}.
One step = the producer + GEMM at each of the four M.  Weights rotate over enough
copies to exceed the 256 MB Infinity Cache, so every step streams them from HBM.

Timing: each step is one hipGraph (the reference's protocol, tools/benchmark_nvfp4_lm_head.py:17-40:
warm, capture, replay, event-timed).  `value` = total algorithmic TFLOP over the step
/ measured step time.  Per-kernel durations come from graphs of back-to-back launches of
that kernel, timed with HIP events on the stream they run on.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

N_OUT, K_IN = 2560, 9216
M_SWEEP = (1, 16, 128, 512)
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 5000.0  # dense MXFP8 (E4M3) scaled MFMA
WEIGHT_COPIES = 16         # 16 x 24.3 MB = 389 MB > 256 MB Infinity Cache


def algorithmic(M: int):
    """flops and bytes of the fused producer + GEMM at one M (SURVEY 8(d) counts):
    weight codes + E8M0 scales + gate_up bf16 in (4 B per K element) + bf16 out."""
    flops = 2.0 * M * N_OUT * K_IN
    w_bytes = N_OUT * K_IN + N_OUT * K_IN // 32
    bytes_ = w_bytes + M * K_IN * 4 + M * N_OUT * 2
    gemm_bytes = w_bytes + M * K_IN * (1 + 1 / 32) + M * N_OUT * 2  # GEMM alone reads MXFP8 A
    return flops, bytes_, gemm_bytes


def graph_time_us(fn_list, stream, replays=20, trials=9):
    """Capture the callables back to back in one graph; median us per graph replay."""
    with torch.cuda.stream(stream):
        for fn in fn_list:
            fn()
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for fn in fn_list:
                fn()
        for _ in range(3):
            g.replay()
        stream.synchronize()
        times = []
        for _ in range(trials):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record(stream)
            for _ in range(replays):
                g.replay()
            e.record(stream)
            e.synchronize()
            times.append(s.elapsed_time(e) * 1000.0 / replays)
    times.sort()
    return times[len(times) // 2], g


def cpu_baseline(budget_s: float = 15.0):
    """The oracle's CPU path (C producer + exact dequantize + BLAS matmul) on a bounded
    sample of the same workload: M = 16 rows of c2, repeated for about `budget_s`."""
    import numpy as np
    import oracle
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(N_OUT, K_IN, generator=g) * 0.02).bfloat16()
    wc, ws = oracle.quant_mxfp8(w, 0)
    wdq = torch.from_numpy(oracle.dequant_mx(wc, ws, 0))
    M = 16
    gu = torch.randn(M, 2 * K_IN, generator=g).bfloat16()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n < 2:
        c, s = oracle.swiglu_mxfp8(gu, oracle.RULE_CEIL_DIV448)
        a = torch.from_numpy(oracle.dequant_mx(c, s, 0))
        _ = (a @ wdq.T).bfloat16()
        n += 1
    dt = (time.perf_counter() - t0) / n
    flops = 2.0 * M * N_OUT * K_IN
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"c2 at M={M}: oracle SwiGLU->MXFP8 (C, 1 thread) + exact dequant + torch fp32 matmul "
                      f"({threads} threads) + bf16, weights pre-dequantized, {n} runs x {dt * 1e3:.1f} ms"}


def kernel_only(pkg, args):
    """Launch one kernel `iters` times (weights rotated as in the step) and print its
    event-timed average, for rocprofv3 kernel-trace and counter runs."""
    ops = pkg.ops
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(1234)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if args.kernel_only == "copy":
        # calibration for HBM byte counters: a plain device copy of known size
        nbytes = 256 << 20
        src = torch.empty(nbytes, dtype=torch.uint8, device=dev).random_(generator=gen)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        s.record()
        for _ in range(args.iters):
            dst.copy_(src)
        e.record()
        e.synchronize()
        us = s.elapsed_time(e) * 1000 / args.iters
        print(json.dumps({"kernel": "copy", "bytes_read": nbytes, "bytes_written": nbytes, "us": round(us, 2),
                          "GBs": round(2 * nbytes / us / 1e3, 1)}))
        return
    w = (torch.randn(N_OUT, K_IN, generator=gen, device=dev) * 0.02).bfloat16()
    wc, ws = torch.ops.mach_amd.quantize_mxfp8(w, 0)
    tiled, tiled_s = ops.pack_weight(wc, ws, ops.E4M3)
    copies = [(tiled.clone(), tiled_s.clone()) for _ in range(WEIGHT_COPIES)]
    gate_up = torch.randn(args.m, 2 * K_IN, generator=gen, device=dev).bfloat16()
    a, sa = torch.ops.mach_amd.swiglu_mxfp8(gate_up, ops.CEIL_DIV448, False)
    if args.kernel_only == "producer":
        fn = lambda i: torch.ops.mach_amd.swiglu_mxfp8(gate_up, ops.CEIL_DIV448, False)
    else:
        fn = lambda i: torch.ops.mach_amd.mx_gemm(a, sa, copies[i % WEIGHT_COPIES][0],
                                                  copies[i % WEIGHT_COPIES][1], N_OUT, K_IN, ops.E4M3, None)
    for i in range(WEIGHT_COPIES):
        fn(i)
    torch.cuda.synchronize()
    s.record()
    for i in range(args.iters):
        fn(i)
    e.record()
    e.synchronize()
    us = s.elapsed_time(e) * 1000 / args.iters
    flops, bytes_, gemm_bytes = algorithmic(args.m)
    print(json.dumps({"kernel": args.kernel_only, "M": args.m, "N": N_OUT, "K": K_IN, "us_eager": round(us, 2),
                      "algorithmic_bytes": int(gemm_bytes if args.kernel_only == "gemm" else args.m * K_IN * 5 + args.m * K_IN // 32),
                      "flops": flops}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-only", choices=["gemm", "producer", "copy"],
                    help="profiling mode: launch one kernel back to back (for rocprofv3)")
    ap.add_argument("--m", type=int, default=512, help="rows for --kernel-only")
    ap.add_argument("--iters", type=int, default=64, help="launches for --kernel-only")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import __graft_entry__
    pkg = __graft_entry__.load_package()
    if args.kernel_only:
        kernel_only(pkg, args)
        return
    ops = pkg.ops
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(1234)

    # weights: quantize once with the product quantizer, pack, then replicate
    w = (torch.randn(N_OUT, K_IN, generator=gen, device=dev) * 0.02).bfloat16()
    wc, ws = torch.ops.mach_amd.quantize_mxfp8(w, 0)
    tiled, tiled_s = ops.pack_weight(wc, ws, ops.E4M3)
    copies = [(tiled.clone(), tiled_s.clone()) for _ in range(WEIGHT_COPIES)]
    del w, wc, ws, tiled, tiled_s
    inputs = {M: torch.randn(M, 2 * K_IN, generator=gen, device=dev).bfloat16() for M in M_SWEEP}
    stream = torch.cuda.Stream()

    def step_fns(ci):
        wt, st = copies[ci]
        return [lambda M=M: ops.swiglu_mx_down(inputs[M], wt, st, N_OUT, ops.E4M3) for M in M_SWEEP]

    # one graph per weight copy; a step replays the next one
    graphs = []
    with torch.cuda.stream(stream):
        for ci in range(WEIGHT_COPIES):
            for fn in step_fns(ci):
                fn()
        stream.synchronize()
        for ci in range(WEIGHT_COPIES):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for fn in step_fns(ci):
                    fn()
            graphs.append(g)
        for i in range(args.warmup):
            graphs[i % WEIGHT_COPIES].replay()
        stream.synchronize()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(args.steps):
            graphs[i % WEIGHT_COPIES].replay()
        end.record(stream)
        end.synchronize()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps
    total_flops = sum(algorithmic(M)[0] for M in M_SWEEP)
    value = total_flops / (ms_per_step * 1e-3) / 1e12

    # per-kernel timing: back-to-back launches of one op over rotated weight copies
    per_m = {}
    for M in M_SWEEP:
        a, sa = torch.ops.mach_amd.swiglu_mxfp8(inputs[M], ops.CEIL_DIV448, False)
        prod_us, _ = graph_time_us([lambda M=M: torch.ops.mach_amd.swiglu_mxfp8(inputs[M], ops.CEIL_DIV448, False)] * 8,
                                   stream)
        gemm_fns = [lambda wt=wt, st=st, a=a, sa=sa: torch.ops.mach_amd.mx_gemm(a, sa, wt, st, N_OUT, K_IN, ops.E4M3, None)
                    for wt, st in copies]
        gemm_us, _ = graph_time_us(gemm_fns, stream)
        gemm_us /= len(gemm_fns)
        prod_us /= 8
        flops, bytes_, gemm_bytes = algorithmic(M)
        t_min = max(flops / (MFMA_PEAK_TFLOPS * 1e12), gemm_bytes / (HBM_PEAK_GBS * 1e9)) * 1e6
        per_m[M] = {"producer_us": round(prod_us, 2), "gemm_us": round(gemm_us, 2),
                    "gemm_tflops": round(flops / gemm_us / 1e6, 2),
                    "gemm_gbs": round(gemm_bytes / gemm_us / 1e3, 1),
                    "gemm_roofline_frac": round(t_min / gemm_us, 3),
                    "bound": "mfma" if flops / (MFMA_PEAK_TFLOPS * 1e12) > gemm_bytes / (HBM_PEAK_GBS * 1e9) else "hbm"}

    dom = max(M_SWEEP, key=lambda M: per_m[M]["gemm_us"])
    d = per_m[dom]
    flops, _, gemm_bytes = algorithmic(dom)
    if d["bound"] == "hbm":
        roof = {"bound": "hbm", "achieved": d["gemm_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(d["gemm_gbs"] / HBM_PEAK_GBS, 4), "traffic": None}
    else:
        roof = {"bound": "mfma", "achieved": d["gemm_tflops"], "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(d["gemm_tflops"] / MFMA_PEAK_TFLOPS, 4), "traffic": None}
    roof["kernel"] = f"mxfp8 gemm_kernel M={dom} N={N_OUT} K={K_IN}"
    roof["algorithmic_bytes_per_launch"] = int(gemm_bytes)

    out = {
        "metric": "GEMM TFLOP/s & HBM GB/s (% roofline) at M=1..512; bit-exact quant codes",
        "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "mxfp8(e4m3+e8m0) x mxfp8, fp32 accumulate, bf16 out",
        "data": "synthetic (seeded randn), weights rotated over 16 copies (cold HBM)",
        "config": {"workload": "c2: SwiGLU->MXFP8 producer + MXFP8 down projection",
                   "M": list(M_SWEEP), "N": N_OUT, "K": K_IN, "parallelism": "single GPU"},
        "per_m": per_m, "roofline": roof,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
