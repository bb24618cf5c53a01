#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul hot path (BASELINE.json metric).

Default workload (BASELINE config 1 of the "configs" list is the dense decode layer; the metric is
quoted on the single Q4_K GEMV at M=1, config 0's shape on the GPU):

    step = quantize_x_q8(x) + gemv_q8(Q4_K W, 17408 x 5120) at M = 1

with the weight rotated over >= 1 GiB of device copies so the 256 MB Infinity Cache cannot serve it.
Prints ONE JSON line:
  value      -- whole-step throughput in GB/s of algorithmic bytes (W + x f32 + y = 50,225,152 B/step)
  roofline   -- the GEMV kernel alone: algorithmic bytes / its average launch duration (HIP events on
                the launch stream) against the 8 TB/s HBM peak
  cpu_baseline -- the oracle's port of the reference's host path (per-row dequant + fp32 dot), timed on
                this host's cores over a bounded sample
Secondary measurements (other configs) are added under "extra" as they become available.

Usage: python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu] [--only cfg0]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # dense bf16 MFMA
ROTATE_BYTES = 1 << 30         # >= 1 GiB of weight copies per rotation


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only", default="", help="comma list of extra measurements to run (default all)")
    return p.parse_args()


def timed(fn, iters, stream):
    """Average ms per call of fn() over `iters` back-to-back launches, HIP events on `stream`."""
    import torch
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(iters):
        fn(i)
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def cfg0_q4k_gemv(args):
    """Headline: Q4_K GEMV at M=1 on 17408 x 5120."""
    import torch
    from hipster_amd import qmm, synth

    N, K = synth.CFG0["N"], synth.CFG0["K"]
    W = synth.matrix(synth.SEEDS["cfg0"], synth.Q4_K, N, K)
    x = synth.normal_f32(synth.SEEDS["cfg0"] + 1, (1, K))
    wbytes = W.nbytes
    ncopy = max(2, -(-ROTATE_BYTES // wbytes))
    Wt = torch.from_numpy(W)
    Wd = [Wt.to("cuda") for _ in range(ncopy)]
    xd = torch.from_numpy(x).to("cuda")
    y = torch.zeros((1, N), dtype=torch.float32, device="cuda")
    xb = qmm.XQ8Buf(1, K)
    stream = torch.cuda.current_stream()
    algo_bytes = wbytes + K * 4 + N * 4            # 50,225,152 B

    def step(i):
        qmm.quantize_x_q8(xd, xb, 1, K)
        qmm.gemv_q8(synth.Q4_K, Wd[i % ncopy], xb, y, N, K, 1)

    def gemv_only(i):
        qmm.gemv_q8(synth.Q4_K, Wd[i % ncopy], xb, y, N, K, 1)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    ms_step = timed(step, args.steps, stream)
    ms_kernel = timed(gemv_only, args.steps, stream)
    return dict(N=N, K=K, W=W, x=x, ncopy=ncopy, algo_bytes=algo_bytes, ms_step=ms_step, ms_kernel=ms_kernel)


def cpu_baseline_gemv(W, x, N, K, seconds):
    """The oracle's restatement of the reference host path (dequant_row + fp32 dot per row), threaded."""
    import oracle
    threads = min(16, os.cpu_count() or 1)
    oracle.gemv_f32(0, W[:64], 64, K, x, nthreads=1)   # warm up code and pages
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        oracle.gemv_f32(0, W, N, K, x, nthreads=threads)
        times.append(time.perf_counter() - t0)
    best = min(times)
    return dict(value=(W.nbytes + K * 4 + N * 4) / best / 1e9, unit="GB/s", cores=threads, kind="port",
                sample=f"{len(times)} full calls of the 17408x5120 Q4_K GEMV at M=1 (best of {len(times)}, "
                       f"{sum(times):.1f} s total), oracle qo_gemv_f32: per-row dequant_q4_K + fp32 dot")


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (every box here has one MI355X); --gpus {args.gpus} is not supported",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    from hipster_amd import _lib
    _lib.lib()   # fails loudly if the HIP library is missing

    r = cfg0_q4k_gemv(args)
    gbs_step = r["algo_bytes"] / (r["ms_step"] * 1e-3) / 1e9
    gbs_kernel = r["algo_bytes"] / (r["ms_kernel"] * 1e-3) / 1e9
    out = {
        "metric": "Q4_K GEMV HBM GB/s (% of peak) at M=1",
        "value": round(gbs_step, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded GGUF Q4_K blocks, x ~ N(0,1)); weights rotated over "
                f"{r['ncopy']} device copies ({r['ncopy'] * r['W'].nbytes / 2**30:.2f} GiB)",
        "config": {"workload": "cfg0: quantize_x_q8 + Q4_K GEMV, M=1, W 17408x5120",
                   "N": r["N"], "K": r["K"], "M": 1, "algo_bytes_per_step": r["algo_bytes"],
                   "pct_of_hbm_peak": round(100 * gbs_step / HBM_PEAK_GBS, 1)},
        "roofline": {"bound": "hbm", "achieved": round(gbs_kernel, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs_kernel / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "k_gemv_q4k_q8<1>", "us_per_launch": round(r["ms_kernel"] * 1e3, 3)},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_gemv(r["W"], r["x"], r["N"], r["K"], args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
