#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul hot path (BASELINE.json metric).

Workload (the configuration the metric is quoted on: BASELINE config 0's shape on one GPU):

    step = qmm_gemv_q8_f32x(Q4_K W 17408 x 5120, x f32, M = 1): the q8 quantisation of x runs inside
           the GEMV's x staging (bit-identical to qmm_quantize_x_q8 + qmm_gemv_q8, which is timed too)

x is f32 N(0,1) [5120], y f32 [17408].  W is rotated over >= 1 GiB of device copies so the 256 MB
Infinity Cache cannot serve it; inputs are resident in HBM before the timed region.  The W warm-up
steps and the K timed steps are each captured into one HIP graph (the engine launches from C++;
graph replay keeps the Python launch cost out of the GPU timeline) and replayed once, bracketed by
torch.cuda.synchronize() and HIP events on the launch stream.

Prints ONE JSON line:
  value        -- whole-step throughput: algorithmic bytes (W + x f32 + y f32 = 50,225,152 B/step) / time
  roofline     -- the dominant kernel (the Q4_K GEMV) alone: the same algorithmic bytes / its average
                  launch duration (a graph of K back-to-back launches, HIP events), against 8 TB/s
  cpu_baseline -- the reference host path (per-row dequant_q4_K + fp32 dot) built from the reference's
                  quant.h (the oracle's restatement when that is absent), on all host cores and on one,
                  timed over a bounded sample (--cpu-seconds); the MoE configs get CPU legs under "extra"

The other BASELINE configurations are measured too and reported under "extra" (parity-test
shapes, not the headline): the dense decode layer at M = 1, 4, 8 (config 1), the MoE decode step at
T = 1, 4, 8 (config 2), the dense prefill GEMM and the M = 3..6 verify GEMVs (config 3) and the MoE
prefill pipeline at 2048 tokens (config 4), and the q8 GEMV of every weight format of the call surface
at config 0's shape.  --no-extra skips them.

Usage: python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu] [--cpu-seconds 10] [--no-extra]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
ROTATE_BYTES = 1 << 30         # >= 1 GiB of weight copies per rotation


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-extra", action="store_true", help="skip the other BASELINE configurations")
    p.add_argument("--only-extra", choices=["activation_producers", "formats", "router", "dense_decode", "moe_decode", "moe_prefill",
                                            "dense_prefill", "moe_uniform"],
                   default=None,
                   help="only run one of the extra measurements and print its JSON (for profiling it alone)")
    p.add_argument("--roofs", action="store_true",
                   help="only run the roof microbenchmarks (streaming read of the GEMV's 50 MB over a >= 1 GiB rotation, "
                        "asymptotic 1 GiB read, matrix-instruction issue rates) and print their JSON")
    p.add_argument("--calib-copy", action="store_true",
                   help="only run 10 plain device copies of 256 MiB (calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    return p.parse_args()


def calib_copy():
    """A plain copy kernel of known size: 10 x 256 MiB read + 256 MiB written (torch's copy kernel).
    The counter reads of these dispatches scale the ones of the measured kernels."""
    import torch
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").random_()
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calib_copy_bytes_read": n, "calib_copy_bytes_written": n, "dispatches": 10}), flush=True)


def roofs(torch):
    """MI355X roofs re-measured by libhipster_roofs.so (hipster_amd/csrc/roofs/roofs.hip, the method of the
    reference's bench/roofline/bandwidth.hip and wmma_rate.hip): streaming-read GB/s of config 0's
    50,135,040 weight bytes rotated over >= 1 GiB of copies (grid-stride loop as bandwidth.hip, and one-shot
    bursts of U loads per thread as the GEMV issues them, plain and nontemporal), the asymptotic read of one
    1 GiB buffer, the issue rate of independent matrix instructions (TFLOP/s, TOP/s) and the LDS read
    rate of ds_read_b128 per CU."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "hipster_amd", "lib", "libhipster_roofs.so"))
    lib.qmm_roof_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                  ctypes.c_void_p]
    lib.qmm_roof_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.qmm_roof_lds.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    sink = torch.zeros(64, dtype=torch.int32, device="cuda")
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = {}

    def read_us(bufs, nbytes, variant, grid, unroll, reps=3):
        def one(b):
            return lambda: lib.qmm_roof_read(ctypes.c_void_p(b.data_ptr()), nbytes, variant, grid, unroll,
                                             ctypes.c_void_p(sink.data_ptr()), st())
        return graph_us(torch, [one(b) for b in bufs], reps=reps) / len(bufs)

    nbytes = 50135040                                     # config 0's Q4_K weight bytes
    ncopy = -(-ROTATE_BYTES // nbytes)
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").random_() for _ in range(ncopy)]
    r50 = {}
    for grid in (1024, 2048, 4096, 8192):
        us = read_us(bufs, nbytes, 0, grid, 0)
        r50[f"stride_grid{grid}"] = {"us": round(us, 2), "GB_s": round(nbytes / us / 1e3, 1)}
    for variant, tag in ((1, "burst"), (2, "burst_nt")):
        for u in (4, 8, 16):
            us = read_us(bufs, nbytes, variant, 0, u)
            r50[f"{tag}_u{u}"] = {"us": round(us, 2), "GB_s": round(nbytes / us / 1e3, 1)}
    best = max(v["GB_s"] for v in r50.values())
    out["read_50MB_rotated"] = dict(r50, best_GB_s=best, pct_of_8TBs=round(100 * best / HBM_PEAK_GBS, 1),
                                    copies=ncopy)
    del bufs
    torch.cuda.empty_cache()
    big = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").random_()
    r1g = {}
    for grid in (4096, 16384, 65536):
        us = read_us([big], 1 << 30, 0, grid, 0, reps=5)
        r1g[f"stride_grid{grid}"] = {"us": round(us, 1), "GB_s": round((1 << 30) / us / 1e3, 1)}
    us = read_us([big], 1 << 30, 1, 0, 16, reps=5)
    r1g["burst_u16"] = {"us": round(us, 1), "GB_s": round((1 << 30) / us / 1e3, 1)}
    out["read_1GiB"] = r1g
    del big
    torch.cuda.empty_cache()
    ops = {0: ("mfma_f32_32x32x16_bf16", 2 * 32 * 32 * 16, 2500.0), 1: ("mfma_f32_16x16x32_bf16", 2 * 16 * 16 * 32, 2500.0),
           2: ("mfma_i32_32x32x32_i8", 2 * 32 * 32 * 32, 5000.0), 3: ("mfma_f32_32x32x2_f32", 2 * 32 * 32 * 2, 157.3),
           4: ("mfma_i32_16x16x64_i8", 2 * 16 * 16 * 64, 5000.0)}
    iters = 4096
    for op, (name, flop, peak) in ops.items():
        res = {}
        for grid in (256, 512, 1024):                     # 8 waves per workgroup: 2, 4, 8 waves per SIMD
            us = graph_us(torch, [lambda: lib.qmm_roof_mfma(op, iters, grid, ctypes.c_void_p(sink.data_ptr()), st())], reps=3)
            tf = grid * 8 * iters * 4 * flop / us / 1e6
            res[f"waves_per_simd{grid * 8 // 1024}"] = round(tf, 1)
        res["best_TFLOPS"] = max(res.values())
        res["pct_of_peak"] = round(100 * res["best_TFLOPS"] / peak, 1)
        out[name] = res
    # LDS read rate: one workgroup per CU, 4 / 8 / 16 waves; bytes per CU per second, and per clock at the
    # nominal 2.4 GHz
    res = {}
    iters, cus = 2000, 256
    for waves in (4, 8, 16):
        us = graph_us(torch, [lambda: lib.qmm_roof_lds(waves, iters, cus, ctypes.c_void_p(sink.data_ptr()), st())], reps=3)
        per_cu = iters * 16 * 1024 * waves / us / 1e3          # GB/s per CU
        res[f"waves{waves}"] = {"TB_s": round(per_cu * cus / 1e3, 1), "B_per_clk_per_CU_at_2.4GHz": round(per_cu / 2.4, 1)}
    out["lds_read_b128"] = res
    return out


def capture(torch, launches):
    """One HIP graph holding the given launch closures, in order, on a side stream."""
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        launches[0]()           # first launch outside capture (library load, lazy init)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        for f in launches:
            f()
    return g


def timed_replay(torch, g):
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def q4k_gemv_m1(args):
    import torch
    from hipster_amd import qmm, synth

    N, K = synth.CFG0["N"], synth.CFG0["K"]
    W = synth.matrix(synth.SEEDS["cfg0"], synth.Q4_K, N, K)
    x = synth.normal_f32(synth.SEEDS["cfg0"] + 1, (1, K))
    ncopy = max(2, -(-ROTATE_BYTES // W.nbytes))
    Wt = torch.from_numpy(W)
    Wd = [Wt.to("cuda") for _ in range(ncopy)]
    xd = torch.from_numpy(x).to("cuda")
    y = torch.zeros((1, N), dtype=torch.float32, device="cuda")
    xb = qmm.XQ8Buf(1, K)
    algo_bytes = W.nbytes + K * 4 + N * 4            # 50,225,152 B

    def step(i):       # the whole step: f32 x in, q8 quantisation fused into the GEMV, y out
        return lambda: qmm.gemv_q8_f32x(synth.Q4_K, Wd[i % ncopy], xd, y, N, K, 1)

    def two_launch(i):  # the same result as quantize_x_q8 + gemv_q8 (two launches)
        def f():
            qmm.quantize_x_q8(xd, xb, 1, K)
            qmm.gemv_q8(synth.Q4_K, Wd[i % ncopy], xb, y, N, K, 1)
        return f

    # the timed rotation starts past the copies the warm-up streamed, so no timed launch finds its weights
    # left in the last-level cache by the warm-up
    g_warm = capture(torch, [step(i) for i in range(args.warmup)])
    g_step = capture(torch, [step(args.warmup + i) for i in range(args.steps)])
    g_two = capture(torch, [two_launch(i) for i in range(args.steps)])
    timed_replay(torch, g_warm)
    ms_step = timed_replay(torch, g_step) / args.steps
    timed_replay(torch, g_two)
    ms_two = timed_replay(torch, g_two) / args.steps
    return dict(N=N, K=K, W=W, x=x, ncopy=ncopy, algo_bytes=algo_bytes, ms_step=ms_step, ms_kernel=ms_step, ms_two=ms_two)


def graph_us(torch, fns, reps=5):
    """Average microseconds of one pass over fns (a list of launch closures), graph replay."""
    g = capture(torch, [f for _ in range(reps) for f in fns])
    timed_replay(torch, g)
    return timed_replay(torch, g) / reps * 1e3


def extra_formats(torch):
    """The other weight formats of the call surface at config 0's shape (17408 x 5120), q8 GEMV at M = 1
    and 4, weights rotated over >= 1 GiB: time per call and weight bytes / time."""
    from hipster_amd import qmm, synth
    N, K = synth.CFG0["N"], synth.CFG0["K"]
    out = {}
    for name, fmt in (("Q4_K", synth.Q4_K), ("Q5_K", synth.Q5_K), ("IQ4_XS", synth.IQ4_XS), ("Q6_K_SOA", synth.Q6_K_SOA),
                      ("Q8_0_SOA", synth.Q8_0_SOA), ("Q5_1_SOA", synth.Q5_1_SOA)):
        W = synth.matrix(synth.SEEDS["cfg0"] + 50 + fmt, fmt, N, K)
        ncopy = max(2, -(-ROTATE_BYTES // W.nbytes))
        Wt = torch.from_numpy(W)
        Wd = [Wt.to("cuda") for _ in range(ncopy)]
        r = {"row_bytes": int(W.shape[1])}
        for M in (1, 4):
            xb = qmm.XQ8Buf(M, K)
            qmm.quantize_x_q8(torch.randn((M, K), device="cuda"), xb, M, K)
            y = torch.zeros((M, N), device="cuda")
            us = graph_us(torch, [(lambda i: (lambda: qmm.gemv_q8(fmt, Wd[i], xb, y, N, K, M)))(i) for i in range(ncopy)],
                          reps=2) / ncopy
            r[f"M{M}"] = {"us": round(us, 2), "GB_s": round(W.nbytes / us / 1e3, 1)}
        out[name] = r
        if fmt == synth.Q4_K:      # the reference's f32-x GEMV (gemv_q4_K_f32) on the same weights
            rf = {}
            for M in (1, 4):
                x = torch.randn((M, K), device="cuda")
                y = torch.zeros((M, N), device="cuda")
                us = graph_us(torch, [(lambda i: (lambda: qmm.gemv_q4_K_f32(Wd[i], x, y, N, K, M)))(i) for i in range(ncopy)],
                              reps=2) / ncopy
                rf[f"M{M}"] = {"us": round(us, 2), "GB_s": round(W.nbytes / us / 1e3, 1)}
            out["Q4_K_gemv_q4_K_f32"] = rf
        del Wd, Wt
        torch.cuda.empty_cache()
    return out


def extra_act(torch):
    """The producers of the matmul inputs at the dense model's shapes (hidden 5120, ffn 17408), decode
    (T = 1) and prefill (T = 2048): time per call and algorithmic bytes / time (x, y, x written back,
    w, the outputs; rows rotated so that a prefill call does not re-read what the last one left in L2)."""
    from hipster_amd import qmm
    n, F = 5120, 17408
    out = {}
    for T in (1, 2048):
        nrot = 1 if T > 1 else 64
        xs = [torch.randn((T, n), device="cuda") for _ in range(nrot)]
        ys = [torch.randn((T, n), device="cuda") * 1e-3 for _ in range(nrot)]
        w = torch.randn(n, device="cuda")
        xn = torch.empty((T, n), device="cuda")
        xq = qmm.XQ8Buf(T, n)
        xb = torch.empty((T, n), dtype=torch.int16, device="cuda")
        us = graph_us(torch, [(lambda i: (lambda: qmm.add_rmsnorm_quant(xs[i], ys[i], w, xn, xq, T, n, 1e-6)))(i)
                              for i in range(nrot)], reps=4) / nrot
        nbytes = T * n * (4 + 4 + 4 + 4 + 1) + T * (n // 32) * 8 + n * 4
        out[f"add_rmsnorm_quant_T{T}"] = {"us": round(us, 2), "GB_s": round(nbytes / us / 1e3, 1)}
        us = graph_us(torch, [(lambda i: (lambda: qmm.add_rmsnorm_bf16(xs[i], ys[i], w, xb, T, n, 1e-6)))(i)
                              for i in range(nrot)], reps=4) / nrot
        nbytes = T * n * (4 + 4 + 4 + 2) + n * 4
        out[f"add_rmsnorm_bf16_T{T}"] = {"us": round(us, 2), "GB_s": round(nbytes / us / 1e3, 1)}
        del xs, ys, xn, xq, xb
        m = T * F
        g = torch.randn(m, device="cuda"); u = torch.randn(m, device="cuda")
        hq = qmm.XQ8Buf(1, m)
        hb = torch.empty(m, dtype=torch.int16, device="cuda")
        us = graph_us(torch, [lambda: qmm.silu_mul_quant(g, u, hq, m)], reps=20)
        out[f"silu_mul_quant_T{T}"] = {"us": round(us, 2), "GB_s": round((m * 9 + m // 32 * 8) / us / 1e3, 1)}
        us = graph_us(torch, [lambda: qmm.silu_mul_bf16(g, u, hb, m)], reps=20)
        out[f"silu_mul_bf16_T{T}"] = {"us": round(us, 2), "GB_s": round(m * 10 / us / 1e3, 1)}
        del g, u, hq, hb
        torch.cuda.empty_cache()
    return out


def extra_router(torch):
    """The MoE router matmul (f32, 513 x hidden 2048 as config 2) and the router + routing call at
    decode batch sizes, router copies rotated beyond one XCD's L2: time per call and W bytes / time."""
    from hipster_amd import qmm
    K, N, R = 2048, 513, 8
    Ws = [torch.randn((N, K), device="cuda") * 0.05 for _ in range(R)]
    out = {}
    for T in (1, 4, 8):
        x = torch.randn((T, K), device="cuda")
        lg = torch.zeros((T, N), device="cuda")
        ids = torch.zeros((T, 11), dtype=torch.int32, device="cuda")
        w = torch.zeros((T, 11), device="cuda")
        us = graph_us(torch, [(lambda i: (lambda: qmm.f32_gemv(Ws[i], x, lg, N, K, T)))(i) for i in range(R)], reps=4) / R
        us2 = graph_us(torch, [(lambda i: (lambda: qmm.moe_router(Ws[i], x, lg, ids, w, T, 512, K, 10)))(i) for i in range(R)],
                       reps=4) / R
        out[f"T{T}"] = {"f32_gemv_us": round(us, 2), "GB_s": round(N * K * 4 / us / 1e3, 1), "router_and_route_us": round(us2, 2)}
    # the prefill router GEMM (BlasLt::gemm_f32): a 2048-token chunk, hidden 2048 (config 4) and 2560
    for Kp in (2048, 2560):
        Wp = [torch.randn((N, Kp), device="cuda") * 0.05 for _ in range(4)]
        A = torch.randn((2048, Kp), device="cuda")
        D = torch.zeros((2048, N), device="cuda")
        us = graph_us(torch, [(lambda i: (lambda: qmm.gemm_f32(A, Wp[i], D, 2048, N, Kp)))(i) for i in range(4)], reps=4) / 4
        out[f"gemm_f32_2048x513x{Kp}"] = {"us": round(us, 2), "TFLOPS": round(2 * 2048 * N * Kp / us / 1e6, 1)}
        del Wp, A, D
    return out


def extra_cfg1(torch):
    """one dense decode layer (gate+up Q4_K 2x17408x5120, down Q6_K 5120x17408 (SoA),
    QKV Q4_K 8192x5120, O Q4_K 5120x6144) at M = 1, 4, 8, weights rotated over >= 1 GiB."""
    from hipster_amd import qmm, synth
    # the down projection in the engine's GEMV layout: Q6_K rows repacked to SoA at load time
    # (engine/kernels/gemv.h:15, gemv.hip:1341-1350)
    sh = dict(gate=(synth.Q4_K, 17408, 5120), up=(synth.Q4_K, 17408, 5120), down=(synth.Q6_K_SOA, 5120, 17408),
              qkv=(synth.Q4_K, 8192, 5120), o=(synth.Q4_K, 5120, 6144))
    host = {k: synth.matrix(synth.SEEDS["cfg1"] + i, *v) for i, (k, v) in enumerate(sh.items())}
    layer_bytes = sum(a.nbytes for a in host.values())
    ncopy = max(2, -(-ROTATE_BYTES // layer_bytes))
    copies = [{k: torch.from_numpy(a).cuda() for k, a in host.items()} for _ in range(ncopy)]
    out = {"layer_weight_bytes": layer_bytes}
    for M in (1, 4, 8):
        xs = {K: qmm.XQ8Buf(M, K) for K in (5120, 17408, 6144)}
        for K, xb in xs.items():
            qmm.quantize_x_q8(torch.randn((M, K), device="cuda"), xb, M, K)
        ys = {k: torch.zeros((M, v[1]), device="cuda") for k, v in sh.items()}

        def layer(c):
            def f():
                W = copies[c]
                qmm.gemv_multi([(synth.Q4_K, W["gate"], ys["gate"], 17408, 5120), (synth.Q4_K, W["up"], ys["up"], 17408, 5120)],
                               xs[5120], M)
                qmm.gemv_q8(synth.Q6_K_SOA, W["down"], xs[17408], ys["down"], 5120, 17408, M)
                qmm.gemv_q8(synth.Q4_K, W["qkv"], xs[5120], ys["qkv"], 8192, 5120, M)
                qmm.gemv_q8(synth.Q4_K, W["o"], xs[6144], ys["o"], 5120, 6144, M)
            return f
        us = graph_us(torch, [layer(c) for c in range(ncopy)], reps=2) / ncopy
        out[f"M{M}"] = {"us_per_layer": round(us, 1), "GB_s": round(layer_bytes / us / 1e3, 1)}
    return out


def moe_tables(torch, keep_host=False):
    """512 Q4_K experts (gate, up [512][F][H], down [512][H][F]) + the shared expert, on the device;
    with keep_host the host arrays too (under "host", for the CPU legs)."""
    from hipster_amd import synth
    H, F, n_exp = 2048, 512, 512
    hst = dict(Wg=synth.experts(synth.SEEDS["cfg4"], synth.Q4_K, n_exp, F, H),
               Wu=synth.experts(synth.SEEDS["cfg4"] + 1, synth.Q4_K, n_exp, F, H),
               Wd=synth.experts(synth.SEEDS["cfg4"] + 2, synth.Q4_K, n_exp, H, F),
               Sg=synth.matrix(synth.SEEDS["cfg4"] + 10, synth.Q4_K, F, H),
               Su=synth.matrix(synth.SEEDS["cfg4"] + 11, synth.Q4_K, F, H),
               Sd=synth.matrix(synth.SEEDS["cfg4"] + 12, synth.Q4_K, H, F))
    tb = {k: torch.from_numpy(v).cuda() for k, v in hst.items()}
    if keep_host:
        tb["host"] = hst
    return tb


def extra_cfg2(torch, tb):
    """MoE decode step (route, gate|up gather GEMV, silu*up q8, down + combine)
    at T = 1, 4, 8 over 512 Q4_K experts + shared; each replayed step routes different logits.  The step
    is qmm_moe_decode (two launches); the four-launch sequence it replaces is timed beside it."""
    import numpy as np
    from hipster_amd import qmm, synth
    H, F, NE = 2048, 512, 11
    per_expert = 3 * tb["Wg"][0].numel()
    out = {"bytes_per_expert": per_expert}
    for T in (1, 4, 8):
        R = 16
        lg = [torch.from_numpy(synth.router_logits(synth.SEEDS["cfg2"] + 100 * T + r, T, 512)).cuda() for r in range(R)]
        xb = qmm.XQ8Buf(T, H)
        qmm.quantize_x_q8(torch.randn((T, H), device="cuda"), xb, T, H)
        ids = [torch.zeros((T, NE), dtype=torch.int32, device="cuda") for _ in range(R)]
        w = [torch.zeros((T, NE), device="cuda") for _ in range(R)]
        g = torch.zeros((T * NE, F), device="cuda"); u = torch.zeros((T * NE, F), device="cuda")
        hq = qmm.XQ8Buf(T * NE, F)
        y = torch.zeros((T, H), device="cuda")

        def step(r):
            def f():
                qmm.moe_route(lg[r], ids[r], w[r], T)
                qmm.gemv_moe(synth.Q4_K, synth.Q4_K, [tb["Wg"], tb["Wu"]], [tb["Sg"], tb["Su"]], [g, u], tb["Wg"][0].numel(),
                             ids[r], NE, xb, F, H, T, False)
                qmm.moe_silu_quant(g, u, hq, T * NE, F)
                qmm.gemv_moe(synth.Q4_K, synth.Q4_K, [tb["Wd"]], [tb["Sd"]], [y], tb["Wd"][0].numel(), ids[r], NE, hq, H, F, T,
                             True, slotw=w[r])
            return f
        us4 = graph_us(torch, [step(r) for r in range(R)], reps=2) / R
        ws = torch.zeros(qmm.moe_decode_ws_bytes(T, 10, F) // 4, device="cuda")
        y2 = torch.zeros((T, H), device="cuda")

        def fused(r):      # the same step in two launches (routing at T = 1, gate|up and silu -> q8; then down + combine)
            return lambda: qmm.moe_decode(synth.Q4_K, tb["Wg"], tb["Wu"], tb["Wd"], tb["Wg"][0].numel(), tb["Wd"][0].numel(), tb["Sg"],
                                          tb["Su"], tb["Sd"], lg[r], 513, 512, 10, xb, T, H, F, ids[r], w[r], ws, y2)
        us = graph_us(torch, [fused(r) for r in range(R)], reps=2) / R
        distinct = float(np.mean([len(np.unique(i.cpu().numpy())) for i in ids]))   # includes the shared slot (-1)
        byts = distinct * per_expert
        out[f"T{T}"] = {"us_per_step": round(us, 1), "four_launch_us_per_step": round(us4, 1),
                        "distinct_experts_incl_shared": distinct, "GB_s": round(byts / us / 1e3, 1)}
    return out


def extra_cfg3(torch):
    """dense prefill GEMM 2048 x 5120 -> 17408 (bf16 A, Q4_K W, f32 D) and the
    M = 3..6 verify GEMVs on the same weight."""
    from hipster_amd import qmm, synth
    M, N, K = synth.CFG3["M"], synth.CFG3["N"], synth.CFG3["K"]
    W = torch.from_numpy(synth.matrix(synth.SEEDS["cfg3"], synth.Q4_K, N, K)).cuda()
    A = torch.randn((M, K), device="cuda").to(torch.bfloat16)
    D = torch.zeros((M, N), device="cuda")
    us = graph_us(torch, [lambda: qmm.gemm_wq(synth.Q4_K, W, A, D, M, N, K)], reps=5)
    flop = 2 * M * N * K
    out = {"gemm_us": round(us, 1), "TFLOPS": round(flop / us / 1e6, 1), "pct_bf16_peak": round(100 * flop / us / 1e6 / 2500, 1)}
    ncopy = max(2, -(-ROTATE_BYTES // W.numel()))
    Ws = [W] + [W.clone() for _ in range(ncopy - 1)]
    for m in synth.CFG3["verify_M"]:
        xb = qmm.XQ8Buf(m, K)
        qmm.quantize_x_q8(torch.randn((m, K), device="cuda"), xb, m, K)
        y = torch.zeros((m, N), device="cuda")
        us = graph_us(torch, [(lambda c=c: qmm.gemv_q8(synth.Q4_K, Ws[c], xb, y, N, K, m)) for c in range(ncopy)], reps=2) / ncopy
        out[f"verify_M{m}_us"] = round(us, 2)
    return out


def extra_cfg4(torch, tb):
    """MoE prefill at 2048 tokens (route, device sort, grouped gate/up GEMM with the
    silu -> bf16 epilogue, grouped down GEMM, combine) with the Zipf-biased routing."""
    import numpy as np
    from hipster_amd import qmm, synth
    H, F, NE, T = 2048, 512, 11, 2048
    x = torch.randn((T, H), device="cuda").to(torch.bfloat16)
    logits = torch.from_numpy(synth.router_logits(synth.SEEDS["cfg4"], T, 512, 1.1)).cuda()
    NS = T * NE
    cap = qmm.moe_tiles_capacity(T, NE, 512)
    ids = torch.zeros((T, NE), dtype=torch.int32, device="cuda"); w = torch.zeros((T, NE), device="cuda")
    kpos = torch.zeros(NS, dtype=torch.int32, device="cuda"); rowtok = torch.zeros(NS, dtype=torch.int32, device="cuda")
    tiles = torch.zeros((cap, 3), dtype=torch.int32, device="cuda"); counts = torch.zeros(2, dtype=torch.int32, device="cuda")
    h = torch.zeros((NS, F), dtype=torch.bfloat16, device="cuda")
    dn = torch.zeros((NS, H), device="cuda"); y = torch.zeros((T, H), device="cuda")
    ebg, ebd = tb["Wg"][0].numel(), tb["Wd"][0].numel()
    route = [lambda: qmm.moe_route(logits, ids, w, T),
             lambda: qmm.moe_sort(ids, T, NE, 512, qmm.MOE_TILE_ROWS, kpos, rowtok, tiles, counts)]
    gemms = [lambda: qmm.moe_gemm_gate_up_bf16(0, 0, tb["Wg"], tb["Sg"], tb["Wu"], tb["Su"], ebg, tiles, counts, cap, rowtok,
                                               x, h, F, H),
             lambda: qmm.moe_gemm_bf16(0, 0, tb["Wd"], tb["Sd"], ebd, tiles, counts, cap, None, h, dn, H, F)]
    comb = [lambda: qmm.moe_combine_sorted(dn, w, kpos, y, T, NE, H)]
    us_all = graph_us(torch, route + gemms + comb, reps=3)
    us_g = graph_us(torch, gemms, reps=3)
    us_gu = graph_us(torch, gemms[:1], reps=3)
    us_dn = graph_us(torch, gemms[1:], reps=3)
    flop = 141733920768       # routed 2*20480*3*512*2048 + shared 2*2048*3*512*2048
    c = counts.cpu().numpy()
    out = {"pipeline_us": round(us_all, 1), "grouped_gemms_us": round(us_g, 1), "gate_up_silu_us": round(us_gu, 1),
           "down_us": round(us_dn, 1), "TFLOPS": round(flop / us_g / 1e6, 1),
           "pct_bf16_peak": round(100 * flop / us_g / 1e6 / 2500, 1), "tiles": [int(c[0]), int(c[1])],
           "distinct_experts_incl_shared": int(len(np.unique(ids.cpu().numpy())))}
    # the reference's own prefill call (qwen4exp.cpp:647-650): moe_gemm with q8 activations (gate, up, down
    # as three calls), host tile counts, tiles of at most 16 ct columns; the int8 matrix-core kernel
    xb = qmm.XQ8Buf(T, H)
    qmm.quantize_x_q8(x.float(), xb, T, H)
    hb = qmm.XQ8Buf(NS, F)
    qmm.quantize_x_q8(torch.randn((NS, F), device="cuda"), hb, NS, F)
    g = torch.zeros((NS, F), device="cuda")
    del h
    for ct in (1, 3):
        maxc = 16 * ct
        capq = qmm.moe_tiles_capacity(T, NE, 512, maxc)
        tq = torch.zeros((capq, 3), dtype=torch.int32, device="cuda")
        qmm.moe_sort(ids, T, NE, 512, maxc, kpos, rowtok, tq, counts)
        nt, nst = [int(v) for v in counts.cpu()]
        st = tq[nt:]
        q8 = [lambda: qmm.moe_gemm(0, 0, tb["Wg"], tb["Sg"], ebg, tq, nt, st, nst, ct, rowtok, xb, g, F, H),
              lambda: qmm.moe_gemm(0, 0, tb["Wu"], tb["Su"], ebg, tq, nt, st, nst, ct, rowtok, xb, g, F, H),
              lambda: qmm.moe_gemm(0, 0, tb["Wd"], tb["Sd"], ebd, tq, nt, st, nst, ct, None, hb, dn, H, F)]
        us_q = graph_us(torch, q8, reps=3)
        out[f"q8_moe_gemm_ct{ct}"] = {"us": round(us_q, 1), "TOPS": round(flop / us_q / 1e6, 1),
                                      "pct_int8_peak": round(100 * flop / us_q / 1e6 / 5000, 2), "tiles": [nt, nst]}
    return out


def extra_moe_uniform(torch):
    """The gate/up grouped GEMM (with silu) on uniform 128-row tiles: 16 Q4_K experts of 1,280 rows each
    (160 tiles), K = 2048, N = 2 x 512 -- the full-tile case of config 4 on its own, four launches."""
    from hipster_amd import qmm, synth
    H, F, T = 2048, 512, 2048
    Wg = torch.from_numpy(synth.experts(5, synth.Q4_K, 16, F, H)).cuda()
    Wu = torch.from_numpy(synth.experts(6, synth.Q4_K, 16, F, H)).cuda()
    x = torch.randn((T, H), device="cuda").to(torch.bfloat16)
    tiles = torch.tensor([[i // 10, 128 * i, 128] for i in range(160)], dtype=torch.int32, device="cuda")
    counts = torch.tensor([160, 0], dtype=torch.int32, device="cuda")
    rowtab = (torch.arange(20480, dtype=torch.int32, device="cuda") % T).contiguous()
    h = torch.zeros((20480, F), dtype=torch.bfloat16, device="cuda")
    gu = lambda: qmm.moe_gemm_gate_up_bf16(0, 0, Wg, Wg[0], Wu, Wu[0], Wg[0].numel(), tiles, counts, 160, rowtab, x, h, F, H)
    us = graph_us(torch, [gu], reps=4)
    flop = 2 * 20480 * 1024 * 2048
    return {"gate_up_us": round(us, 1), "TFLOPS": round(flop / us / 1e6, 1), "tiles": 160, "rows_per_tile": 128}


def host_threads():
    """All host cores this process may use, capped by the box's CPU share (OMP_NUM_THREADS, at most 16)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    try:
        cap = int(os.environ.get("OMP_NUM_THREADS", "16"))
    except ValueError:
        cap = 16
    return max(1, min(n, cap, 16))


def timed_calls(fn, seconds):
    calls, t0 = 0, time.perf_counter()
    while True:
        fn()
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds and calls >= 2:
            return calls, el


def cpu_baseline_gemv(W, x, N, K, seconds):
    """The reference host path (bench_gemv.cpp:95-104: quant.h dequant_row + fp32 dot per row) on all
    host cores and on one, compiled from the reference's own quant.h (oracle/_ref, kind "reference");
    the oracle's restatement (kind "port") when that library was not built."""
    import oracle
    threads = host_threads()
    if oracle.ref_lib() is not None:
        kind, what = "reference", "reference quant.h dequant_row + f32 dot (oracle/_ref, ISA clones up to x86-64-v4)"
        run = lambda nt: oracle.ref_gemv_f32(12, W, N, K, x, nthreads=nt)
    else:
        kind, what = "port", "oracle qo_gemv_f32: per-row dequant_q4_K + f32 dot"
        run = lambda nt: oracle.gemv_f32(0, W, N, K, x, nthreads=nt)
    run(threads)                                   # warm up code and pages
    byts = W.nbytes + K * 4 + N * 4
    calls, el = timed_calls(lambda: run(threads), seconds * 0.6)
    c1, e1 = timed_calls(lambda: run(1), seconds * 0.4)
    return dict(value=round(byts * calls / el / 1e9, 2), unit="GB/s", cores=threads, kind=kind,
                single_thread={"value": round(byts * c1 / e1 / 1e9, 3), "unit": "GB/s", "cores": 1},
                host_cpu_count=os.cpu_count(),
                sample=f"{calls} full calls of the 17408x5120 Q4_K GEMV at M=1 in {el:.1f} s on {threads} threads, "
                       f"{c1} in {e1:.1f} s on 1 (mean rates): {what}")


def cpu_moe_legs(tb, seconds):
    """CPU time of configs 2 and 4 on bounded samples, with the oracle's restatement of the reference's
    host MoE (kind "port"): routing (softmax + top-10), then per slot dequant . dot for gate, up and
    down and the slot-ordered combine; config 4 runs a sample of its 2048 tokens on all host cores."""
    import numpy as np
    import oracle
    from hipster_amd import synth
    hst = tb["host"]
    H, F = 2048, 512
    out = {}
    lg = synth.router_logits(synth.SEEDS["cfg2"] + 100, 1, 512)
    x = synth.normal_f32(synth.SEEDS["cfg2"] + 1, (1, H))

    def dec():
        ids, w = oracle.moe_route(lg, 512, 10)
        oracle.moe_decode(0, hst["Wg"], hst["Wu"], hst["Wd"], hst["Sg"], hst["Su"], hst["Sd"], x, ids, w, H, F)
    dec()
    calls, el = timed_calls(dec, seconds * 0.4)
    out["cfg2_T1"] = {"us_per_step": round(el / calls * 1e6, 1), "cores": 1, "kind": "port",
                      "sample": f"{calls} T=1 steps (route + 11 slots of gate/up/down + combine) in {el:.1f} s"}
    T, ntok = 2048, 64
    logits = synth.router_logits(synth.SEEDS["cfg4"], T, 512, 1.1)
    ids, w = oracle.moe_route(logits, 512, 10)
    xb = (synth.normal_f32(synth.SEEDS["cfg4"] + 5, (T, H)).view(np.uint32) >> 16).astype(np.uint16)
    toks = np.arange(0, T, T // ntok, dtype=np.int32)[:ntok]
    threads = host_threads()
    lgs = logits[toks]

    def pre():     # the sample's routing, then its slots (ids / w of the full batch are the same rows)
        oracle.moe_route(lgs, 512, 10)
        oracle.moe_prefill_tokens(0, hst["Wg"], hst["Wu"], hst["Wd"], hst["Sg"], hst["Su"], hst["Sd"], xb, ids, w, H, F, toks,
                                  nthreads=threads)
    calls, el = timed_calls(pre, seconds * 0.6)
    per_tok = el / calls / ntok
    out["cfg4_T2048"] = {"ms_per_step_est": round(per_tok * T * 1e3, 1), "cores": threads, "kind": "port",
                         "sample": f"{calls} passes over {ntok} of the 2048 tokens (every 32nd; route + per-slot "
                                   f"dequant . dot + combine) in {el:.1f} s, scaled to 2048 tokens"}
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: every box here has one MI355X, so --gpus {args.gpus} is not "
              "supported (the multi-GPU sharding of this path is a design note, not a measured configuration)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if args.calib_copy:
        calib_copy()
        return
    if args.roofs:
        print(json.dumps({"roofs": roofs(torch)}), flush=True)
        return
    if args.only_extra:
        fn = {"activation_producers": extra_act, "formats": extra_formats, "router": extra_router, "dense_decode": extra_cfg1,
              "moe_decode": lambda t: extra_cfg2(t, moe_tables(t)), "moe_prefill": lambda t: extra_cfg4(t, moe_tables(t)),
              "dense_prefill": extra_cfg3, "moe_uniform": extra_moe_uniform}[args.only_extra]
        print(json.dumps({args.only_extra: fn(torch)}), flush=True)
        return
    from hipster_amd import _lib
    _lib.lib()   # fails loudly if the HIP library is missing

    r = q4k_gemv_m1(args)
    kernel = "k_gemv_q4k_fx<1,5,256>"
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "q4k_gemv_m1_traffic.json")
    if os.path.exists(tfile):   # HBM bytes per launch from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes
        t = json.load(open(tfile))
        if t.get("kernel") == kernel:
            traffic = t.get("traffic_bytes")
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
        "config": {"workload": "cfg0: y = W x, x f32 [5120] quantised to q8 per 32 inside the Q4_K GEMV "
                               "(one launch, bit-identical to quantize_x_q8 + gemv_q8), M=1, W 17408x5120",
                   "N": r["N"], "K": r["K"], "M": 1, "algo_bytes_per_step": r["algo_bytes"],
                   "pct_of_hbm_peak": round(100 * gbs_step / HBM_PEAK_GBS, 1),
                   "two_launch_us_per_step": round(r["ms_two"] * 1e3, 3)},
        "roofline": {"bound": "hbm", "achieved": round(gbs_kernel, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs_kernel / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": kernel, "us_per_launch": round(r["ms_kernel"] * 1e3, 3)},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_gemv(r["W"], r["x"], r["N"], r["K"], args.cpu_seconds)
    if not args.no_extra:
        del r
        torch.cuda.empty_cache()
        extra = {"cfg1_dense_decode_layer": extra_cfg1(torch)}
        torch.cuda.empty_cache()
        tb = moe_tables(torch, keep_host=not args.no_cpu)
        extra["cfg2_moe_decode"] = extra_cfg2(torch, tb)
        extra["cfg4_moe_prefill"] = extra_cfg4(torch, tb)
        if not args.no_cpu:
            cpu = cpu_moe_legs(tb, args.cpu_seconds)
            extra["cfg2_moe_decode"]["cpu_baseline_T1"] = cpu["cfg2_T1"]
            extra["cfg4_moe_prefill"]["cpu_baseline"] = cpu["cfg4_T2048"]
        del tb
        torch.cuda.empty_cache()
        extra["cfg3_dense_prefill"] = extra_cfg3(torch)
        torch.cuda.empty_cache()
        extra["formats_gemv_17408x5120"] = extra_formats(torch)
        extra["activation_producers"] = extra_act(torch)
        extra["moe_router"] = extra_router(torch)
        out["extra"] = extra
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
