"""GPU parity of the decode GEMV path against the CPU oracle, through the C ABI.

Bars:
  * x quantiser: bit-exact with the oracle (engine/bench/bench_gemv.cpp:17-25).
  * int8-activation GEMV: against the same-math oracle (q8-rounded x, double dot), rel-L2 <= 1e-5 and the
    reference validator's own metric max |ref-got| / sum|w*x| < 1e-5 (bench_gemv.cpp:110-111).
  * f32-activation Q4_K GEMV: against the f32-x oracle, rel-L2 <= 1e-5.
  * T-invariance (column c bitwise equal for ncol = 1 and ncol = k) and run-to-run determinism.
"""
import numpy as np
import pytest
import torch

import oracle
from hipster_amd import qmm, synth
from tests.gpu_util import dev, host, max_rel_mag, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-5


def q8_on_gpu(x):
    ncol, K = x.shape
    xb = qmm.XQ8Buf(ncol, K)
    qmm.quantize_x_q8(dev(x), xb, ncol, K)
    return xb


@pytest.mark.parametrize("ncol,K", [(1, 256), (3, 5120), (8, 17408), (2, 2048)])
def test_quantize_x_q8_bit_exact(gpu, ncol, K):
    x = synth.normal_f32(100 + K, (ncol, K))
    x[0, :32] = 0.0                                 # amax = 0 block
    x[-1, 32:64] = np.linspace(-3, 3, 32)           # exact ties after scaling are possible
    x[0, 64:96] *= 1e-30                            # tiny magnitudes
    xb = qmm.XQ8Buf(ncol, K, with_ds=True)
    qmm.quantize_x_q8(dev(x), xb, ncol, K)
    q, d, s = oracle.quantize_x_q8(x)
    assert np.array_equal(host(xb.q), q)
    assert np.array_equal(host(xb.d).view(np.uint32), d.view(np.uint32))
    assert np.array_equal(host(xb.s).view(np.uint32), s.view(np.uint32))
    ds = host(xb.ds)
    assert np.array_equal(ds[..., 0], d) and np.array_equal(ds[..., 1], s)


def run_q8(fmt, W, N, K, x, ncol):
    xb = q8_on_gpu(x[:ncol])
    y = torch.zeros((ncol, N), dtype=torch.float32, device="cuda")
    qmm.gemv_q8(fmt, dev(W), xb, y, N, K, ncol)
    return host(y)


def q8_reference(fmt, W, N, K, x):
    q, d, _ = oracle.quantize_x_q8(x)
    xr = oracle.q8_to_f32(q, d)
    return oracle.gemv_ref(fmt, W, N, K, xr)


SHAPES = [(synth.Q4_K, 17408, 5120), (synth.Q4_K, 1000, 256), (synth.Q4_K, 77, 2048), (synth.Q4_K, 5120, 17408),
          (synth.Q4_K, 8192, 5120), (synth.Q4_K, 5120, 6144),        # config 1: QKV 5120 -> 6144+1024+1024, O 6144 -> 5120
          (synth.Q6_K, 5120, 17408), (synth.Q6_K, 333, 5120), (synth.Q6_K, 64, 768),
          (synth.Q6_K_SOA, 5120, 17408), (synth.Q6_K_SOA, 129, 512)]


@pytest.mark.parametrize("fmt,N,K", SHAPES)
def test_gemv_q8_parity(gpu, fmt, N, K):
    W = synth.matrix(200 + N + K, fmt, N, K)
    x = synth.normal_f32(300 + K, (8, K))
    ref, mag = q8_reference(fmt, W, N, K, x)
    for ncol in (1, 3, 8):
        y = run_q8(fmt, W, N, K, x, ncol)
        print(f"fmt={fmt} N={N} K={K} ncol={ncol}", flush=True)
        assert rel_l2(y, ref[:ncol]) <= TOL
        assert max_rel_mag(y, ref[:ncol], mag[:ncol]) < TOL


@pytest.mark.parametrize("fmt,N,K", [(synth.Q4_K, 4099, 5120), (synth.Q6_K, 1031, 5120), (synth.Q6_K_SOA, 515, 2048),
                                     (synth.Q6_K_SOA, 5120, 17408), (synth.Q6_K, 1037, 17408)])
def test_gemv_q8_t_invariant_and_deterministic(gpu, fmt, N, K):
    """every column bitwise the same for ncol 1..8 (Q6_K from 5 columns on: all columns staged at once
    per 16-row workgroup, the config-1 down shape included)"""
    W = synth.matrix(400 + N, fmt, N, K)
    x = synth.normal_f32(401, (8, K))
    Wd = dev(W)
    xb = q8_on_gpu(x)
    outs = {}
    for ncol in range(1, 9):
        y = torch.zeros((ncol, N), dtype=torch.float32, device="cuda")
        qmm.gemv_q8(fmt, Wd, xb, y, N, K, ncol)
        outs[ncol] = host(y)
    # column 0 is the same for every ncol, and columns 0..ncol-2 of ncol equal those of ncol-1:
    # together every column c is bitwise the same for all ncol > c
    for ncol in range(2, 9):
        assert np.array_equal(outs[ncol][0].view(np.uint32), outs[1][0].view(np.uint32)), ncol
        assert np.array_equal(outs[ncol][:ncol - 1].view(np.uint32), outs[ncol - 1].view(np.uint32)), ncol
    y2 = torch.zeros((8, N), dtype=torch.float32, device="cuda")
    qmm.gemv_q8(fmt, Wd, xb, y2, N, K, 8)
    assert np.array_equal(host(y2).view(np.uint32), outs[8].view(np.uint32))


def test_gemv_q8_column_alone_equals_column_in_batch(gpu):
    N, K = 2051, 5120
    W = synth.matrix(500, synth.Q4_K, N, K)
    x = synth.normal_f32(501, (8, K))
    Wd = dev(W)
    y8 = run_q8(synth.Q4_K, W, N, K, x, 8)
    for c in (1, 5, 7):
        y1 = run_q8(synth.Q4_K, W, N, K, x[c:c + 1], 1)
        assert np.array_equal(y1[0].view(np.uint32), y8[c].view(np.uint32))


def test_gemv_multi_equals_separate_calls(gpu):
    K = 5120
    segs_np = [(synth.Q4_K, 1024), (synth.Q6_K, 512), (synth.Q4_K, 128)]
    x = synth.normal_f32(600, (4, K))
    xb = q8_on_gpu(x)
    segs, ref = [], []
    for i, (fmt, N) in enumerate(segs_np):
        W = dev(synth.matrix(610 + i, fmt, N, K))
        y = torch.zeros((4, N), dtype=torch.float32, device="cuda")
        y1 = torch.zeros((4, N), dtype=torch.float32, device="cuda")
        qmm.gemv_q8(fmt, W, xb, y1, N, K, 4)
        segs.append((fmt, W, y, N, K)); ref.append(y1)
    qmm.gemv_multi(segs, xb, 4)
    for (_, _, y, _, _), y1 in zip(segs, ref):
        assert torch.equal(y, y1)


@pytest.mark.parametrize("K", [5120, 17408, 768])
def test_gemv_multi_q4k_one_launch_equals_separate_calls(gpu, K):
    """all-Q4_K segments in one dot4 launch (ncol 1..3; ncol 17: a matrix-core pass of 16 columns, then the
    17th on the dot4 kernel) bitwise the separate one-segment calls; ragged row counts, K = 17408 takes the
    streamed long-row form"""
    Ns = [1000, 77, 4099, 16]
    x = synth.normal_f32(620, (17, K))
    xb = q8_on_gpu(x)
    Ws = [dev(synth.matrix(630 + i + K, synth.Q4_K, N, K)) for i, N in enumerate(Ns)]
    for ncol in (1, 2, 3, 17):
        print(f"gemv_multi q4k K={K} ncol={ncol}", flush=True)
        segs, ref = [], []
        for W, N in zip(Ws, Ns):
            y = torch.full((ncol, N), float("nan"), dtype=torch.float32, device="cuda")
            y1 = torch.zeros((ncol, N), dtype=torch.float32, device="cuda")
            for c0 in range(0, ncol, 8):
                nc = min(8, ncol - c0)
                xc = qmm.XQ8Buf(nc, K)
                xc.q.copy_(xb.q[c0:c0 + nc]); xc.d.copy_(xb.d[c0:c0 + nc]); xc.s.copy_(xb.s[c0:c0 + nc])
                qmm.gemv_q8(synth.Q4_K, W, xc, y1[c0:c0 + nc], N, K, nc)
            segs.append((synth.Q4_K, W, y, N, K)); ref.append(y1)
        qmm.gemv_multi(segs, xb, ncol)
        for (_, _, y, _, _), y1 in zip(segs, ref):
            assert np.array_equal(host(y).view(np.uint32), host(y1).view(np.uint32)), ncol


@pytest.mark.parametrize("N,K", [(17408, 5120), (999, 256), (4096, 2048), (77, 768), (300, 17408)])
def test_gemv_q4_K_f32_parity(gpu, N, K):
    """f32 x (the 1e-5 semantics of gemv.hip:1177-1216) against the oracle; column 0 is bitwise the
    same for every ncol (K = 17408 exercises the long-row kernel)"""
    W = synth.matrix(700 + N, synth.Q4_K, N, K)
    x = synth.normal_f32(701, (8, K))
    ref, mag = oracle.gemv_ref(synth.Q4_K, W, N, K, x)
    Wd = dev(W)
    col0 = None
    for ncol in (1, 2, 3, 4, 8):
        y = torch.zeros((ncol, N), dtype=torch.float32, device="cuda")
        qmm.gemv_q4_K_f32(Wd, dev(x[:ncol]), y, N, K, ncol)
        yh = host(y)
        print(f"f32x N={N} K={K} ncol={ncol} relL2={rel_l2(yh, ref[:ncol]):.2e}", flush=True)
        assert rel_l2(yh, ref[:ncol]) <= TOL
        assert max_rel_mag(yh, ref[:ncol], mag[:ncol]) < TOL
        if col0 is None:
            col0 = yh[0].copy()
        assert np.array_equal(yh[0].view(np.uint32), col0.view(np.uint32))


@pytest.mark.parametrize("N,K,ncol", [(17408, 5120, 1), (17408, 5120, 4), (1000, 256, 2), (77, 2048, 3), (333, 6144, 1),
                                      (5, 768, 4)])
def test_gemv_q8_f32x_equals_quantize_then_gemv(gpu, N, K, ncol):
    """the fused f32-x entry (quantisation inside the GEMV) is bit for bit quantize_x_q8 + gemv_q8"""
    W = synth.matrix(1300 + N, synth.Q4_K, N, K)
    x = synth.normal_f32(1301 + K, (ncol, K))
    x[0, :32] = 0.0                                 # amax = 0 block
    x[-1, 64:96] *= 1e-30                           # tiny magnitudes
    ref = run_q8(synth.Q4_K, W, N, K, x, ncol)
    y = torch.full((ncol, N), float("nan"), dtype=torch.float32, device="cuda")
    qmm.gemv_q8_f32x(synth.Q4_K, dev(W), dev(x), y, N, K, ncol)
    got = host(y)
    print(f"gemv_q8_f32x N={N} K={K} ncol={ncol}: {int((got.view(np.uint32) != ref.view(np.uint32)).sum())} differing", flush=True)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("N,K", [(17408, 5120), (16411, 512), (16384, 256), (16500, 4352), (20000, 6144), (16385, 768),
                                 (30000, 2048), (17000, 5120)])
def test_q4k_large_n_columns_and_fused_entry(gpu, N, K):
    """Large decode shapes over every pair-iteration class (K = 256 .. 6144) and ragged N: each column
    of ncol = 1..4 is bitwise the column of ncol = 5, the fused f32-x entry gives the same bits as
    quantize + gemv_q8, and column 0 matches the oracle."""
    W = synth.matrix(1500 + N + K, synth.Q4_K, N, K)
    x = synth.normal_f32(1501 + K, (5, K))
    Wd = dev(W)
    xb = q8_on_gpu(x)
    y5 = torch.zeros((5, N), dtype=torch.float32, device="cuda")
    qmm.gemv_q8(synth.Q4_K, Wd, xb, y5, N, K, 5)
    ref5 = host(y5)
    q, d, _ = oracle.quantize_x_q8(x[:1])
    ref, mag = oracle.gemv_ref(synth.Q4_K, W, N, K, oracle.q8_to_f32(q, d))
    assert rel_l2(ref5[:1], ref) <= TOL
    assert max_rel_mag(ref5[:1], ref, mag) < TOL
    for ncol in (1, 2, 3, 4):
        y = torch.full((ncol, N), float("nan"), dtype=torch.float32, device="cuda")
        qmm.gemv_q8(synth.Q4_K, Wd, xb, y, N, K, ncol)
        got = host(y)
        print(f"large-N q8 N={N} K={K} ncol={ncol}: {int((got.view(np.uint32) != ref5[:ncol].view(np.uint32)).sum())} differing", flush=True)
        assert np.array_equal(got.view(np.uint32), ref5[:ncol].view(np.uint32))
        yf = torch.full((ncol, N), float("nan"), dtype=torch.float32, device="cuda")
        qmm.gemv_q8_f32x(synth.Q4_K, Wd, dev(x[:ncol]), yf, N, K, ncol)
        assert np.array_equal(host(yf).view(np.uint32), ref5[:ncol].view(np.uint32))
