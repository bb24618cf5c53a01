"""GPU parity of the q8 GEMV for the other formats of the call surface (Q5_K, IQ4_XS, Q8_0_SOA,
Q5_1_SOA -- hipster_amd/csrc/gemv_fmt.hip) against the CPU oracle, through the C ABI.

Bars as for Q4_K / Q6_K: against the same-math oracle (q8-rounded x,
weights dequantised by the reference's own formulas -- pinned bit for bit by
tests/test_oracle_formats.py --, double dot): rel-L2 <= 1e-5 and the reference validator's metric
max |ref - got| / sum |w x| < 1e-5 (bench_gemv.cpp:110-111); T-invariance (a column is bitwise the same
for every ncol) and run-to-run determinism; Q5_0 rows through the library's own repack into the Q5_1
SoA layout against the Q5_0 definition; gemv_multi over mixed formats equal to separate calls.
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


def run_q8(fmt, W, N, K, x, ncol):
    xb = q8_on_gpu(x[:ncol])
    y = torch.zeros((ncol, N), dtype=torch.float32, device="cuda")
    qmm.gemv_q8(fmt, dev(W), xb, y, N, K, ncol)
    return host(y)


def q8_reference(fmt, W, N, K, x):
    q, d, _ = oracle.quantize_x_q8(x)
    return oracle.gemv_ref(fmt, W, N, K, oracle.q8_to_f32(q, d))


SHAPES = [(synth.Q5_K, 17408, 5120), (synth.Q5_K, 777, 256), (synth.Q5_K, 130, 17408),
          (synth.IQ4_XS, 5120, 17408), (synth.IQ4_XS, 1001, 2048), (synth.IQ4_XS, 4096, 5120),
          (synth.Q8_0_SOA, 4096, 5120), (synth.Q8_0_SOA, 130, 17408), (synth.Q8_0_SOA, 63, 256),
          (synth.Q5_1_SOA, 2048, 5120), (synth.Q5_1_SOA, 65, 768), (synth.Q5_1_SOA, 515, 17408),
          # the engine's expert down projection, K = 640 (qwen4exp.h:22), and small K of 32-weight blocks
          (synth.Q5_1_SOA, 2048, 640), (synth.Q8_0_SOA, 2048, 640), (synth.Q5_1_SOA, 100, 96), (synth.Q8_0_SOA, 33, 192)]


@pytest.mark.parametrize("fmt,N,K", SHAPES)
def test_gemv_q8_formats_parity(gpu, fmt, N, K):
    W = synth.matrix(800 + N + K + fmt, fmt, N, K)
    x = synth.normal_f32(900 + K, (8, K))
    ref, mag = q8_reference(fmt, W, N, K, x)
    for ncol in (1, 3, 8):
        print(f"fmt={fmt} N={N} K={K} ncol={ncol}", flush=True)
        y = run_q8(fmt, W, N, K, x, ncol)
        assert rel_l2(y, ref[:ncol]) <= TOL
        assert max_rel_mag(y, ref[:ncol], mag[:ncol]) < TOL


@pytest.mark.parametrize("fmt", [synth.Q5_K, synth.IQ4_XS, synth.Q8_0_SOA, synth.Q5_1_SOA])
def test_gemv_q8_formats_t_invariant_and_deterministic(gpu, fmt):
    N, K = 1029, 5120
    W = synth.matrix(1100 + fmt, fmt, N, K)
    x = synth.normal_f32(1101, (8, K))
    Wd, xb = dev(W), q8_on_gpu(x)
    outs = {}
    for ncol in range(1, 9):
        y = torch.zeros((ncol, N), dtype=torch.float32, device="cuda")
        qmm.gemv_q8(fmt, Wd, xb, y, N, K, ncol)
        outs[ncol] = host(y)
    for ncol in range(2, 9):
        assert np.array_equal(outs[ncol][:ncol - 1].view(np.uint32), outs[ncol - 1].view(np.uint32)), ncol
    y2 = torch.zeros((8, N), dtype=torch.float32, device="cuda")
    qmm.gemv_q8(fmt, Wd, xb, y2, N, K, 8)
    assert np.array_equal(host(y2).view(np.uint32), outs[8].view(np.uint32))


def test_q5_0_rows_through_the_repack(gpu):
    """Q5_0 rows repacked by qmm_repack_row_q5_0 into the Q5_1 SoA layout (m = -16 d), then the Q5_1_SOA
    GEMV, against the oracle on the Q5_0 rows themselves (w = (q - 16) d)."""
    N, K = 300, 2048
    W = synth.matrix(1200, synth.Q5_0, N, K)
    soa = np.stack([qmm.repack_row_q5_0(W[r], K) for r in range(N)])
    x = synth.normal_f32(1201, (3, K))
    ref, mag = q8_reference(synth.Q5_0, W, N, K, x)
    y = run_q8(synth.Q5_1_SOA, soa, N, K, x, 3)
    assert rel_l2(y, ref) <= TOL and max_rel_mag(y, ref, mag) < TOL


def test_gemv_multi_mixed_formats_equals_separate_calls(gpu):
    K = 5120
    segs_np = [(synth.Q5_K, 1024), (synth.IQ4_XS, 512), (synth.Q8_0_SOA, 300), (synth.Q4_K, 128)]
    x = synth.normal_f32(1300, (4, K))
    xb = q8_on_gpu(x)
    segs, ref = [], []
    for i, (fmt, N) in enumerate(segs_np):
        W = dev(synth.matrix(1310 + i, fmt, N, K))
        y = torch.zeros((4, N), dtype=torch.float32, device="cuda")
        y1 = torch.zeros((4, N), dtype=torch.float32, device="cuda")
        qmm.gemv_q8(fmt, W, xb, y1, N, K, 4)
        segs.append((fmt, W, y, N, K)); ref.append(y1)
    qmm.gemv_multi(segs, xb, 4)
    for (_, _, y, _, _), y1 in zip(segs, ref):
        assert torch.equal(y, y1)


@pytest.mark.parametrize("ncol", [1, 3, 8, 12])
@pytest.mark.parametrize("layout", [((synth.Q5_K, 1024), (synth.Q5_K, 300), (synth.Q5_K, 17), (synth.IQ4_XS, 512)),
                                    ((synth.IQ4_XS, 700), (synth.IQ4_XS, 64), (synth.Q8_0_SOA, 256), (synth.Q8_0_SOA, 130)),
                                    ((synth.Q5_1_SOA, 96), (synth.Q5_1_SOA, 1000), (synth.Q5_1_SOA, 33), (synth.Q5_1_SOA, 512)),
                                    ((synth.Q6_K_SOA, 256), (synth.Q6_K_SOA, 100), (synth.Q4_K, 512), (synth.Q4_K, 48))])
def test_gemv_multi_same_format_runs(gpu, layout, ncol):
    """Runs of consecutive same-format segments go out as one launch per column pass; every segment's
    rows are bitwise its own gemv_q8 (the per-row arithmetic does not depend on the other segments)."""
    K = 5120
    print(f"gemv_multi runs {[f for f, _ in layout]} ncol={ncol}", flush=True)
    x = synth.normal_f32(1400 + ncol, (ncol, K))
    xb = q8_on_gpu(x)
    segs, ref = [], []
    for i, (fmt, N) in enumerate(layout):
        W = dev(synth.matrix(1410 + 7 * i + fmt, fmt, N, K))
        y = torch.full((ncol, N), float("nan"), dtype=torch.float32, device="cuda")
        y1 = torch.zeros((ncol, N), dtype=torch.float32, device="cuda")
        for c0 in range(0, ncol, 8):
            nc = min(8, ncol - c0)
            xc = qmm.XQ8Buf(nc, K)
            xc.q.copy_(xb.q[c0:c0 + nc]); xc.d.copy_(xb.d[c0:c0 + nc]); xc.s.copy_(xb.s[c0:c0 + nc])
            y1c = torch.zeros((nc, N), dtype=torch.float32, device="cuda")
            qmm.gemv_q8(fmt, W, xc, y1c, N, K, nc)
            y1[c0:c0 + nc] = y1c
        segs.append((fmt, W, y, N, K)); ref.append(y1)
    qmm.gemv_multi(segs, xb, ncol)
    for (_, _, y, _, _), y1 in zip(segs, ref):
        assert torch.equal(y, y1)


@pytest.mark.parametrize("fmt,K", [(synth.Q5_K, 5120), (synth.Q5_K, 17408), (synth.IQ4_XS, 5120), (synth.IQ4_XS, 2048),
                                   (synth.Q8_0_SOA, 5120), (synth.Q8_0_SOA, 640), (synth.Q5_1_SOA, 5120),
                                   (synth.Q5_1_SOA, 640), (synth.Q5_1_SOA, 96)])
def test_gemv_q8_formats_x_in_lds_equals_global(gpu, fmt, K):
    """x staged in LDS (ahead of the weights or before them, as the launcher picks per format and
    width) gives the same bits as x read from global memory, at every width 1..8 (knob
    qmm_set_gemv_fmt_xlds; K = 96 is not a multiple of 128 and always reads global x)."""
    from hipster_amd import _lib
    N = 1029
    W = synth.matrix(1200 + fmt + K, fmt, N, K)
    x = synth.normal_f32(1201 + K, (8, K))
    Wd, xb = dev(W), q8_on_gpu(x)
    L = _lib.lib()
    try:
        for ncol in range(1, 9):
            print(f"fmt={fmt} K={K} ncol={ncol}", flush=True)
            ys = []
            for on in (0, 1):
                L.qmm_set_gemv_fmt_xlds(on)
                y = torch.zeros((ncol, N), dtype=torch.float32, device="cuda")
                qmm.gemv_q8(fmt, Wd, xb, y, N, K, ncol)
                ys.append(host(y))
            assert np.array_equal(ys[0].view(np.uint32), ys[1].view(np.uint32)), ncol
    finally:
        L.qmm_set_gemv_fmt_xlds(1)
