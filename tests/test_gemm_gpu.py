"""GPU parity of the prefill path: bit-exact dequantisation to bf16, the fused Q4_K GEMM and the
plain bf16 GEMM, through the C ABI.

Bars: dequant_bf16 bit-exact against the oracle (quant.h arithmetic, RNE to bf16), the golden
special blocks included; GEMM outputs within rel-L2 2e-3 (north star, bf16 MFMA path) of the
oracle's double-precision product of the same bf16 operands, checked on sampled (m, n) pairs at the
full BASELINE config-3 shape and on the whole matrix against a torch float32 reference."""
import numpy as np
import pytest
import torch

import oracle
from hipster_amd import qmm, synth
from tests.gpu_util import dev, host, rel_l2

pytestmark = pytest.mark.gpu
GOLD = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "quant_golden.npz"))
TOL = 2e-3


def bf16_dev(a_bits):
    return torch.from_numpy(np.ascontiguousarray(a_bits).view(np.int16)).cuda().view(torch.bfloat16)


@pytest.mark.parametrize("fmt,N,K", [(synth.Q4_K, 333, 5120), (synth.Q6_K, 129, 2048), (synth.Q6_K_SOA, 64, 4096),
                                     (synth.Q4_K, 17408, 5120), (synth.Q5_K, 300, 5120), (synth.IQ4_XS, 129, 2048),
                                     (synth.Q8_0_SOA, 77, 4096), (synth.Q5_1_SOA, 256, 2560), (synth.Q5_K, 4096, 17408)])
def test_dequant_bf16_bit_exact(gpu, fmt, N, K):
    W = synth.matrix(900 + N, fmt, N, K)
    out = torch.zeros((N, K), dtype=torch.int16, device="cuda")
    qmm.dequant_bf16(fmt, dev(W), out, N, K)
    ref = oracle.dequant_rows_bf16(fmt, W, K)
    assert np.array_equal(host(out).view(np.uint16), ref)


@pytest.mark.parametrize("fmt,key", [(synth.Q5_K, "q5k"), (synth.IQ4_XS, "iq4xs")])
def test_dequant_bf16_golden_blocks_other_formats(gpu, fmt, key):
    """GGUF blocks (edge blocks included) whose f32 values the reference's own quant.h wrote"""
    G = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "quant_golden_fmt.npz"))
    blocks = G[key + "_blocks"]
    out = torch.zeros((blocks.shape[0], 256), dtype=torch.int16, device="cuda")
    qmm.dequant_bf16(fmt, dev(blocks), out, blocks.shape[0], 256)
    assert np.array_equal(host(out).view(np.uint16), synth.to_bf16_bits(G[key + "_y"]))


@pytest.mark.parametrize("fmt,key", [(synth.Q4_K, "q4k"), (synth.Q6_K, "q6k")])
def test_dequant_bf16_golden_blocks(gpu, fmt, key):
    blocks = GOLD[key + "_blocks"]
    out = torch.zeros((blocks.shape[0], 256), dtype=torch.int16, device="cuda")
    qmm.dequant_bf16(fmt, dev(blocks), out, blocks.shape[0], 256)
    assert np.array_equal(host(out).view(np.uint16), synth.to_bf16_bits(GOLD[key + "_y"]))


def gemm_check(M, N, K, seed, npairs=0):
    W = synth.matrix(seed, synth.Q4_K, N, K)
    A = synth.to_bf16_bits(synth.normal_f32(seed + 1, (M, K)))
    D = torch.full((M, N), float("nan"), device="cuda")
    Wd, Ad = dev(W), bf16_dev(A)
    qmm.gemm_wq(synth.Q4_K, Wd, Ad, D, M, N, K)
    Dh = host(D)
    assert np.isfinite(Dh).all()
    # full matrix against torch float32 on the exactly dequantised bf16 weights
    Wb = torch.zeros((N, K), dtype=torch.int16, device="cuda")
    qmm.dequant_bf16(synth.Q4_K, Wd, Wb, N, K)
    ref = torch.matmul(Ad.float(), Wb.view(torch.bfloat16).float().t().contiguous())
    err = rel_l2(Dh, host(ref))
    print(f"gemm_wq M={M} N={N} K={K} rel-L2 vs torch fp32 {err:.2e}", flush=True)
    assert err <= TOL
    if npairs:
        g = synth.rng(seed + 2)
        ms, ns = g.integers(0, M, npairs).astype(np.int32), g.integers(0, N, npairs).astype(np.int32)
        o = np.argsort(ns, kind="stable")
        ms, ns = ms[o], ns[o]
        r = oracle.gemm_wq_ref(synth.Q4_K, W, A, M, N, K, ms, ns)
        e2 = rel_l2(Dh[ms, ns], r)
        print(f"  sampled vs oracle rel-L2 {e2:.2e}", flush=True)
        assert e2 <= TOL


@pytest.mark.parametrize("M,N,K", [(256, 128, 256), (300, 200, 512), (37, 1000, 2048), (513, 129, 5120)])
def test_gemm_wq_small_and_ragged(gpu, M, N, K):
    gemm_check(M, N, K, 1300 + M, npairs=64)


@pytest.mark.parametrize("M,N,K", [(2048, 8548, 512), (300, 40000, 256)])
def test_gemm_wq_split_last_round(gpu, M, N, K):
    """shapes whose last round of 256 x 256 tiles would be thin: the trailing columns (ragged) go to
    the grouped kernel's implicit row tiles (ragged M too); the whole D is checked"""
    gemm_check(M, N, K, 1350 + M, npairs=64)


def test_gemm_wq_config3_full_shape(gpu):
    gemm_check(2048, 17408, 5120, synth.SEEDS["cfg3"], npairs=256)


@pytest.mark.parametrize("M,N,K", [(256, 128, 64), (300, 515, 640), (2048, 2048, 2048), (129, 384, 192)])
def test_gemm_bf16(gpu, M, N, K):
    """K % 128 == 0 runs the two-waves-per-SIMD kernel with bf16 rows as its W source, other K the
    4-wave kernel"""
    A = synth.to_bf16_bits(synth.normal_f32(70 + M, (M, K)))
    W = synth.to_bf16_bits(synth.normal_f32(71 + N, (N, K)))
    D = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
    Ad, Wd = bf16_dev(A), bf16_dev(W)
    qmm.gemm_bf16(Ad, Wd, D, M, N, K)
    ref = torch.matmul(Ad.float(), Wd.float().t().contiguous())
    assert rel_l2(host(D.float()), host(ref)) <= 4e-3      # bf16 output rounding (2^-9) dominates


@pytest.mark.parametrize("fmt,M,N,K", [(synth.Q5_K, 300, 515, 512), (synth.IQ4_XS, 128, 256, 256),
                                         (synth.Q8_0_SOA, 257, 300, 640), (synth.Q5_1_SOA, 100, 1000, 128),
                                         (synth.Q5_K, 2048, 2048, 2048), (synth.Q5_1_SOA, 513, 2560, 640),
                                         (synth.Q6_K_SOA, 300, 515, 512), (synth.Q6_K_SOA, 2048, 5120, 17408)])
def test_gemm_wq_other_formats(gpu, fmt, M, N, K):
    """the fused GEMM for the other formats (dequantisation exactly as qmm_dequant_bf16, in the kernel)
    against torch float32 of the same bf16 operands; the bar of the bf16 MFMA path, 2e-3 (measured
    errors ~1e-7: f32 accumulation of exact bf16 products)"""
    W = dev(synth.matrix(1450 + fmt + K, fmt, N, K))
    A = bf16_dev(synth.to_bf16_bits(synth.normal_f32(1451 + M, (M, K))))
    D = torch.full((M, N), float("nan"), device="cuda")
    qmm.gemm_wq(fmt, W, A, D, M, N, K)
    Wb = torch.zeros((N, K), dtype=torch.int16, device="cuda")
    qmm.dequant_bf16(fmt, W, Wb, N, K)
    ref = torch.matmul(A.float(), Wb.view(torch.bfloat16).float().t().contiguous())
    err = rel_l2(host(D), host(ref))
    print(f"gemm_wq fmt={fmt} M={M} N={N} K={K} rel-L2 {err:.2e}", flush=True)
    assert err <= 2e-3


@pytest.mark.parametrize("M,N,K", [(512, 512, 1024), (300, 768, 2048)])
def test_gemm_wq_q4k_is_the_bf16_gemm_of_its_dequantisation(gpu, M, N, K):
    """the fused Q4_K GEMM feeds the matrix cores exactly qmm_dequant_bf16's weights: rounded to bf16 its
    f32 output equals, bit for bit, the bf16 GEMM (the same kernel body and K order) on the dequantised
    rows"""
    W = dev(synth.matrix(1460 + N, synth.Q4_K, N, K))
    A = bf16_dev(synth.to_bf16_bits(synth.normal_f32(1461 + M, (M, K))))
    D = torch.full((M, N), float("nan"), device="cuda")
    qmm.gemm_wq(synth.Q4_K, W, A, D, M, N, K)
    Wb = torch.zeros((N, K), dtype=torch.int16, device="cuda")
    qmm.dequant_bf16(synth.Q4_K, W, Wb, N, K)
    Db = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
    qmm.gemm_bf16(A, Wb.view(torch.bfloat16), Db, M, N, K)
    assert np.array_equal(synth.to_bf16_bits(host(D)), host(Db.view(torch.int16)).view(np.uint16))


def test_gemm_deterministic(gpu):
    M, N, K = 512, 384, 1024
    W = dev(synth.matrix(1400, synth.Q4_K, N, K))
    A = bf16_dev(synth.to_bf16_bits(synth.normal_f32(1401, (M, K))))
    D1 = torch.zeros((M, N), device="cuda"); D2 = torch.zeros((M, N), device="cuda")
    qmm.gemm_wq(synth.Q4_K, W, A, D1, M, N, K)
    qmm.gemm_wq(synth.Q4_K, W, A, D2, M, N, K)
    assert torch.equal(D1, D2)


def test_bf16_helpers(gpu):
    x = synth.normal_f32(80, (33, 70))
    xb = torch.zeros(x.size, dtype=torch.int16, device="cuda")
    qmm.f32_to_bf16(dev(x), xb, x.size)
    assert np.array_equal(host(xb).view(np.uint16), synth.to_bf16_bits(x).ravel())
    back = torch.zeros(x.size, device="cuda")
    qmm.bf16_to_f32(xb, back, x.size)
    assert np.array_equal(host(back), synth.bf16_bits_to_f32(synth.to_bf16_bits(x)).ravel())
    seg = torch.zeros((33, 20), device="cuda")
    qmm.bf16_to_f32_seg2(xb, xb, 70, 30, 20, seg, 33)
    want = 2 * synth.bf16_bits_to_f32(synth.to_bf16_bits(x))[:, 30:50]
    assert np.array_equal(host(seg), want)
