"""GPU parity of the router matmul (engine/kernels/fn.hip:251-277, fn::f32_gemv), of the router
matmul + routing call (qwen4exp.cpp:346-347) against the CPU oracle, and of the prefill router GEMM
(hip::BlasLt::gemm_f32, gemm.hip:162-186, called at qwen4exp.cpp:626), through the C ABI.

Bars: the decode logits bit-exact (the library computes them with the reference's lane partition, fma
contraction and summation tree, which the oracle restates); ids bit-exact apart from near-ties in p
that the device exp may decide (see assert_route_matches); weights within 1e-5.  The prefill GEMM's
order is the reference's hipBLASLt's, which nothing specifies: its bar is the f32-accumulation one,
rel-L2 <= 1e-5 against the float64 product and max |err| / sum_k |a w| < 1e-5 per output; the routing
of its logits is held bit-exact to the oracle's routing of the same logits.
"""
import numpy as np
import pytest
import torch

import oracle
from hipster_amd import qmm, synth
from tests.gpu_util import assert_route_matches, dev, host, rel_l2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,K,T", [(513, 2560, 1), (513, 2048, 8), (513, 2560, 13), (100, 2052, 3), (7, 4, 2),
                                   (513, 132, 9), (64, 1024, 64)])
def test_f32_gemv_bit_exact(gpu, N, K, T):
    print(f"f32_gemv N={N} K={K} T={T}", flush=True)
    W = synth.normal_f32(800 + K, (N, K)) * 0.05
    x = synth.normal_f32(801 + T, (T, K))
    y = torch.full((T, N), float("nan"), device="cuda")
    qmm.f32_gemv(dev(W), dev(x), y, N, K, T)
    ref = oracle.f32_gemv(W, x)
    got = host(y)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), int((got != ref).sum())


def test_f32_gemv_t_invariant(gpu):
    """A token's logits are the same bits alone and inside a batch of any size."""
    N, K = 513, 2048
    W = dev(synth.normal_f32(810, (N, K)) * 0.05)
    x = synth.normal_f32(811, (11, K))
    yb = torch.zeros((11, N), device="cuda")
    qmm.f32_gemv(W, dev(x), yb, N, K, 11)
    for t in (0, 7, 10):
        y1 = torch.zeros((1, N), device="cuda")
        qmm.f32_gemv(W, dev(x[t:t + 1]), y1, N, K, 1)
        assert torch.equal(y1[0], yb[t])


@pytest.mark.parametrize("T,K", [(1, 2048), (4, 2560), (8, 2048), (300, 2048)])
def test_moe_router(gpu, T, K):
    print(f"moe_router T={T} K={K}", flush=True)
    nexp = 512
    Wr = synth.normal_f32(820 + K, (nexp + 1, K)) * 0.05
    x = synth.normal_f32(821 + T, (T, K))
    logits = torch.zeros((T, nexp + 1), device="cuda")
    ids = torch.zeros((T, 11), dtype=torch.int32, device="cuda")
    w = torch.zeros((T, 11), device="cuda")
    qmm.moe_router(dev(Wr), dev(x), logits, ids, w, T, nexp, K, 10)
    lg_ref = oracle.f32_gemv(Wr, x)
    assert np.array_equal(host(logits).view(np.uint32), lg_ref.view(np.uint32))
    ids_ref, w_ref = oracle.moe_route(lg_ref, nexp, 10)
    assert_route_matches(host(ids), host(w), ids_ref, w_ref, lg_ref, nexp)


@pytest.mark.parametrize("M,N,K", [(2048, 513, 2560), (128, 513, 2048), (77, 130, 100), (1, 1, 4), (64, 64, 32),
                                   (65, 65, 36), (300, 513, 2052),
                                   # K % 32 == 0 with a partial last M block: the DMA kernel's row clamp and masked store
                                   (77, 130, 96), (300, 513, 2048), (33, 1, 32)])
def test_gemm_f32(gpu, M, N, K):
    print(f"gemm_f32 M={M} N={N} K={K}", flush=True)
    A = synth.normal_f32(830 + K, (M, K))
    W = synth.normal_f32(831 + N, (N, K)) * 0.05
    D = torch.full((M, N), float("nan"), device="cuda")
    qmm.gemm_f32(dev(A), dev(W), D, M, N, K)
    got = host(D)
    ref = A.astype(np.float64) @ W.astype(np.float64).T
    mag = np.abs(A).astype(np.float64) @ np.abs(W).astype(np.float64).T
    assert np.all(np.isfinite(got))
    assert rel_l2(got, ref) <= 1e-5
    assert np.max(np.abs(got - ref) / (mag + 1e-30)) < 1e-5


def test_gemm_f32_routing(gpu):
    """The prefill router: logits by the f32 GEMM over a 128-row-padded chunk, then the routing of
    the first T rows, held to the oracle's routing of the same logits."""
    T, Mp, K, nexp = 300, 384, 2560, 512
    A = np.zeros((Mp, K), np.float32)
    A[:T] = synth.normal_f32(840, (T, K))
    Wr = synth.normal_f32(841, (nexp + 1, K)) * 0.05
    lg = torch.zeros((Mp, nexp + 1), device="cuda")
    qmm.gemm_f32(dev(A), dev(Wr), lg, Mp, nexp + 1, K)
    lgh = host(lg)
    assert np.all(lgh[T:] == 0.0)
    ids = torch.zeros((T, 11), dtype=torch.int32, device="cuda")
    w = torch.zeros((T, 11), device="cuda")
    qmm.moe_route(lg[:T].contiguous(), ids, w, T)
    ids_ref, w_ref = oracle.moe_route(lgh[:T], nexp, 10)
    assert_route_matches(host(ids), host(w), ids_ref, w_ref, lgh[:T], nexp)
