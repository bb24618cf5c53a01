"""The Q4_K and Q6_K_SOA decode GEMVs on the int8 matrix cores (gemv_mfma.hip), through the C ABI.

Bars: every column bitwise equal to the one-column dot4 kernel's result for the same x (so a column's
bits do not depend on ncol, 1..16, nor on which kernel ran), at the headline shape and at shapes whose
block count is not a multiple of 4 or whose rows are not a multiple of 16; several segments in one
launch equal separate calls; and the result against the oracle within the GEMV bar (1e-5).
"""
import numpy as np
import pytest
import torch

import oracle
from hipster_amd import _lib, qmm, synth
from tests.gpu_util import dev, host, max_rel_mag, rel_l2

pytestmark = pytest.mark.gpu


def q8_on_gpu(x):
    ncol, K = x.shape
    xb = qmm.XQ8Buf(ncol, K)
    qmm.quantize_x_q8(dev(x), xb, ncol, K)
    return xb


class min_ncol:
    """qmm_set_gemv_mfma_min_ncol for the duration of a block"""

    def __init__(self, n):
        self.n = n

    def __enter__(self):
        self.prev = _lib.lib().qmm_set_gemv_mfma_min_ncol(self.n)

    def __exit__(self, *a):
        _lib.lib().qmm_set_gemv_mfma_min_ncol(self.prev)


def multi(Wd, xb, N, K, ncol):
    y = torch.full((ncol, N), float("nan"), dtype=torch.float32, device="cuda")
    qmm.gemv_multi([(synth.Q4_K, Wd, y, N, K)], xb, ncol)
    torch.cuda.synchronize()
    return host(y)


def test_columns_equal_one_column_kernel_ncol_1_to_16(gpu):
    """17408 x 5120: for ncol = 1..16 every column is bitwise the one-column kernel's"""
    N, K = 17408, 5120
    print(f"mfma T-invariance N={N} K={K}", flush=True)
    Wd = dev(synth.matrix(700, synth.Q4_K, N, K))
    x = synth.normal_f32(701, (16, K))
    xb = q8_on_gpu(x)
    single = []
    for c in range(16):
        xc = q8_on_gpu(x[c:c + 1])
        single.append(multi(Wd, xc, N, K, 1)[0])
    single = np.stack(single)
    for ncol in range(1, 17):
        y = multi(Wd, xb, N, K, ncol)
        assert np.array_equal(y.view(np.uint32), single[:ncol].view(np.uint32)), ncol
    q, d, _ = oracle.quantize_x_q8(x)
    ref, mag = oracle.gemv_ref(synth.Q4_K, host(Wd), N, K, oracle.q8_to_f32(q, d))
    assert rel_l2(single, ref) <= 1e-5
    assert max_rel_mag(single, ref, mag) < 1e-5


@pytest.mark.parametrize("N,K", [(4099, 5120), (77, 768), (300, 1280), (16, 256), (1000, 17408), (33, 2048)])
def test_mfma_equals_dot4_same_ncol(gpu, N, K):
    """the same call with the matrix-core kernel switched off (dot4 kernels) and on: the same bits"""
    print(f"mfma vs dot4 N={N} K={K}", flush=True)
    Wd = dev(synth.matrix(710 + N, synth.Q4_K, N, K))
    x = synth.normal_f32(711 + K, (16, K))
    xb = q8_on_gpu(x)
    for ncol in (2, 3, 4, 5, 8, 9, 16):
        with min_ncol(17):
            y0 = multi(Wd, xb, N, K, ncol)
        with min_ncol(2):
            y1 = multi(Wd, xb, N, K, ncol)
        assert np.all(np.isfinite(y1))
        assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32)), ncol
    # gemv_q8 (up to 8 columns) takes the same route
    y = torch.zeros((8, N), dtype=torch.float32, device="cuda")
    qmm.gemv_q8(synth.Q4_K, Wd, xb, y, N, K, 8)
    assert np.array_equal(host(y).view(np.uint32), y1[:8].view(np.uint32))


@pytest.mark.parametrize("ncol", [2, 6, 16, 21])
def test_segments_in_one_launch_equal_separate_calls(gpu, ncol):
    K = 2048
    Ns = [1024, 77, 513]
    x = synth.normal_f32(720, (ncol, K))
    xb = q8_on_gpu(x)
    segs, ref = [], []
    for i, N in enumerate(Ns):
        Wh = synth.matrix(721 + i, synth.Q4_K, N, K)
        W = dev(Wh)
        y = torch.full((ncol, N), float("nan"), dtype=torch.float32, device="cuda")
        segs.append((synth.Q4_K, W, y, N, K))
        ref.append(np.stack([multi(W, q8_on_gpu(x[c:c + 1]), N, K, 1)[0] for c in range(ncol)]))
    qmm.gemv_multi(segs, xb, ncol)
    torch.cuda.synchronize()
    for (_, _, y, _, _), r in zip(segs, ref):
        assert np.array_equal(host(y).view(np.uint32), r.view(np.uint32))


class q6_min_ncol:
    """qmm_set_gemv_q6k_mfma_min_ncol for the duration of a block"""

    def __init__(self, n):
        self.n = n

    def __enter__(self):
        self.prev = _lib.lib().qmm_set_gemv_q6k_mfma_min_ncol(self.n)

    def __exit__(self, *a):
        _lib.lib().qmm_set_gemv_q6k_mfma_min_ncol(self.prev)


def q6_gemv(Wd, xb, N, K, ncol):
    y = torch.full((ncol, N), float("nan"), dtype=torch.float32, device="cuda")
    qmm.gemv_q8(synth.Q6_K_SOA, Wd, xb, y, N, K, ncol)
    torch.cuda.synchronize()
    return host(y)


@pytest.mark.parametrize("N,K", [(5120, 17408), (129, 512), (515, 2048), (77, 1024), (1000, 5120)])
def test_q6k_matrix_cores_bitwise_dot4(gpu, N, K):
    """Q6_K_SOA on the int8 matrix cores (forced from one column on) against the dot4 kernels (the
    matrix cores switched off): every column bitwise equal, ncol 1..8; rows not a multiple of 16,
    K = 512 (two blocks: two of the four waves have none) and block counts not a multiple of 4"""
    print(f"q6k mfma vs dot4 N={N} K={K}", flush=True)
    Wd = dev(synth.matrix(720 + N, synth.Q6_K_SOA, N, K))
    x = synth.normal_f32(721, (8, K))
    xb = q8_on_gpu(x)
    for ncol in range(1, 9):
        with q6_min_ncol(9):
            ref = q6_gemv(Wd, xb, N, K, ncol)
        with q6_min_ncol(1):
            got = q6_gemv(Wd, xb, N, K, ncol)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), ncol


def test_q6k_matrix_cores_against_oracle(gpu):
    """the matrix-core Q6_K_SOA GEMV at 4 and 8 columns against the oracle within the GEMV bar"""
    N, K = 333, 5120
    W = synth.matrix(730, synth.Q6_K_SOA, N, K)
    x = synth.normal_f32(731, (8, K))
    q, d, _ = oracle.quantize_x_q8(x)
    ref, mag = oracle.gemv_ref(synth.Q6_K_SOA, W, N, K, oracle.q8_to_f32(q, d))
    xb = q8_on_gpu(x)
    Wd = dev(W)
    with q6_min_ncol(1):
        for ncol in (4, 8):
            y = q6_gemv(Wd, xb, N, K, ncol)
            assert rel_l2(y, ref[:ncol]) <= 1e-5
            assert max_rel_mag(y, ref[:ncol], mag[:ncol]) < 1e-5


def test_q6k_matrix_cores_large_k_falls_back(gpu):
    """ncol * K above the kernel's x-scale staging (8 x 65536) runs the dot4 kernels: the same bits"""
    N, K = 64, 65536
    Wd = dev(synth.matrix(740, synth.Q6_K_SOA, N, K))
    xb = q8_on_gpu(synth.normal_f32(741, (8, K)))
    with q6_min_ncol(9):
        ref = q6_gemv(Wd, xb, N, K, 8)
    with q6_min_ncol(1):
        got = q6_gemv(Wd, xb, N, K, 8)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


class q80_min_ncol:
    """qmm_set_gemv_q80_mfma_min_ncol for the duration of a block"""

    def __init__(self, n):
        self.n = n

    def __enter__(self):
        self.prev = _lib.lib().qmm_set_gemv_q80_mfma_min_ncol(self.n)

    def __exit__(self, *a):
        _lib.lib().qmm_set_gemv_q80_mfma_min_ncol(self.prev)


def q80_gemv(Wd, xb, N, K, ncol):
    y = torch.full((ncol, N), float("nan"), dtype=torch.float32, device="cuda")
    qmm.gemv_q8(synth.Q8_0_SOA, Wd, xb, y, N, K, ncol)
    torch.cuda.synchronize()
    return host(y)


@pytest.mark.parametrize("N,K", [(17408, 5120), (129, 64), (515, 2048), (77, 1088), (1000, 5120), (40, 8192)])
def test_q80_matrix_cores_bitwise_dot4(gpu, N, K):
    """Q8_0_SOA on the int8 matrix cores (forced from one column on) against the dot4 kernels (the
    matrix cores switched off): every column bitwise equal, ncol 1..8; rows not a multiple of 16, one
    64-weight chunk (three of the four waves have none), chunk counts not a multiple of 4 or of 32, 8
    columns at K = 5120 (the most x the kernel stages) and the largest K it takes (8192: matrix cores up
    to 5 columns, the dot4 kernels above)"""
    print(f"q8_0 mfma vs dot4 N={N} K={K}", flush=True)
    Wd = dev(synth.matrix(750 + N, synth.Q8_0_SOA, N, K))
    xb = q8_on_gpu(synth.normal_f32(751, (8, K)))
    for ncol in range(1, 9):
        with q80_min_ncol(9):
            ref = q80_gemv(Wd, xb, N, K, ncol)
        with q80_min_ncol(1):
            got = q80_gemv(Wd, xb, N, K, ncol)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), ncol


def test_q80_matrix_cores_against_oracle(gpu):
    """the matrix-core Q8_0_SOA GEMV at 2, 5 and 8 columns against the oracle within the GEMV bar"""
    N, K = 333, 5120
    W = synth.matrix(760, synth.Q8_0_SOA, N, K)
    x = synth.normal_f32(761, (8, K))
    q, d, _ = oracle.quantize_x_q8(x)
    ref, mag = oracle.gemv_ref(synth.Q8_0_SOA, W, N, K, oracle.q8_to_f32(q, d))
    xb = q8_on_gpu(x)
    Wd = dev(W)
    with q80_min_ncol(1):
        for ncol in (2, 5, 8):
            y = q80_gemv(Wd, xb, N, K, ncol)
            assert rel_l2(y, ref[:ncol]) <= 1e-5
            assert max_rel_mag(y, ref[:ncol], mag[:ncol]) < 1e-5


def test_q80_matrix_cores_large_k_falls_back(gpu):
    """K above what the kernel stages (8192) runs the dot4 kernels: the same bits"""
    N, K = 64, 32768
    Wd = dev(synth.matrix(770, synth.Q8_0_SOA, N, K))
    xb = q8_on_gpu(synth.normal_f32(771, (8, K)))
    with q80_min_ncol(9):
        ref = q80_gemv(Wd, xb, N, K, 8)
    with q80_min_ncol(1):
        got = q80_gemv(Wd, xb, N, K, 8)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
