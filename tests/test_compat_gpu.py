"""GPU parity of the reference-signature entry points that keep the engine's remaining call sites
working (compat.hip, gemm.hip), through the C ABI:

  gemv_splitk     each partial within 1e-5 of the oracle's double dot over its K range (the reference's
                  256-block split, gemv.hip:1404), and the partials' sum within 1e-5 of the whole GEMV
  moe_gemm (q8)   every sorted row within 1e-5 of the oracle's q8 GEMV of its expert (the reference's
                  integer arithmetic, not bf16), routed and shared tiles of the reference's widths
  q8k             quantize_x_q8k bit-exact against the oracle; gemv_wmma_q8k within 1e-5 of the double dot
  gemm_bf16_ld    strided operands give the bits of gemm_bf16 on contiguous copies
  gemv_q8 rpt 4   (the reference's route to its T-invariant GEMV) = gemv_multi, up to 16 columns
  gemv_q8 layouts rpt 5 / rpt 4 + tpr 3 on the reference's interleaved weight layouts, within 1e-5 of the
                  oracle on the row-major matrix
"""
import numpy as np
import pytest
import torch

import oracle
from hipster_amd import qmm, synth
from tests.gpu_util import dev, host, max_rel_mag, rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-5


def q8(x):
    xb = qmm.XQ8Buf(x.shape[0], x.shape[1])
    qmm.quantize_x_q8(dev(x), xb, x.shape[0], x.shape[1])
    return xb


def q8_dequant(x):
    q, d, _ = oracle.quantize_x_q8(x)
    return oracle.q8_to_f32(q, d)


@pytest.mark.parametrize("fmt,N,K,ksplit", [(synth.Q8_0_SOA, 320, 10240, 8), (synth.Q4_K, 320, 10240, 8),
                                            (synth.Q5_1_SOA, 96, 2560, 3), (synth.Q6_K_SOA, 130, 5120, 5),
                                            (synth.Q8_0_SOA, 57, 320, 2), (synth.Q4_K, 64, 17408, 8)])
@pytest.mark.parametrize("ncol", [1, 3, 9])
def test_gemv_splitk(gpu, fmt, N, K, ksplit, ncol):
    print(f"splitk fmt={fmt} N={N} K={K} ksplit={ksplit} ncol={ncol}", flush=True)
    W = synth.matrix(500 + fmt + K, fmt, N, K)
    x = synth.normal_f32(501 + K, (ncol, K))
    part = torch.full((ncol, ksplit, N), np.nan, dtype=torch.float32, device="cuda")
    qmm.gemv_splitk(fmt, dev(W), q8(x), part, N, K, ksplit, ncol)
    p = host(part)
    Wf = oracle.dequant_rows(fmt, W, K).astype(np.float64)
    xr = q8_dequant(x).astype(np.float64)
    nb = (K + 255) // 256
    for ks in range(ksplit):
        k0, k1 = ks * nb // ksplit * 256, min((ks + 1) * nb // ksplit * 256, K)
        ref = xr[:, k0:k1] @ Wf[:, k0:k1].T
        mag = np.abs(xr[:, k0:k1]) @ np.abs(Wf[:, k0:k1]).T
        assert max_rel_mag(p[:, ks], ref, mag) < TOL, ks
    full, mag = oracle.gemv_ref(fmt, W, N, K, q8_dequant(x))
    s = np.zeros((ncol, N), np.float64)
    for ks in range(ksplit):
        s += p[:, ks]
    assert max_rel_mag(s, full, mag) < TOL


def _tiles(ids, maxc):
    kpos, rowtok, tl, st = oracle.moe_sort(ids, maxc)
    return kpos, rowtok, tl, st


@pytest.mark.parametrize("fmt,sfmt,N,K,T,n_exp,ct", [(synth.Q4_K, synth.Q4_K, 512, 2048, 96, 32, 1),
                                                      (synth.Q4_K, synth.Q8_0_SOA, 2048, 512, 64, 16, 3),
                                                      (synth.Q4_K, synth.Q4_K, 200, 512, 40, 12, 4),
                                                      (synth.Q8_0_SOA, synth.Q4_K, 192, 512, 30, 12, 2),
                                                      (synth.Q5_1_SOA, synth.Q5_1_SOA, 256, 640, 40, 12, 2),
                                                      (synth.Q5_K, synth.Q8_0_SOA, 640, 512, 33, 12, 1),
                                                      (synth.IQ4_XS, synth.IQ4_XS, 128, 768, 20, 10, 2),
                                                      (synth.Q8_0_SOA, synth.Q8_0_SOA, 200, 320, 17, 16, 1)])
def test_moe_gemm_q8(gpu, fmt, sfmt, N, K, T, n_exp, ct):
    """rows gathered by rowtab (gate/up) and in place (down, rowtab = NULL); Q4_K tile lists run on the
    int8 matrix cores (N = 200: a partial 64-row block; ct = 4: tiles of 64 columns, two passes)"""
    print(f"moe_gemm fmt={fmt}/{sfmt} N={N} K={K} T={T} E={n_exp} ct={ct}", flush=True)
    NE = 11
    assert n_exp >= 10                                   # top-10 routing
    ids, _ = oracle.moe_route(synth.router_logits(520 + T, T, n_exp), n_exp, 10)
    kpos, rowtok, tl, st = _tiles(ids, 16 * ct)
    E = synth.experts(521 + fmt, fmt, n_exp, N, K)
    S = synth.matrix(522 + sfmt, sfmt, N, K)
    eb = E.shape[1] if E.ndim == 2 else E[0].nbytes
    Ed, Sd = dev(E), dev(S)
    NS = T * NE
    for gather in (True, False):
        xrows = T if gather else NS
        x = synth.normal_f32(523 + xrows, (xrows, K))
        xb = q8(x)
        y = torch.full((NS, N), np.nan, dtype=torch.float32, device="cuda")
        qmm.moe_gemm(fmt, sfmt, Ed, Sd, eb, dev(tl), len(tl), dev(st), len(st), ct, dev(rowtok) if gather else None,
                     xb, y, N, K)
        got = host(y)
        assert not np.isnan(got).any()
        xr = q8_dequant(x)
        ks = np.arange(NS)
        rows_x = rowtok if gather else ks
        # expert of each sorted position
        eid = np.full(NS, -2, np.int64)
        for e, k0, nc in np.concatenate([tl, st]):
            eid[k0:k0 + nc] = e
        assert (eid >= -1).all()
        for e in np.unique(eid):
            sel = np.nonzero(eid == e)[0]
            Wm = S if e < 0 else E[e]
            ref, mag = oracle.gemv_ref(sfmt if e < 0 else fmt, Wm, N, K, xr[rows_x[sel]])
            assert max_rel_mag(got[sel], ref, mag) < TOL, (gather, e)


def test_moe_gemm_q8_many_tiles(gpu):
    """65535 routed + 2 shared Q4_K tiles: more grid rows than one launch holds, so the routed and
    shared lists go in two launches; every row still matches its expert's q8 GEMV"""
    N, K, T, ntl, nst = 64, 256, 8, 65535, 2
    print(f"moe_gemm many tiles N={N} K={K} tiles={ntl}+{nst}", flush=True)
    E = synth.experts(540, synth.Q4_K, 2, N, K)
    S = synth.matrix(541, synth.Q4_K, N, K)
    NS = ntl + nst
    tl = np.stack([np.arange(ntl) % 2, np.arange(ntl), np.ones(ntl)], 1).astype(np.int32)
    st = np.stack([np.full(nst, -1), ntl + np.arange(nst), np.ones(nst)], 1).astype(np.int32)
    rowtab = (np.arange(NS) % T).astype(np.int32)
    x = synth.normal_f32(542, (T, K))
    y = torch.full((NS, N), np.nan, dtype=torch.float32, device="cuda")
    eb = E.shape[1] if E.ndim == 2 else E[0].nbytes
    qmm.moe_gemm(synth.Q4_K, synth.Q4_K, dev(E), dev(S), eb, dev(tl), ntl, dev(st), nst, 1, dev(rowtab),
                 q8(x), y, N, K)
    got = host(y)
    xr = q8_dequant(x)
    eid = np.concatenate([tl[:, 0], st[:, 0]])
    for e in (-1, 0, 1):
        sel = np.nonzero(eid == e)[0]
        ref, mag = oracle.gemv_ref(synth.Q4_K, S if e < 0 else E[e], N, K, xr)
        assert max_rel_mag(got[sel], ref[rowtab[sel]], mag[rowtab[sel]]) < TOL, e


@pytest.mark.parametrize("ncol,K", [(1, 256), (5, 5120), (16, 2048)])
def test_quantize_x_q8k_bit_exact(gpu, ncol, K):
    x = synth.normal_f32(530 + K, (ncol, K))
    x[0, :256] = 0.0
    x[-1, 256:288] *= 1e-30
    xb = qmm.XQ8KBuf(ncol, K)
    qmm.quantize_x_q8k(dev(x), xb, ncol, K)
    q, d, bs = oracle.quantize_x_q8k(x)
    assert np.array_equal(host(xb.q), q)
    assert np.array_equal(host(xb.d)[:, :ncol].view(np.uint32), d[:, :ncol].view(np.uint32))
    assert np.array_equal(host(xb.bs)[:, :ncol], bs[:, :ncol])


@pytest.mark.parametrize("fmt,N,K", [(synth.Q4_K, 17408, 5120), (synth.Q5_K, 300, 2048), (synth.IQ4_XS, 257, 1024),
                                     (synth.Q6_K_SOA, 512, 5120), (synth.Q8_0_SOA, 100, 2560)])
@pytest.mark.parametrize("ncol", [1, 7, 16])
def test_gemv_wmma_q8k(gpu, fmt, N, K, ncol):
    W = synth.matrix(540 + fmt, fmt, N, K)
    x = synth.normal_f32(541 + K, (ncol, K))
    xb = qmm.XQ8KBuf(ncol, K)
    qmm.quantize_x_q8k(dev(x), xb, ncol, K)
    y = torch.zeros((ncol, N), dtype=torch.float32, device="cuda")
    Wd = dev(W)
    qmm.gemv_wmma_q8k([(fmt, Wd, y, N, K)], xb, ncol)
    q, d, _ = oracle.quantize_x_q8k(x)
    ref, mag = oracle.gemv_ref(fmt, W, N, K, oracle.q8k_to_f32(q, d))
    assert max_rel_mag(host(y), ref, mag) < TOL
    assert rel_l2(host(y), ref) < TOL
    if ncol > 1:        # column 0 alone: the same bits
        y1 = torch.zeros((1, N), dtype=torch.float32, device="cuda")
        qmm.gemv_wmma_q8k([(fmt, Wd, y1, N, K)], xb, 1)
        assert np.array_equal(host(y1)[0], host(y)[0])


@pytest.mark.parametrize("M,N,K", [(300, 520, 1024), (2048, 768, 8704), (64, 256, 192)])
def test_gemm_bf16_ld(gpu, M, N, K):
    """BlasLt::gemm_ld's use: the two K halves of [rows][2K] operands as strided views (qwen35.cpp:230-231)"""
    g = torch.Generator(device="cuda").manual_seed(M + N)
    A = torch.randn((M, 2 * K), device="cuda", generator=g).to(torch.bfloat16)
    W = torch.randn((N, 2 * K), device="cuda", generator=g).to(torch.bfloat16)
    for h in (0, 1):
        D = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
        qmm.gemm_bf16_ld(A[:, h * K:], 2 * K, W[:, h * K:], 2 * K, D, M, N, K)
        D2 = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
        qmm.gemm_bf16(A[:, h * K:(h + 1) * K].contiguous(), W[:, h * K:(h + 1) * K].contiguous(), D2, M, N, K)
        torch.cuda.synchronize()
        assert torch.equal(D.view(torch.int16), D2.view(torch.int16))
    with pytest.raises(qmm.QmmError):          # lda below K
        qmm.gemm_bf16_ld(A, K - 8, W, 2 * K, D, M, N, K)


def test_gemv_q8_rpt4_is_the_multi_gemv(gpu):
    """rpt = 4 (the reference's route to gemv_wmma, up to 16 columns) gives the bits of gemv_multi; any
    other tpr / rpt (the reference's launch knobs, unlisted values included) gives the plain GEMV's."""
    N, K = 4099, 5120
    W = dev(synth.matrix(550, synth.Q4_K, N, K))
    x = synth.normal_f32(551, (16, K))
    xb = q8(x)
    y = torch.zeros((16, N), dtype=torch.float32, device="cuda")
    qmm.gemv_q8(synth.Q4_K, W, xb, y, N, K, 16, tpr=2, rpt=4)
    y2 = torch.zeros((16, N), dtype=torch.float32, device="cuda")
    qmm.gemv_multi([(synth.Q4_K, W, y2, N, K)], xb, 16)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    for tpr, rpt in ((0, 1), (3, 1), (7, 3), (64, 0)):
        qmm.gemv_q8(synth.Q4_K, W, xb, y, N, K, 8, tpr=tpr, rpt=rpt)
        qmm.gemv_q8(synth.Q4_K, W, xb, y2, N, K, 8)
        torch.cuda.synchronize()
        assert torch.equal(y[:8], y2[:8]), (tpr, rpt)


IL_CASES = [(8, synth.Q4_K, 4104, 5120), (8, synth.Q5_K, 520, 2048), (8, synth.IQ4_XS, 264, 1024),
            (16, synth.Q4_K, 4099, 5120), (16, synth.Q5_K, 300, 2048), (16, synth.IQ4_XS, 257, 1024),
            (16, synth.Q6_K_SOA, 130, 5120), (16, synth.Q8_0_SOA, 100, 2560)]


@pytest.mark.parametrize("rows,fmt,N,K", IL_CASES)
def test_gemv_q8_interleaved_layouts(gpu, rows, fmt, N, K):
    """The reference's experimental layouts (rpt 5: repack_interleave8, 8 rows; rpt 4 with tpr 3:
    repack_wmma_il, 16 rows, N padded): the repacked bytes uploaded, every row within 1e-5 of the
    oracle's q8 GEMV on the row-major matrix, at column counts that take one and several launches
    (8, then 4, then the rest); the 32-weight-unit formats give the bits of their plain GEMV."""
    print(f"gemv_q8 layout rows={rows} fmt={fmt} N={N} K={K}", flush=True)
    Wr = synth.matrix(560 + fmt + rows, fmt, N, K)
    Wil = qmm.repack_interleave8(fmt, Wr, N, K) if rows == 8 else qmm.repack_wmma_il(fmt, Wr, N, K)
    tpr, rpt = (0, 5) if rows == 8 else (3, 4)
    ncols = (1, 5, 8) if rows == 8 else (1, 11, 16)
    x = synth.normal_f32(561 + K, (16, K))
    xb = q8(x)
    xr = q8_dequant(x)
    ref, mag = oracle.gemv_ref(fmt, Wr, N, K, xr)
    Wd = dev(Wil)
    for ncol in ncols:
        y = torch.full((ncol, N), np.nan, dtype=torch.float32, device="cuda")
        qmm.gemv_q8(fmt, Wd, xb, y, N, K, ncol, tpr=tpr, rpt=rpt)
        got = host(y)
        assert max_rel_mag(got, ref[:ncol], mag[:ncol]) < TOL, ncol
    if fmt in (synth.Q5_K, synth.IQ4_XS, synth.Q8_0_SOA):
        yp = torch.zeros((8, N), dtype=torch.float32, device="cuda")
        qmm.gemv_q8(fmt, dev(Wr), xb, yp, N, K, 8)
        y = torch.zeros((8, N), dtype=torch.float32, device="cuda")
        qmm.gemv_q8(fmt, Wd, xb, y, N, K, 8, tpr=tpr, rpt=rpt)
        torch.cuda.synchronize()
        assert torch.equal(y, yp)
    with pytest.raises(qmm.QmmError):          # the layouts' formats only
        qmm.gemv_q8(synth.Q5_1_SOA, Wd, xb, y, N, K, 1, tpr=tpr, rpt=rpt)
