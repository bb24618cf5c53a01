"""GPU parity of the MoE decode GEMVs (qmm_gemv_moe: expert gather for gate|up, and the down projection
with the slot-weighted combine) for the expert formats of the reference's gemv_moe other than all-Q4_K
(engine/kernels/gemv.hip:1385-1394): routed experts in Q5_K, IQ4_XS, Q8_0_SOA or Q5_1_SOA with the
shared expert in the same format or in Q8_0_SOA, and Q4_K routed experts with a Q8_0_SOA shared expert.
The reference engine's own MoE has expert FF 640 (qwen4exp.h:22): a down projection with K = 640 needs
the 32-weight-block formats.

Bars: each slot's gate/up rows bit for bit the plain q8 GEMV of its expert on its token's x
(qmm_gemv_q8, the same per-row arithmetic; the Q4_K routed experts of the mixed table use the
32-lane-unit decode rather than the Q4_K pair kernel and are held to the tolerance instead); against
the same-math oracle (q8 x, weights dequantised by the reference's formulas, double dot) within
rel-L2 1e-5 and max |ref - got| / sum |w x| < 1e-5; the down output within the same tolerance of the
oracle's slot-weighted sum, and bit for bit the slot-ordered fma combine of the per-slot GEMVs.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest
import torch

import oracle
from hipster_amd import qmm, synth
from tests.gpu_util import dev, host, max_rel_mag, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-5
NEXP_TOTAL, NE = 24, 11          # experts in the table; slots per token (10 routed + shared)
COMBOS = [(synth.Q5_1_SOA, synth.Q5_1_SOA), (synth.Q5_1_SOA, synth.Q8_0_SOA), (synth.Q8_0_SOA, synth.Q8_0_SOA),
          (synth.Q5_K, synth.Q5_K), (synth.Q5_K, synth.Q8_0_SOA), (synth.IQ4_XS, synth.IQ4_XS),
          (synth.IQ4_XS, synth.Q8_0_SOA), (synth.Q4_K, synth.Q8_0_SOA)]

_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.fmaf.restype = ctypes.c_float
_libm.fmaf.argtypes = [ctypes.c_float] * 3


def ffn_for(fmt, sfmt):
    """The engine's expert FF (640) where both formats take K % 32, else 512 (K % 256)."""
    soa = (synth.Q8_0_SOA, synth.Q5_1_SOA)
    return 640 if fmt in soa and sfmt in soa else 512


def tables(seed, fmt, sfmt, N, K):
    E = synth.experts(seed, fmt, NEXP_TOTAL, N, K)
    S = synth.matrix(seed + 1, sfmt, N, K)
    return E, S


def q8_gpu(x):
    xb = qmm.XQ8Buf(x.shape[0], x.shape[1])
    qmm.quantize_x_q8(dev(x), xb, x.shape[0], x.shape[1])
    return xb


def plain_gemv(fmt, W, xb_rows, N, K):
    """qmm_gemv_q8 of one expert on single q8 rows (the T-invariant per-column arithmetic)."""
    y = torch.zeros((1, N), device="cuda")
    qmm.gemv_q8(fmt, W, xb_rows, y, N, K, 1)
    return host(y)[0]


def sub_xq8(xb, r):
    """An XQ8Buf view of row r of xb (no copy)."""
    v = qmm.XQ8Buf.__new__(qmm.XQ8Buf)
    v.ncol, v.K = 1, xb.K
    v.q, v.d, v.s, v.ds = xb.q[r:r + 1], xb.d[r:r + 1], xb.s[r:r + 1], None
    return v


@pytest.mark.parametrize("fmt,sfmt", COMBOS)
@pytest.mark.parametrize("T", [1, 5])
def test_moe_gather_formats(gpu, fmt, sfmt, T):
    H = 2048
    F = ffn_for(fmt, sfmt)
    print(f"moe gather fmt={fmt} shared={sfmt} T={T} N={F} K={H}", flush=True)
    Eg, Sg = tables(1500 + fmt, fmt, sfmt, F, H)
    Eu, Su = tables(1510 + fmt, fmt, sfmt, F, H)
    ids_h, _ = oracle.moe_route(synth.router_logits(1520 + T, T, NEXP_TOTAL), NEXP_TOTAL, 10)
    x = synth.normal_f32(1530 + T, (T, H))
    xb = q8_gpu(x)
    ids = dev(ids_h)
    g = torch.full((T * NE, F), float("nan"), device="cuda")
    u = torch.full((T * NE, F), float("nan"), device="cuda")
    dEg, dEu, dSg, dSu = dev(Eg), dev(Eu), dev(Sg), dev(Su)
    qmm.gemv_moe(fmt, sfmt, [dEg, dEu], [dSg, dSu], [g, u], Eg[0].nbytes, ids, NE, xb, F, H, T, False)
    gh, uh = host(g), host(u)
    q, d, _ = oracle.quantize_x_q8(x)
    xr = oracle.q8_to_f32(q, d)
    for te in range(T * NE):
        t, e = divmod(te, NE)
        eid = int(ids_h[t, e])
        for out, Et, St in ((gh, Eg, Sg), (uh, Eu, Su)):
            Wm, wf = (Et[eid], fmt) if eid >= 0 else (St, sfmt)
            ref, mag = oracle.gemv_ref(wf, Wm, F, H, xr[t:t + 1])
            assert rel_l2(out[te], ref[0]) <= TOL, (te, eid)
            assert max_rel_mag(out[te:te + 1], ref, mag) < TOL, (te, eid)
        if eid < 0 or fmt != synth.Q4_K:       # bitwise the plain GEMV of the expert
            Wm, wf = (dEg[eid], fmt) if eid >= 0 else (dSg, sfmt)
            assert np.array_equal(gh[te].view(np.uint32), plain_gemv(wf, Wm, sub_xq8(xb, t), F, H).view(np.uint32)), te


@pytest.mark.parametrize("fmt,sfmt", COMBOS)
@pytest.mark.parametrize("T", [1, 3])
def test_moe_down_formats(gpu, fmt, sfmt, T):
    H = 2048
    F = ffn_for(fmt, sfmt)
    print(f"moe down fmt={fmt} shared={sfmt} T={T} N={H} K={F}", flush=True)
    Ed, Sd = tables(1540 + fmt, fmt, sfmt, H, F)
    ids_h, w_h = oracle.moe_route(synth.router_logits(1550 + T, T, NEXP_TOTAL), NEXP_TOTAL, 10)
    h = synth.normal_f32(1560 + T, (T * NE, F))
    hb = q8_gpu(h)
    dEd, dSd = dev(Ed), dev(Sd)
    y = torch.full((T, H), float("nan"), device="cuda")
    qmm.gemv_moe(fmt, sfmt, [dEd], [dSd], [y], Ed[0].nbytes, dev(ids_h), NE, hb, H, F, T, True, slotw=dev(w_h))
    yh = host(y)
    q, d, _ = oracle.quantize_x_q8(h)
    hr = oracle.q8_to_f32(q, d)
    for t in range(T):
        ref = np.zeros(H)
        mag = np.zeros(H)
        comb = np.zeros(H, np.float32)
        for e in range(NE):
            eid = int(ids_h[t, e])
            Wm, wf = (Ed[eid], fmt) if eid >= 0 else (Sd, sfmt)
            r, m = oracle.gemv_ref(wf, Wm, H, F, hr[t * NE + e:t * NE + e + 1])
            ref += float(w_h[t, e]) * r[0]
            mag += abs(float(w_h[t, e])) * m[0]
            if fmt != synth.Q4_K or eid < 0:
                Wd = dEd[eid] if eid >= 0 else dSd
                v = plain_gemv(wf, Wd, sub_xq8(hb, t * NE + e), H, F)
                comb = np.array([_libm.fmaf(float(w_h[t, e]), float(v[i]), float(comb[i])) for i in range(H)], np.float32)
        assert rel_l2(yh[t], ref) <= TOL, t
        assert np.max(np.abs(yh[t] - ref) / (mag + 1e-20)) < TOL, t
        if fmt != synth.Q4_K:                  # the combine: fma over the slots in order, bit for bit
            assert np.array_equal(yh[t].view(np.uint32), comb.view(np.uint32)), t


def test_moe_formats_refused(gpu):
    """Combinations the reference does not have: a shared expert in another format than the routed
    one (other than Q8_0_SOA), Q6_K-SoA experts; K not a multiple of the format's block."""
    H, F, T = 256, 64, 1
    xb = q8_gpu(synth.normal_f32(1570, (T, H)))
    E = dev(synth.experts(1571, synth.Q5_1_SOA, 4, F, H))
    ids = dev(np.array([[0, 1, 2, -1]], np.int32))
    y = torch.zeros((T * 4, F), device="cuda")
    with pytest.raises(qmm.QmmError):
        qmm.gemv_moe(synth.Q5_1_SOA, synth.Q5_K, [E], [E[0]], [y], E[0].numel(), ids, 4, xb, F, H, T, False)
    with pytest.raises(qmm.QmmError):
        qmm.gemv_moe(synth.Q6_K_SOA, synth.Q6_K_SOA, [E], [E[0]], [y], E[0].numel(), ids, 4, xb, F, H, T, False)
    with pytest.raises(qmm.QmmError):
        qmm.gemv_moe(synth.Q5_K, synth.Q5_K, [E], [E[0]], [y], E[0].numel(), ids, 4, xb, F, 160, T, False)
