"""GPU parity of the MoE decode path (routing, expert gather GEMV, silu*up -> q8, down + combine,
prefill combine) against the CPU oracle, through the C ABI.

Bars: routing ids bit-exact; weights and outputs within rel 1e-5 of the
oracle fed with the same stage inputs; per-slot expert outputs bitwise equal to the plain decode GEMV
of that expert (so the device-side expert dedup changes nothing); a token's result bitwise the same
alone and inside a batch (T-invariance).
"""
import numpy as np
import pytest
import torch

import oracle
from hipster_amd import qmm, synth
from tests.gpu_util import assert_route_matches, dev, host, rel_l2

pytestmark = pytest.mark.gpu

H, F = 2048, 512          # hidden 2048, expert FF 512


def experts(seed, n_exp, N, K):
    return synth.experts(seed, synth.Q4_K, n_exp, N, K)


@pytest.mark.parametrize("T,zipf", [(1, None), (4, None), (8, None), (2048, 1.1)])
def test_route_matches_oracle(gpu, T, zipf):
    logits = synth.router_logits(1200 + T, T, 512, zipf)
    ids_ref, w_ref = oracle.moe_route(logits, 512, 10)
    ids = torch.zeros((T, 11), dtype=torch.int32, device="cuda")
    w = torch.zeros((T, 11), dtype=torch.float32, device="cuda")
    qmm.moe_route(dev(logits), ids, w, T)
    ids_h = host(ids)
    print(f"route T={T}: {int((ids_h != ids_ref).any(axis=1).sum())} tokens differ from the oracle", flush=True)
    assert_route_matches(ids_h, host(w), ids_ref, w_ref, logits, 512)


def test_route_selects_on_rounded_probabilities(gpu):
    """Experts 3 (logit -2^-30) and 8 (logit 0) both get exp(.) = 1.0 and so the same p: the lower id
    is taken first, as the reference's argmax on p does (fn.hip:176-180)."""
    logits = np.full((2, 513), -4.0, np.float32)
    logits[:, 8] = 0.0
    logits[:, 3] = -2.0 ** -30
    ids = torch.zeros((2, 11), dtype=torch.int32, device="cuda")
    w = torch.zeros((2, 11), dtype=torch.float32, device="cuda")
    qmm.moe_route(dev(logits), ids, w, 2)
    ids_h, w_h = host(ids), host(w)
    assert list(ids_h[0, :2]) == [3, 8] and w_h[0, 0] == w_h[0, 1]
    ids_ref, _ = oracle.moe_route(logits, 512, 10)
    assert np.array_equal(ids_h, ids_ref)


def test_route_ties_and_small_expert_counts(gpu):
    logits = synth.router_logits(7, 6, 64)
    logits[0, [3, 9, 40]] = 5.0          # exact ties: lower ids first
    logits[1, :64] = 1.0                 # all equal
    logits[2, 60:64] = 9.0
    for nexp, topk in ((64, 4), (64, 10), (33, 16)):
        lg = np.ascontiguousarray(logits[:, :nexp + 1] if nexp + 1 <= 65 else logits)
        ids_ref, w_ref = oracle.moe_route(lg, nexp, topk)
        ids = torch.zeros((6, topk + 1), dtype=torch.int32, device="cuda")
        w = torch.zeros((6, topk + 1), dtype=torch.float32, device="cuda")
        qmm.moe_route_n(dev(lg), ids, w, 6, nexp, lg.shape[1], topk)
        assert_route_matches(host(ids), host(w), ids_ref, w_ref, lg, nexp)


def test_moe_silu_quant(gpu):
    rows, n = 88, 512
    g = synth.normal_f32(30, (rows, n)) * 3
    u = synth.normal_f32(31, (rows, n))
    g[0, :32] = 0.0
    xq = qmm.XQ8Buf(rows, n)
    qmm.moe_silu_quant(dev(g), dev(u), xq, rows, n)
    h = np.empty_like(g)
    oracle.lib().qo_silu_mul(oracle._ptr(g), oracle._ptr(u), g.size, oracle._ptr(h))
    q, d, s = oracle.quantize_x_q8(h)
    gq, gd = host(xq.q), host(xq.d)
    # silu's exp may differ from the host libm by an ulp, which can move a value across a rounding
    # boundary of the quantiser: allow a difference of one quantum on at most 0.1% of the values
    assert np.max(np.abs(gq.astype(int) - q.astype(int))) <= 1
    assert np.mean(gq != q) < 1e-3
    np.testing.assert_allclose(gd, d, rtol=1e-5)
    np.testing.assert_allclose(oracle.q8_to_f32(gq, gd), oracle.q8_to_f32(q, d), rtol=0, atol=float(d.max()) * 1.01)


def gather(ids, nexp, Wg, Wu, Sg, Su, x, T):
    """GPU gate|up for all slots: returns g, u [T*nexp][F] and the x quantised on the GPU."""
    xb = qmm.XQ8Buf(T, H)
    qmm.quantize_x_q8(dev(x), xb, T, H)
    g = torch.full((T * nexp, F), float("nan"), device="cuda")
    u = torch.full((T * nexp, F), float("nan"), device="cuda")
    eb = Wg[0].nbytes
    qmm.gemv_moe(synth.Q4_K, synth.Q4_K, [Wg, Wu], [Sg, Su], [g, u], eb, ids, nexp, xb, F, H, T, False)
    return g, u, xb


@pytest.mark.parametrize("T", [1, 4, 8])
def test_gemv_moe_gate_up_equals_per_expert_gemv(gpu, T):
    n_exp = 64
    Wg_h, Wu_h = experts(1210, n_exp, F, H), experts(1211, n_exp, F, H)
    Sg_h, Su_h = synth.matrix(1212, synth.Q4_K, F, H), synth.matrix(1213, synth.Q4_K, F, H)
    x = synth.normal_f32(1214, (T, H))
    logits = synth.router_logits(1215, T, n_exp)
    ids_h, _ = oracle.moe_route(logits, n_exp, 10)
    if T >= 4:                      # force experts shared between tokens (exercise the dedup)
        ids_h[1, 3] = ids_h[0, 5]
        ids_h[2, 0] = ids_h[0, 5]
        ids_h[3, 9] = ids_h[1, 1]
    nexp = 11
    Wg, Wu, Sg, Su = dev(Wg_h), dev(Wu_h), dev(Sg_h), dev(Su_h)
    ids = dev(ids_h)
    g, u, xb = gather(ids, nexp, Wg, Wu, Sg, Su, x, T)
    gh, uh = host(g), host(u)
    q, d, _ = oracle.quantize_x_q8(x)
    xr = oracle.q8_to_f32(q, d)
    for t in range(T):
        for e in range(nexp):
            te, eid = t * nexp + e, ids_h[t, e]
            for seg, (Wx, Sx, out) in enumerate(((Wg, Sg, gh), (Wu, Su, uh))):
                Wm = Wx[eid] if eid >= 0 else Sx
                y1 = torch.zeros((1, F), device="cuda")
                xb1 = qmm.XQ8Buf(1, H)
                qmm.quantize_x_q8(dev(x[t:t + 1]), xb1, 1, H)
                qmm.gemv_q8(synth.Q4_K, Wm.contiguous(), xb1, y1, F, H, 1)
                assert np.array_equal(out[te].view(np.uint32), host(y1)[0].view(np.uint32)), (t, e, seg)
        # and against the oracle (same-math q8 x, double dot)
        for e in (0, 7, 10):
            eid = ids_h[t, e]
            Wm = Wg_h[eid] if eid >= 0 else Sg_h
            ref, _ = oracle.gemv_ref(synth.Q4_K, Wm, F, H, xr[t:t + 1])
            assert rel_l2(gh[t * nexp + e], ref[0]) <= 1e-5


def test_gemv_moe_down_combine_matches_oracle(gpu):
    T, nexp, n_exp = 8, 11, 64
    Wd_h = experts(1220, n_exp, H, F)
    Sd_h = synth.matrix(1221, synth.Q4_K, H, F)
    logits = synth.router_logits(1222, T, n_exp)
    ids_h, w_h = oracle.moe_route(logits, n_exp, 10)
    ids_h[5, 2] = ids_h[4, 2]
    hrows = synth.normal_f32(1223, (T * nexp, F))
    hq = qmm.XQ8Buf(T * nexp, F)
    qmm.quantize_x_q8(dev(hrows), hq, T * nexp, F)
    y = torch.full((T, H), float("nan"), device="cuda")
    qmm.gemv_moe(synth.Q4_K, synth.Q4_K, [dev(Wd_h)], [dev(Sd_h)], [y], Wd_h[0].nbytes, dev(ids_h), nexp, hq, H, F, T,
                 True, slotw=dev(w_h))
    dn_ref, y_ref = oracle.moe_down_q8(synth.Q4_K, Wd_h, Sd_h, host(hq.q), host(hq.d), ids_h, w_h, H, F)
    yh = host(y)
    for t in range(T):
        assert rel_l2(yh[t], y_ref[t]) <= 1e-5, t


def test_moe_decode_t_invariant_and_end_to_end(gpu):
    """Full decode MoE on device (route -> gate|up -> silu q8 -> down+combine) for T = 8, and each
    token again alone: bitwise equal.  Each stage against the oracle on the previous stage's device
    output: gate and up rows within 1e-5 (on the device's ids), h within one q8 quantum of the oracle's
    silu * up of the device's g and u, down + combine within 1e-5 (on the device's h).  End to end
    against the oracle's own pipeline within 1e-3 (its silu uses the host libm exp, which can flip a
    q8 rounding of h, and the down projection carries that flip)."""
    n_exp, T, nexp = 64, 8, 11
    Wg_h, Wu_h, Wd_h = experts(1230, n_exp, F, H), experts(1231, n_exp, F, H), experts(1232, n_exp, H, F)
    Sg_h, Su_h, Sd_h = (synth.matrix(1233 + i, synth.Q4_K, *s) for i, s in enumerate(((F, H), (F, H), (H, F))))
    W = [dev(a) for a in (Wg_h, Wu_h, Wd_h, Sg_h, Su_h, Sd_h)]
    x = synth.normal_f32(1236, (T, H))
    logits = synth.router_logits(1237, T, n_exp)

    def run(xs, lg):
        Tn = xs.shape[0]
        ids = torch.zeros((Tn, nexp), dtype=torch.int32, device="cuda")
        w = torch.zeros((Tn, nexp), dtype=torch.float32, device="cuda")
        qmm.moe_route_n(dev(lg), ids, w, Tn, n_exp, lg.shape[1], 10)
        g, u, _ = gather(ids, nexp, W[0], W[1], W[3], W[4], xs, Tn)
        hq = qmm.XQ8Buf(Tn * nexp, F)
        qmm.moe_silu_quant(g, u, hq, Tn * nexp, F)
        y = torch.zeros((Tn, H), device="cuda")
        qmm.gemv_moe(synth.Q4_K, synth.Q4_K, [W[2]], [W[5]], [y], Wd_h[0].nbytes, ids, nexp, hq, H, F, Tn, True, slotw=w)
        return host(y), host(ids), host(w), (host(g), host(u), host(hq.q), host(hq.d))

    yT, idsT, wT, (gT, uT, hqT, hdT) = run(x, logits)
    for t in range(T):
        y1, _, _, _ = run(x[t:t + 1], logits[t:t + 1])
        assert np.array_equal(y1[0].view(np.uint32), yT[t].view(np.uint32)), t
    g_ref, u_ref, _, y_ref = oracle.moe_decode(synth.Q4_K, Wg_h, Wu_h, Wd_h, Sg_h, Su_h, Sd_h, x, idsT, wT, H, F)
    for r in range(T * nexp):
        assert rel_l2(gT[r], g_ref[r]) <= 1e-5 and rel_l2(uT[r], u_ref[r]) <= 1e-5, r
    gc, uc = np.ascontiguousarray(gT), np.ascontiguousarray(uT)
    h_ref = np.empty_like(gc)
    oracle.lib().qo_silu_mul(oracle._ptr(gc), oracle._ptr(uc), gc.size, oracle._ptr(h_ref))
    hq_ref, hd_ref, _ = oracle.quantize_x_q8(h_ref)
    assert np.abs(hqT.reshape(-1).astype(np.int32) - hq_ref.reshape(-1).astype(np.int32)).max() <= 1
    np.testing.assert_allclose(hdT.reshape(-1), hd_ref.reshape(-1), rtol=1e-5)
    _, y_chain = oracle.moe_down_q8(synth.Q4_K, Wd_h, Sd_h, hqT, hdT, idsT, wT, H, F)
    for t in range(T):
        assert rel_l2(yT[t], y_chain[t]) <= 1e-5, t
    assert rel_l2(yT, y_ref) <= 1e-3


def test_moe_full_512_experts_gate_up(gpu):
    """The BASELINE config-2 expert table (512 Q4_K experts + shared) at T = 8."""
    n_exp, T, nexp = 512, 8, 11
    Wg_h, Wu_h = experts(1240, n_exp, F, H), experts(1241, n_exp, F, H)
    Sg_h, Su_h = synth.matrix(1242, synth.Q4_K, F, H), synth.matrix(1243, synth.Q4_K, F, H)
    x = synth.normal_f32(1244, (T, H))
    ids_h, _ = oracle.moe_route(synth.router_logits(1245, T, n_exp), n_exp, 10)
    g, u, _ = gather(dev(ids_h), nexp, dev(Wg_h), dev(Wu_h), dev(Sg_h), dev(Su_h), x, T)
    q, d, _ = oracle.quantize_x_q8(x)
    xr = oracle.q8_to_f32(q, d)
    gh, uh = host(g), host(u)
    for t in (0, 7):
        for e in range(nexp):
            eid = ids_h[t, e]
            for W_h, S_h, out in ((Wg_h, Sg_h, gh), (Wu_h, Su_h, uh)):
                ref, _ = oracle.gemv_ref(synth.Q4_K, W_h[eid] if eid >= 0 else S_h, F, H, xr[t:t + 1])
                assert rel_l2(out[t * nexp + e], ref[0]) <= 1e-5


def test_moe_combine_sorted(gpu):
    T, nexp, E = 64, 11, 2048
    NS = T * nexp
    down = synth.normal_f32(1250, (NS, E))
    w = np.abs(synth.normal_f32(1251, (T, nexp)))
    kpos = synth.rng(1252).permutation(NS).astype(np.int32)
    y = torch.zeros((T, E), device="cuda")
    qmm.moe_combine_sorted(dev(down), dev(w), dev(kpos), y, T, nexp, E)
    ref = np.einsum("te,ted->td", w.astype(np.float64), down[kpos.reshape(T, nexp)].astype(np.float64))
    assert rel_l2(host(y), ref) <= 1e-6
    # views 4 bytes off a 16-byte boundary take the scalar path: the same bits
    dbuf = torch.zeros(NS * E + 1, device="cuda")
    dbuf[1:] = dev(down).reshape(-1)
    ybuf = torch.full((T * E + 1,), float("nan"), device="cuda")
    qmm.moe_combine_sorted(dbuf[1:], dev(w), dev(kpos), ybuf[1:], T, nexp, E)
    assert np.array_equal(host(ybuf[1:]).reshape(T, E).view(np.uint32), host(y).view(np.uint32))


# (T, n_exp, H, F): config 2 at T = 1 / 4 / 8, a small expert table, and a wider shape (H 4096, F 1024) whose
# tokens' x no longer fits the registers the two launches load it into ahead of the expert rows (both
# launches then stage x after their ids, the other code path)
@pytest.mark.parametrize("T,n_exp,H,F", [(1, 512, H, F), (4, 512, H, F), (8, 512, H, F), (3, 40, H, F), (8, 16, 4096, 1024),
                                         (1, 16, 4096, 1024)])
def test_moe_decode_step_bitwise(gpu, T, n_exp, H, F):
    """qmm_moe_decode (routing, each distinct expert's gate|up rows once for its slots and silu*up -> q8 in
    the first launch, the q8 down projection in the second) against the four-launch sequence of separate calls
    on the same inputs: ids, weights, y and the workspace's q8 of h bit for bit.  Then y against the
    oracle's down projection + combine fed with the device's q8 h and routing (1e-5: every stage after the
    device exp of silu pinned)."""
    print(f"moe_decode T={T} n_exp={n_exp} H={H} F={F}", flush=True)
    nexp = 11
    Wg_h, Wu_h, Wd_h = experts(1260, n_exp, F, H), experts(1261, n_exp, F, H), experts(1262, n_exp, H, F)
    Sg_h, Su_h, Sd_h = (synth.matrix(1263 + i, synth.Q4_K, *s) for i, s in enumerate(((F, H), (F, H), (H, F))))
    W = [dev(a) for a in (Wg_h, Wu_h, Wd_h, Sg_h, Su_h, Sd_h)]
    x = synth.normal_f32(1266 + T, (T, H))
    lg = dev(synth.router_logits(1267 + T, T, n_exp))
    xb = qmm.XQ8Buf(T, H)
    qmm.quantize_x_q8(dev(x), xb, T, H)
    # four launches
    ids = torch.zeros((T, nexp), dtype=torch.int32, device="cuda")
    w = torch.zeros((T, nexp), dtype=torch.float32, device="cuda")
    qmm.moe_route_n(lg, ids, w, T, n_exp, n_exp + 1, 10)
    g = torch.zeros((T * nexp, F), device="cuda"); u = torch.zeros((T * nexp, F), device="cuda")
    qmm.gemv_moe(synth.Q4_K, synth.Q4_K, [W[0], W[1]], [W[3], W[4]], [g, u], Wg_h[0].nbytes, ids, nexp, xb, F, H, T, False)
    hq = qmm.XQ8Buf(T * nexp, F)
    qmm.moe_silu_quant(g, u, hq, T * nexp, F)
    y = torch.zeros((T, H), device="cuda")
    qmm.gemv_moe(synth.Q4_K, synth.Q4_K, [W[2]], [W[5]], [y], Wd_h[0].nbytes, ids, nexp, hq, H, F, T, True, slotw=w)
    # two launches
    ids2 = torch.full((T, nexp), -7, dtype=torch.int32, device="cuda")
    w2 = torch.zeros((T, nexp), dtype=torch.float32, device="cuda")
    ws = torch.zeros(qmm.moe_decode_ws_bytes(T, 10, F) // 4, dtype=torch.float32, device="cuda")
    y2 = torch.full((T, H), float("nan"), device="cuda")
    qmm.moe_decode(synth.Q4_K, W[0], W[1], W[2], Wg_h[0].nbytes, Wd_h[0].nbytes, W[3], W[4], W[5], lg, n_exp + 1, n_exp, 10, xb,
                   T, H, F, ids2, w2, ws, y2)
    assert np.array_equal(host(ids2), host(ids))
    assert np.array_equal(host(w2).view(np.uint32), host(w).view(np.uint32))
    assert np.array_equal(host(y2).view(np.uint32), host(y).view(np.uint32))
    NS = T * nexp
    hb = host(ws).view(np.uint8)   # the first launch writes h as q8 (as moe_silu_quant does) to the workspace
    assert np.array_equal(hb[:NS * F].view(np.int8), host(hq.q).reshape(-1))
    nsb = NS * F // 32
    assert np.array_equal(hb[NS * F:NS * F + 8 * nsb].view(np.float32), np.concatenate([host(hq.d).reshape(-1), host(hq.s).reshape(-1)]))
    _, y_ref = oracle.moe_down_q8(synth.Q4_K, Wd_h, Sd_h, host(hq.q), host(hq.d), host(ids), host(w), H, F)
    assert rel_l2(host(y2), y_ref) <= 1e-5
    with pytest.raises(qmm.QmmError, match="WORKSPACE"):
        qmm.moe_decode(synth.Q4_K, W[0], W[1], W[2], Wg_h[0].nbytes, Wd_h[0].nbytes, W[3], W[4], W[5], lg, n_exp + 1, n_exp, 10,
                       xb, T, H, F, ids2, w2, ws[:8], y2)
