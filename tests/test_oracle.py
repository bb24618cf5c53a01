"""CPU tests that pin the oracle (oracle/qmm_oracle.c) before it is trusted as the GPU checker.

Each oracle function is pinned by something a plausible mistake would fail:
  * dequant (Q4_K, Q6_K, Q6_K SoA), f16->f32, scale/min unpack: bit-exact against golden vectors
    written by the reference's own engine/src/quant.h (tests/golden/make_golden.py), and against the
    compiled reference itself when oracle/_ref is present;
  * known-answer blocks (closed forms) and the Q6_K signed-byte identity by brute force;
  * x quantiser: closed forms (amax element -> +-127, round-half-even ties, amax = 0);
  * GEMV reference: one-hot activations reproduce the golden dequantised columns bit-exactly;
    linearity; sampled-row variant equal to the full one;
  * routing: brute force (full sort in float64) incl. planted ties;
  * expert sort/tiles: numpy stable argsort + structural invariants;
  * MoE decode/prefill and the dense prefill GEMM references: one-hot routing weights, linearity,
    and numpy float64 recomputation from the pinned pieces on small shapes.
"""
import numpy as np
import pytest

import oracle
from hipster_amd import synth

GOLD = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "quant_golden.npz"))


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ----------------------------------------------------------------------------- number formats
def test_f16_to_f32_all_halfs_match_reference():
    L = oracle.lib()
    got = np.array([L.qo_f16_to_f32(int(h)) for h in GOLD["f16_bits"]], dtype=np.float32)
    ref = GOLD["f16_f32"]
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(ref)[~nan])
    # and numpy's IEEE half conversion agrees on every non-NaN value (subnormals included)
    assert np.array_equal(bits(GOLD["f16_bits"].view(np.float16).astype(np.float32))[~nan], bits(ref)[~nan])


def test_bf16_round_nearest_even():
    L = oracle.lib()
    cases = {1.0: 0x3F80, 1.00390625: 0x3F80, 1.01171875: 0x3F82, -2.0: 0xC000, 0.0: 0x0000,
             float(np.float32(1.0) + np.float32(2 ** -8)): 0x3F80,   # exact tie -> even
             float(np.float32(1.0) + np.float32(3 * 2 ** -8)): 0x3F82}
    for v, want in cases.items():
        assert L.qo_f32_to_bf16(v) == want, v
    x = synth.normal_f32(5, 4096)
    np.testing.assert_array_equal(np.array([L.qo_f32_to_bf16(float(v)) for v in x[:512]], np.uint16),
                                  synth.to_bf16_bits(x[:512]))


# ----------------------------------------------------------------------------- blocks
def test_scale_min_k4_matches_reference():
    L = oracle.lib()
    import ctypes
    for i in range(GOLD["scale_in"].shape[0]):
        s = np.ascontiguousarray(GOLD["scale_in"][i])
        for j in range(8):
            d = ctypes.c_uint8(); m = ctypes.c_uint8()
            L.qo_scale_min_k4(j, s.ctypes.data, ctypes.addressof(d), ctypes.addressof(m))
            assert (d.value, m.value) == tuple(GOLD["scale_out"][i, j])


@pytest.mark.parametrize("fmt,key", [(oracle.Q4_K, "q4k"), (oracle.Q6_K, "q6k")])
def test_dequant_matches_reference_golden(fmt, key):
    blocks = GOLD[key + "_blocks"]
    y = oracle.dequant_rows(fmt, blocks, 256)
    assert np.array_equal(bits(y), bits(GOLD[key + "_y"]))


def test_dequant_q6k_soa_matches_reference_golden():
    blocks = GOLD["q6k_blocks"]
    # 5 blocks per row so the SoA streams interleave several blocks
    n = blocks.shape[0] // 5 * 5
    W = blocks[:n].reshape(n // 5, 5 * 210)
    soa = synth.repack_q6k_soa(W, 5 * 256)
    y = oracle.dequant_rows(oracle.Q6_K_SOA, soa, 5 * 256)
    assert np.array_equal(bits(y.reshape(-1, 256)), bits(GOLD["q6k_y"][:n]))


def test_repack_q6k_matches_oracle_restatement():
    W = synth.matrix(3, synth.Q6_K, 3, 1024)
    soa = synth.repack_q6k_soa(W, 1024)
    L = oracle.lib()
    for r in range(3):
        out = np.empty(W.shape[1], np.uint8)
        src = np.ascontiguousarray(W[r])
        L.qo_repack_row_q6_K(src.ctypes.data, out.ctypes.data, 1024)
        assert np.array_equal(out, soa[r])


def test_dequant_known_answers():
    q4 = GOLD["q4k_blocks"]
    y = oracle.dequant_rows(oracle.Q4_K, q4[:2], 256)
    assert np.all(y[0] == 0.0)
    want = np.tile(np.concatenate([np.full(32, 1.0), np.full(32, 2.0)]), 4).astype(np.float32)
    assert np.array_equal(y[1], want)
    y6 = oracle.dequant_rows(oracle.Q6_K, GOLD["q6k_blocks"][:2], 256)
    assert np.all(y6[0] == -32.0) and np.all(y6[1] == 31.0)


def test_dequant_random_blocks_vs_compiled_reference():
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    for fmt, gtype, gen in ((oracle.Q4_K, 12, synth.q4k_blocks), (oracle.Q6_K, 14, synth.q6k_blocks)):
        blocks = gen(synth.rng(99), 2000)
        W = blocks.reshape(100, -1)
        y = oracle.dequant_rows(fmt, W, 20 * 256)
        r = np.empty_like(y)
        for i in range(W.shape[0]):
            row = np.ascontiguousarray(W[i])
            ref.ref_dequant_row(gtype, row.ctypes.data, r[i].ctypes.data, 20 * 256)
        assert np.array_equal(bits(y), bits(r))


def test_q6_signed_byte_identity_brute_force():
    q = np.arange(64, dtype=np.uint32)
    packed = (q | (q << 8) | (q << 16) | (q << 24)).astype(np.uint32)
    conv = ((packed + np.uint32(0x60606060)) ^ np.uint32(0x80808080)).astype(np.uint32)
    b = conv.view(np.uint8).reshape(64, 4).view(np.int8)
    assert np.array_equal(b, np.repeat((q.astype(np.int64) - 32)[:, None], 4, axis=1))


# ----------------------------------------------------------------------------- activations
def test_quantize_x_q8_closed_forms():
    x = synth.normal_f32(11, (3, 512))
    x[1, :32] = 0.0                        # amax = 0 block
    x[2, :32] = np.arange(32) - 16.0       # amax 16
    q, d, s = oracle.quantize_x_q8(x)
    assert np.all(q[1, :32] == 0) and d[1, 0] == 0 and s[1, 0] == 0
    for c in range(3):
        for b in range(x.shape[1] // 32):
            blk = x[c, 32 * b:32 * b + 32]
            amax = np.float32(np.max(np.abs(blk)))
            if amax == 0:
                continue
            assert d[c, b] == np.float32(amax / np.float32(127.0))
            qb = q[c, 32 * b:32 * b + 32].astype(np.int32)
            assert np.max(np.abs(qb)) == 127
            assert qb[np.argmax(np.abs(blk))] == np.sign(blk[np.argmax(np.abs(blk))]) * 127
            idf = np.float32(127.0) / amax
            scaled = (blk * idf).astype(np.float32)
            assert np.all(np.abs(qb - scaled) <= 0.5)
            assert np.array_equal(qb, np.rint(scaled).astype(np.int32))        # numpy rint = half-even
            assert s[c, b] == np.float32(d[c, b] * np.float32(qb.sum()))


def test_quantize_x_q8_ties_round_to_even():
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 127.0                        # amax 127 -> id = 1 exactly
    x[0, 1:6] = [2.5, 3.5, -2.5, -0.5, 0.5]
    q, d, s = oracle.quantize_x_q8(x)
    assert list(q[0, :6]) == [127, 2, 4, -2, 0, 0]


# ----------------------------------------------------------------------------- GEMV reference
@pytest.mark.parametrize("fmt,key,blk", [(oracle.Q4_K, "q4k", 144), (oracle.Q6_K, "q6k", 210)])
def test_gemv_ref_one_hot_columns_equal_golden(fmt, key, blk):
    blocks = GOLD[key + "_blocks"][:250]
    W = blocks.reshape(50, 5 * blk)            # 50 rows, K = 1280
    K = 1280
    gold = GOLD[key + "_y"][:250].reshape(50, K)
    ks = [0, 1, 31, 32, 63, 64, 200, 255, 256, 777, 1279]
    x = np.zeros((len(ks), K), np.float32)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    y, mag = oracle.gemv_ref(fmt, W, 50, K, x)
    for i, k in enumerate(ks):
        assert np.array_equal(y[i], gold[:, k].astype(np.float64))
        assert np.array_equal(mag[i], np.abs(gold[:, k]).astype(np.float64))


def test_gemv_ref_linear_and_rows_variant():
    W = synth.matrix(21, synth.Q4_K, 64, 1024)
    x = synth.normal_f32(22, (2, 1024))
    y, _ = oracle.gemv_ref(oracle.Q4_K, W, 64, 1024, x)
    y2, mag2 = oracle.gemv_ref(oracle.Q4_K, W, 64, 1024, (x[0] + x[1])[None])
    # x[0] + x[1] is rounded to f32, so linearity holds to ~1 ulp of the |w*x| sums
    assert np.all(np.abs(y2[0] - (y[0] + y[1])) <= 1e-6 * mag2[0])
    rows = [63, 0, 17]
    yr, _ = oracle.gemv_ref_rows(oracle.Q4_K, W, 64, 1024, x, rows)
    assert np.array_equal(yr, y[:, rows])
    yf = oracle.gemv_f32(oracle.Q4_K, W, 64, 1024, x, nthreads=3)
    np.testing.assert_allclose(yf, y, rtol=2e-5, atol=2e-5 * np.abs(y).max())
    # the reference-code CPU baseline (quant.h dequant_row + f32 dot, threaded) computes the same GEMV
    if oracle.ref_lib() is not None:
        for nt in (1, 3):
            yr = oracle.ref_gemv_f32(12, W, 64, 1024, x[0], nthreads=nt)
            np.testing.assert_allclose(yr, y[0], rtol=2e-5, atol=2e-5 * np.abs(y[0]).max())


# ----------------------------------------------------------------------------- routing / sort
def route_brute(logits, nexp=512, topk=10):
    T = logits.shape[0]
    ids = np.zeros((T, topk + 1), np.int32)
    w = np.zeros((T, topk + 1), np.float64)
    for t in range(T):
        l = logits[t, :nexp].astype(np.float64)
        p = np.exp(l - l.max()); p /= p.sum()
        order = sorted(range(nexp), key=lambda i: (-p[i], i))[:topk]
        ids[t, :topk] = order
        w[t, :topk] = p[order] / p[order].sum()
        ids[t, topk] = -1
        w[t, topk] = 1 / (1 + np.exp(-np.float64(logits[t, nexp])))
    return ids, w


def test_route_matches_brute_force():
    logits = synth.router_logits(31, 64)
    ids, w = oracle.moe_route(logits)
    bi, bw = route_brute(logits)
    assert np.array_equal(ids, bi)
    np.testing.assert_allclose(w, bw, rtol=2e-6, atol=1e-7)


def test_route_ties_go_to_lower_id_and_zipf():
    logits = synth.router_logits(32, 8, zipf_s=1.1)
    logits[0, :512] = -5.0
    logits[0, [400, 7, 300, 9]] = 3.0     # four-way tie on top
    logits[1, :512] = 0.0                 # all equal: ids 0..9
    ids, w = oracle.moe_route(logits)
    assert list(ids[0, :4]) == [7, 9, 300, 400]
    assert list(ids[1, :10]) == list(range(10)) and np.allclose(w[1, :10], 0.1)
    bi, bw = route_brute(logits)
    assert np.array_equal(ids, bi)


def test_route_selects_on_rounded_probabilities():
    """fn.hip:176-180: the argmax runs on p = exp(l - max) / sum as floats, ties to the lower id.  Logits
    0 and -2^-30 both give exp(.) = 1.0f (the exact value 1 - 9.3e-10 is far closer to 1 than to the
    next float below, 1 - 6e-8), so experts 3 (logit -2^-30) and 8 (logit 0, the larger) tie on p and
    the lower id, 3, is taken first; a rule on the logits would take 8 first."""
    logits = np.full((1, 65), -4.0, np.float32)
    logits[0, 8] = 0.0
    logits[0, 3] = -2.0 ** -30
    ids, w = oracle.moe_route(logits, 64, 4)
    assert list(ids[0, :2]) == [3, 8]
    assert w[0, 0] == w[0, 1]


def test_sort_tiles_invariants():
    logits = synth.router_logits(41, 300, zipf_s=1.1)
    ids, _ = oracle.moe_route(logits)
    T, NE = ids.shape
    for maxc in (16, 32, 48):
        kpos, rowtok, tiles, stiles = oracle.moe_sort(ids, maxc)
        flat = ids.reshape(-1)
        order = np.lexsort((np.arange(T * NE), flat))      # by (eid, te), stable
        assert np.array_equal(np.argsort(kpos), order)
        assert np.array_equal(rowtok, order // NE)
        assert sorted(kpos.tolist()) == list(range(T * NE))
        # shared slots first, then experts ascending
        assert np.all(flat[order][:T] == -1)
        covered = np.zeros(T * NE, np.int32)
        for e, k0, nc in np.concatenate([tiles, stiles]):
            assert 1 <= nc <= maxc
            assert np.all(flat[order][k0:k0 + nc] == e)
            covered[k0:k0 + nc] += 1
        assert np.all(covered == 1)
        # a new tile starts exactly at each expert boundary or after maxc columns
        for lst in (tiles, stiles):
            for a, b in zip(lst[:-1], lst[1:]):
                assert b[1] == a[1] + a[2]
                assert b[0] != a[0] or a[2] == maxc


# ----------------------------------------------------------------------------- MoE references
def _tiny_moe(seed, T=2, n_exp=6, H=512, F=256):
    Wg = synth.experts(seed, synth.Q4_K, n_exp, F, H)
    Wu = synth.experts(seed + 1, synth.Q4_K, n_exp, F, H)
    Wd = synth.experts(seed + 2, synth.Q4_K, n_exp, H, F)
    Sg, Su, Sd = (synth.experts(seed + 3 + i, synth.Q4_K, 1, *shape)[0] for i, shape in enumerate([(F, H), (F, H), (H, F)]))
    x = synth.normal_f32(seed + 9, (T, H))
    return Wg, Wu, Wd, Sg, Su, Sd, x


def test_moe_decode_one_hot_and_linearity():
    Wg, Wu, Wd, Sg, Su, Sd, x = _tiny_moe(50)
    T, H, F = 2, 512, 256
    ids = np.array([[3, 0, -1], [5, 3, -1]], np.int32)
    w = np.array([[1.0, 0.0, 0.0], [0.25, 0.5, 0.25]], np.float32)
    g, u, dn, y = oracle.moe_decode(oracle.Q4_K, Wg, Wu, Wd, Sg, Su, Sd, x, ids, w, H, F)
    np.testing.assert_allclose(y[0], dn[0], rtol=1e-6)            # one-hot weight -> that slot's output
    np.testing.assert_allclose(y[1], 0.25 * dn[3] + 0.5 * dn[4] + 0.25 * dn[5], rtol=1e-5, atol=1e-6)
    # gate of slot (t=0, e=0) is expert 3 applied to q8(x[0]), recomputed from pinned pieces
    q, d, _ = oracle.quantize_x_q8(x)
    xr = oracle.q8_to_f32(q, d)
    Wg3 = oracle.dequant_rows(oracle.Q4_K, Wg[3], H)
    np.testing.assert_allclose(g[0], (Wg3.astype(np.float64) @ xr[0].astype(np.float64)).astype(np.float32), rtol=1e-6)
    # slot 2 of token 1 is the shared expert
    Su0 = oracle.dequant_rows(oracle.Q4_K, Su, H)
    np.testing.assert_allclose(u[5], (Su0.astype(np.float64) @ xr[1]).astype(np.float32), rtol=1e-6)
    # down stage alone, fed the q8 of the same h, reproduces dn and y
    h = (g / (1 + np.exp(-g.astype(np.float64))) * u).astype(np.float32)
    hq, hd, _ = oracle.quantize_x_q8(h)
    dn2, y2 = oracle.moe_down_q8(oracle.Q4_K, Wd, Sd, hq, hd, ids, w, H, F)
    np.testing.assert_allclose(dn2, dn, rtol=1e-3, atol=1e-3 * np.abs(dn).max())


def test_moe_prefill_tokens_matches_float64_recompute():
    Wg, Wu, Wd, Sg, Su, Sd, x = _tiny_moe(60)
    T, H, F = 2, 512, 256
    xb = synth.to_bf16_bits(x)
    ids = np.array([[1, 4, -1], [2, 1, -1]], np.int32)
    w = np.array([[0.7, 0.3, 0.5], [0.6, 0.4, 0.9]], np.float32)
    y = oracle.moe_prefill_tokens(oracle.Q4_K, Wg, Wu, Wd, Sg, Su, Sd, xb, ids, w, H, F, [1, 0])
    xf = synth.bf16_bits_to_f32(xb).astype(np.float64)

    def deq(Wm, K):
        return synth.bf16_bits_to_f32(oracle.dequant_rows_bf16(oracle.Q4_K, Wm, K)).astype(np.float64)

    for i, t in enumerate([1, 0]):
        acc = np.zeros(H)
        for e in range(3):
            eid = ids[t, e]
            wg, wu, wd = (Wg[eid], Wu[eid], Wd[eid]) if eid >= 0 else (Sg, Su, Sd)
            gv = (deq(wg, H) @ xf[t]).astype(np.float32)
            uv = (deq(wu, H) @ xf[t]).astype(np.float32)
            hv = synth.bf16_bits_to_f32(synth.to_bf16_bits((gv / (1 + np.exp(-gv)) * uv).astype(np.float32)))
            acc += np.float64(w[t, e]) * (deq(wd, F) @ hv.astype(np.float64)).astype(np.float32)
        np.testing.assert_allclose(y[i], acc, rtol=1e-4, atol=1e-5 * np.abs(acc).max())


def test_gemm_wq_ref_matches_numpy():
    M, N, K = 5, 7, 512
    W = synth.matrix(70, synth.Q4_K, N, K)
    A = synth.to_bf16_bits(synth.normal_f32(71, (M, K)))
    ms = np.repeat(np.arange(M), N)
    ns = np.tile(np.arange(N), M)
    out = oracle.gemm_wq_ref(oracle.Q4_K, W, A, M, N, K, ms, ns)
    Wb = synth.bf16_bits_to_f32(oracle.dequant_rows_bf16(oracle.Q4_K, W, K)).astype(np.float64)
    Af = synth.bf16_bits_to_f32(A).astype(np.float64)
    np.testing.assert_allclose(out.reshape(M, N), Af @ Wb.T, rtol=1e-12, atol=1e-12)
    # the bf16 dequant is the RNE of the (golden-pinned) f32 dequant
    Wf = oracle.dequant_rows(oracle.Q4_K, W, K)
    assert np.array_equal(oracle.dequant_rows_bf16(oracle.Q4_K, W, K), synth.to_bf16_bits(Wf))


def test_quantize_x_q8k_pinned_to_q8():
    """Q8_K (one scale per 256) reduces to the pinned per-32 quantiser when every 32-sub-block of a 256-block
    holds the block's amax: then q, d agree with qo_quantize_x_q8 exactly and bs is the per-32 integer sum.
    Plus the closed forms: an all-zero block gives d = 0, q = 0; amax maps to +-127."""
    g = np.random.default_rng(5)
    K, ncol = 1024, 3
    x = g.standard_normal((ncol, K)).astype(np.float32)
    for c in range(ncol):
        for b in range(K // 256):
            blk = x[c, b * 256:(b + 1) * 256]
            amax = np.float32(np.abs(blk).max() * 1.5 + 0.25)
            for j in range(8):
                blk[32 * j + (j * 5) % 32] = amax if (j + b + c) % 2 else -amax
    x[2, 256:512] = 0.0                                  # an all-zero block
    q, d, bs = oracle.quantize_x_q8k(x)
    q8, d8, s8 = oracle.quantize_x_q8(x)
    assert np.array_equal(q, q8)
    for c in range(ncol):
        for b in range(K // 256):
            assert np.all(d8[c, 8 * b:8 * b + 8] == d[b, c])
            assert np.array_equal(bs[b, c], q8[c, 256 * b:256 * (b + 1)].reshape(8, 32).astype(np.int64).sum(axis=1))
    assert d[1, 2] == 0 and not q[2, 256:512].any() and not bs[1, 2].any()
    assert np.abs(q).max() == 127
    # columns beyond ncol untouched, and a column alone gives the same bits
    assert not d[:, ncol:].any()
    q1, d1, bs1 = oracle.quantize_x_q8k(x[1:2])
    assert np.array_equal(q1[0], q[1]) and np.array_equal(d1[:, 0], d[:, 1]) and np.array_equal(bs1[:, 0], bs[:, 1])
