"""GPU parity of the MoE prefill path: device expert sort (bit-exact against the oracle's restatement
of qwen4exp.cpp:628-641), the grouped expert GEMM (within rel-L2 2e-3 of a torch float32 product of
the exactly dequantised bf16 experts) and the whole config-4 pipeline against the oracle's bf16 path."""
import numpy as np
import pytest
import torch

import oracle
from hipster_amd import qmm, synth
from tests.gpu_util import dev, host, rel_l2

pytestmark = pytest.mark.gpu
H, F, NE = 2048, 512, 11


def bf16_dev(a_bits):
    return torch.from_numpy(np.ascontiguousarray(a_bits).view(np.int16)).cuda().view(torch.bfloat16)


def sort_on_gpu(ids_h, n_exp, maxc=qmm.MOE_TILE_ROWS):
    T, nslot = ids_h.shape
    cap = qmm.moe_tiles_capacity(T, nslot, n_exp, maxc)
    kpos = torch.full((T * nslot,), -7, dtype=torch.int32, device="cuda")
    rowtok = torch.full((T * nslot,), -7, dtype=torch.int32, device="cuda")
    tiles = torch.full((cap, 3), -7, dtype=torch.int32, device="cuda")
    counts = torch.zeros(2, dtype=torch.int32, device="cuda")
    qmm.moe_sort(dev(ids_h), T, nslot, n_exp, maxc, kpos, rowtok, tiles, counts)
    return kpos, rowtok, tiles, counts, cap


@pytest.mark.parametrize("T,n_exp,zipf,maxc", [(1, 512, None, 64), (7, 64, None, 16), (2048, 512, 1.1, 64),
                                               (2048, 512, None, 64), (300, 1000, 1.1, 32), (4096, 512, 1.1, 128),
                                               (8192, 1000, 1.1, 128), (777, 128, 1.1, 16)])
def test_moe_sort_matches_oracle(gpu, T, n_exp, zipf, maxc):
    """one workgroup for small slot counts, several (count / offsets / scatter) for large ones:
    kpos, rowtok and the tiles bit-exact against the oracle either way"""
    ids_h, _ = oracle.moe_route(synth.router_logits(1400 + T, T, n_exp, zipf), n_exp, 10)
    kpos, rowtok, tiles, counts, _ = sort_on_gpu(ids_h, n_exp, maxc)
    kp, rt, tl, st = oracle.moe_sort(ids_h, maxc)
    c = host(counts)
    assert np.array_equal(host(kpos), kp) and np.array_equal(host(rowtok), rt)
    assert c[0] == len(tl) and c[1] == len(st)
    th = host(tiles)
    assert np.array_equal(th[:c[0]], tl) and np.array_equal(th[c[0]:c[0] + c[1]], st)


def test_moe_sort_degenerate_routing(gpu):
    """every token routed to the same experts (one giant run), and a batch of one slot per token"""
    T = 1000
    ids_h = np.tile(np.array([[5, 3, 511, 0, -1]], np.int32), (T, 1))
    kpos, rowtok, tiles, counts, _ = sort_on_gpu(ids_h, 512)
    kp, rt, tl, st = oracle.moe_sort(ids_h, qmm.MOE_TILE_ROWS)
    c = host(counts)
    assert np.array_equal(host(kpos), kp) and np.array_equal(host(rowtok), rt)
    assert np.array_equal(host(tiles)[:c[0] + c[1]], np.concatenate([tl, st]))


def test_moe_sort_refuses_tiles_over_128_rows(gpu):
    ids = torch.zeros((4, 11), dtype=torch.int32, device="cuda")
    with pytest.raises(qmm.QmmError, match="SHAPE"):
        sort_on_gpu(host(ids), 512, maxc=qmm.MOE_TILE_ROWS + 1)
    assert qmm.MOE_TILE_ROWS == 128


def test_moe_sort_clamps_out_of_range_ids(gpu):
    """ids outside [-1, n_exp-1] (a corrupt router output) sort as the nearest valid id: no index
    leaves the buffers, and the result is the oracle's sort of the clamped ids"""
    n_exp = 64
    ids_h, _ = oracle.moe_route(synth.router_logits(1490, 300, n_exp, None), n_exp, 10)
    bad = ids_h.copy()
    bad[::7, 3] = 5000
    bad[::11, 5] = -9
    kpos, rowtok, tiles, counts, _ = sort_on_gpu(bad, n_exp)
    kp, rt, tl, st = oracle.moe_sort(np.clip(bad, -1, n_exp - 1), qmm.MOE_TILE_ROWS)
    c = host(counts)
    assert np.array_equal(host(kpos), kp) and np.array_equal(host(rowtok), rt)
    assert np.array_equal(host(tiles)[:c[0] + c[1]], np.concatenate([tl, st]))


def dequant_experts_f32(Wd, n_exp, N, K):
    out = torch.zeros((n_exp, N, K), dtype=torch.int16, device="cuda")
    for e in range(n_exp):
        qmm.dequant_bf16(synth.Q4_K, Wd[e].contiguous(), out[e], N, K)
    return out.view(torch.bfloat16).float()


@pytest.mark.parametrize("T,N,K,gather,maxc", [(96, F, H, True, 128), (300, H, F, False, 128), (64, 512, 768, True, 128),
                                                (200, 384, 512, True, 64), (150, F, 1024, True, 16),
                                                (120, 256, 512, False, 96)])
def test_moe_gemm_bf16_matches_torch(gpu, T, N, K, gather, maxc):
    """tiles of 128, 96, 64 and 16 rows (one to four 32-row MFMA blocks, ragged last tiles), weight
    row counts that are not a multiple of the 256-row workgroup block"""
    n_exp = 32
    W_h = synth.experts(1410 + N, synth.Q4_K, n_exp, N, K)
    S_h = synth.matrix(1411 + N, synth.Q4_K, N, K)
    ids_h, _ = oracle.moe_route(synth.router_logits(1412 + T, T, n_exp, 1.1), n_exp, 10)
    kpos, rowtok, tiles, counts, cap = sort_on_gpu(ids_h, n_exp, maxc)
    NS = T * NE
    rows_a = T if gather else NS
    A = bf16_dev(synth.to_bf16_bits(synth.normal_f32(1413, (rows_a, K))))
    D = torch.full((NS, N), float("nan"), device="cuda")
    Wd, Sd = dev(W_h), dev(S_h)
    qmm.moe_gemm_bf16(synth.Q4_K, synth.Q4_K, Wd, Sd, W_h[0].nbytes, tiles, counts, cap, rowtok if gather else None, A, D, N, K)
    Wf = dequant_experts_f32(Wd, n_exp, N, K)
    Sf = dequant_experts_f32(Sd.view(1, N, -1), 1, N, K)[0]
    rt = host(rowtok)
    kp = host(kpos)
    ref = torch.zeros((NS, N), device="cuda")
    Af = A.float()
    for te in range(NS):
        e = ids_h.reshape(-1)[te]
        k = kp[te]
        arow = Af[rt[k]] if gather else Af[k]
        ref[k] = torch.mv((Wf[e] if e >= 0 else Sf), arow)
    err = rel_l2(host(D), host(ref))
    print(f"moe_gemm_bf16 T={T} N={N} K={K} maxc={maxc} rel-L2 {err:.2e}", flush=True)
    assert err <= 2e-3


@pytest.mark.parametrize("T,N,K,maxc", [(300, F, H, 128), (77, 384, 512, 32), (2048, F, H, 128)])
def test_moe_gate_up_fused_equals_unfused(gpu, T, N, K, maxc):
    """qmm_moe_gemm_gate_up_bf16 == moe_gemm_bf16(gate), moe_gemm_bf16(up), moe_silu_bf16, bit for bit"""
    n_exp = 64
    Wg_h, Wu_h = synth.experts(1440, synth.Q4_K, n_exp, N, K), synth.experts(1441, synth.Q4_K, n_exp, N, K)
    Sg_h, Su_h = synth.matrix(1442, synth.Q4_K, N, K), synth.matrix(1443, synth.Q4_K, N, K)
    ids_h, _ = oracle.moe_route(synth.router_logits(1444 + T, T, n_exp, 1.1), n_exp, 10)
    kpos, rowtok, tiles, counts, cap = sort_on_gpu(ids_h, n_exp, maxc)
    NS = T * NE
    A = bf16_dev(synth.to_bf16_bits(synth.normal_f32(1445, (T, K))))
    Wg, Wu, Sg, Su = (dev(a) for a in (Wg_h, Wu_h, Sg_h, Su_h))
    g = torch.zeros((NS, N), device="cuda"); u = torch.zeros((NS, N), device="cuda")
    qmm.moe_gemm_bf16(synth.Q4_K, synth.Q4_K, Wg, Sg, Wg_h[0].nbytes, tiles, counts, cap, rowtok, A, g, N, K)
    qmm.moe_gemm_bf16(synth.Q4_K, synth.Q4_K, Wu, Su, Wu_h[0].nbytes, tiles, counts, cap, rowtok, A, u, N, K)
    h_ref = torch.zeros((NS, N), dtype=torch.bfloat16, device="cuda")
    qmm.moe_silu_bf16(g, u, h_ref, NS * N)
    h = torch.full((NS, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    qmm.moe_gemm_gate_up_bf16(synth.Q4_K, synth.Q4_K, Wg, Sg, Wu, Su, Wg_h[0].nbytes, tiles, counts, cap, rowtok, A, h, N, K)
    a, b = host(h.view(torch.int16)), host(h_ref.view(torch.int16))
    print(f"gate/up fused T={T} N={N} K={K} maxc={maxc}: {int((a != b).sum())} differing of {a.size}", flush=True)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("N,K", [(F, H), (640, 768)])
def test_moe_gemm_bf16_tile_size_invariant(gpu, N, K):
    """the sorted positions do not depend on the tile size, and neither do the results: every output
    element is the same MFMA sequence whether its tile has 128, 64 or 32 rows (four, two or one 32-row
    MFMA blocks) -- bit for bit, gate/up fused as well"""
    T, n_exp = 700, 24
    W_h, S_h = synth.experts(1450 + N, synth.Q4_K, n_exp, N, K), synth.matrix(1451 + N, synth.Q4_K, N, K)
    U_h, SU_h = synth.experts(1452 + N, synth.Q4_K, n_exp, N, K), synth.matrix(1453 + N, synth.Q4_K, N, K)
    ids_h, _ = oracle.moe_route(synth.router_logits(1454 + N, T, n_exp, 1.1), n_exp, 10)
    A = bf16_dev(synth.to_bf16_bits(synth.normal_f32(1455, (T, K))))
    Wd, Sd, Ud, SUd = dev(W_h), dev(S_h), dev(U_h), dev(SU_h)
    outs, hs = [], []
    for maxc in (128, 64, 32):
        kpos, rowtok, tiles, counts, cap = sort_on_gpu(ids_h, n_exp, maxc)
        D = torch.full((T * NE, N), float("nan"), device="cuda")
        qmm.moe_gemm_bf16(synth.Q4_K, synth.Q4_K, Wd, Sd, W_h[0].nbytes, tiles, counts, cap, rowtok, A, D, N, K)
        h = torch.full((T * NE, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        qmm.moe_gemm_gate_up_bf16(synth.Q4_K, synth.Q4_K, Wd, Sd, Ud, SUd, W_h[0].nbytes, tiles, counts, cap, rowtok, A, h, N, K)
        outs.append(host(D).view(np.int32))
        hs.append(host(h.view(torch.int16)))
        print(f"tile-size invariance N={N} K={K} maxc={maxc}: "
              f"{int((outs[-1] != outs[0]).sum())} / {int((hs[-1] != hs[0]).sum())} differing", flush=True)
    assert not np.isnan(host(D)).any()
    for o, hh in zip(outs[1:], hs[1:]):
        assert np.array_equal(o, outs[0]) and np.array_equal(hh, hs[0])


def test_moe_prefill_config4_pipeline(gpu):
    """2048 tokens, hidden 2048, 512 Q4_K experts + shared, top-10 with the Zipf
    bias.  Device pipeline: route -> sort -> gate/up/silu (one launch) -> down -> combine; 12 sampled tokens
    against the oracle's bf16 path (bf16 weights and activations, double accumulation): every 8th token
    and the edges (266 tokens)."""
    T, n_exp = 2048, 512
    Wg_h, Wu_h, Wd_h = (synth.experts(1420 + i, synth.Q4_K, n_exp, *s) for i, s in enumerate(((F, H), (F, H), (H, F))))
    Sg_h, Su_h, Sd_h = (synth.matrix(1425 + i, synth.Q4_K, *s) for i, s in enumerate(((F, H), (F, H), (H, F))))
    x_bits = synth.to_bf16_bits(synth.normal_f32(1430, (T, H)))
    logits = synth.router_logits(1431, T, n_exp, 1.1)
    Wg, Wu, Wd, Sg, Su, Sd = (dev(a) for a in (Wg_h, Wu_h, Wd_h, Sg_h, Su_h, Sd_h))
    x = bf16_dev(x_bits)
    ids = torch.zeros((T, NE), dtype=torch.int32, device="cuda")
    w = torch.zeros((T, NE), device="cuda")
    qmm.moe_route(dev(logits), ids, w, T)
    NS = T * NE
    cap = qmm.moe_tiles_capacity(T, NE, n_exp)
    kpos = torch.zeros(NS, dtype=torch.int32, device="cuda"); rowtok = torch.zeros(NS, dtype=torch.int32, device="cuda")
    tiles = torch.zeros((cap, 3), dtype=torch.int32, device="cuda"); counts = torch.zeros(2, dtype=torch.int32, device="cuda")
    qmm.moe_sort(ids, T, NE, n_exp, qmm.MOE_TILE_ROWS, kpos, rowtok, tiles, counts)
    h = torch.zeros((NS, F), dtype=torch.bfloat16, device="cuda")
    qmm.moe_gemm_gate_up_bf16(synth.Q4_K, synth.Q4_K, Wg, Sg, Wu, Su, Wg_h[0].nbytes, tiles, counts, cap, rowtok, x, h, F, H)
    dn = torch.zeros((NS, H), device="cuda")
    qmm.moe_gemm_bf16(synth.Q4_K, synth.Q4_K, Wd, Sd, Wd_h[0].nbytes, tiles, counts, cap, None, h, dn, H, F)
    y = torch.zeros((T, H), device="cuda")
    qmm.moe_combine_sorted(dn, w, kpos, y, T, NE, H)
    ids_h, w_h = host(ids), host(w)
    toks = np.unique(np.concatenate([np.arange(0, T, 8), [1, 2, 511, 777, 1023, 1025, 1500, 2045, 2046, 2047]])).astype(np.int32)
    y_ref = oracle.moe_prefill_tokens(synth.Q4_K, Wg_h, Wu_h, Wd_h, Sg_h, Su_h, Sd_h, x_bits, ids_h, w_h, H, F, toks)
    err = rel_l2(host(y)[toks], y_ref)
    print(f"config-4 MoE prefill, {len(toks)} sampled tokens rel-L2 {err:.2e}", flush=True)
    assert err <= 2e-3


def test_moe_prefill_pipeline_every_token_against_oracle(gpu):
    """The whole device pipeline (route, sort, gate/up/silu, down, combine) at 300 tokens over 64 Q4_K
    experts + shared with the Zipf bias (small and full tiles, several tiles for the popular experts):
    every token against the oracle's bf16 path."""
    T, n_exp = 300, 64
    Wg_h, Wu_h, Wd_h = (synth.experts(1460 + i, synth.Q4_K, n_exp, *s) for i, s in enumerate(((F, H), (F, H), (H, F))))
    Sg_h, Su_h, Sd_h = (synth.matrix(1465 + i, synth.Q4_K, *s) for i, s in enumerate(((F, H), (F, H), (H, F))))
    x_bits = synth.to_bf16_bits(synth.normal_f32(1470, (T, H)))
    logits = synth.router_logits(1471, T, n_exp, 1.1)
    Wg, Wu, Wd, Sg, Su, Sd = (dev(a) for a in (Wg_h, Wu_h, Wd_h, Sg_h, Su_h, Sd_h))
    ids = torch.zeros((T, NE), dtype=torch.int32, device="cuda")
    w = torch.zeros((T, NE), device="cuda")
    qmm.moe_route_n(dev(logits), ids, w, T, n_exp, n_exp + 1, 10)
    NS = T * NE
    cap = qmm.moe_tiles_capacity(T, NE, n_exp)
    kpos = torch.zeros(NS, dtype=torch.int32, device="cuda"); rowtok = torch.zeros(NS, dtype=torch.int32, device="cuda")
    tiles = torch.zeros((cap, 3), dtype=torch.int32, device="cuda"); counts = torch.zeros(2, dtype=torch.int32, device="cuda")
    qmm.moe_sort(ids, T, NE, n_exp, qmm.MOE_TILE_ROWS, kpos, rowtok, tiles, counts)
    h = torch.zeros((NS, F), dtype=torch.bfloat16, device="cuda")
    qmm.moe_gemm_gate_up_bf16(synth.Q4_K, synth.Q4_K, Wg, Sg, Wu, Su, Wg_h[0].nbytes, tiles, counts, cap, rowtok, bf16_dev(x_bits),
                              h, F, H)
    dn = torch.zeros((NS, H), device="cuda")
    qmm.moe_gemm_bf16(synth.Q4_K, synth.Q4_K, Wd, Sd, Wd_h[0].nbytes, tiles, counts, cap, None, h, dn, H, F)
    y = torch.zeros((T, H), device="cuda")
    qmm.moe_combine_sorted(dn, w, kpos, y, T, NE, H)
    toks = np.arange(T, dtype=np.int32)
    y_ref = oracle.moe_prefill_tokens(synth.Q4_K, Wg_h, Wu_h, Wd_h, Sg_h, Su_h, Sd_h, x_bits, host(ids), host(w), H, F, toks)
    err = rel_l2(host(y), y_ref)
    print(f"MoE prefill T={T} E={n_exp}: every token rel-L2 {err:.2e}, tiles {host(counts).tolist()}", flush=True)
    assert err <= 2e-3
