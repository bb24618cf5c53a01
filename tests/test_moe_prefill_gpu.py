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
                                               (2048, 512, None, 64), (300, 1000, 1.1, 32)])
def test_moe_sort_matches_oracle(gpu, T, n_exp, zipf, maxc):
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


def dequant_experts_f32(Wd, n_exp, N, K):
    out = torch.zeros((n_exp, N, K), dtype=torch.int16, device="cuda")
    for e in range(n_exp):
        qmm.dequant_bf16(synth.Q4_K, Wd[e].contiguous(), out[e], N, K)
    return out.view(torch.bfloat16).float()


@pytest.mark.parametrize("T,N,K,gather", [(96, F, H, True), (300, H, F, False), (64, 512, 768, True)])
def test_moe_gemm_bf16_matches_torch(gpu, T, N, K, gather):
    n_exp = 32
    W_h = synth.experts(1410 + N, synth.Q4_K, n_exp, N, K)
    S_h = synth.matrix(1411 + N, synth.Q4_K, N, K)
    ids_h, _ = oracle.moe_route(synth.router_logits(1412 + T, T, n_exp, 1.1), n_exp, 10)
    kpos, rowtok, tiles, counts, cap = sort_on_gpu(ids_h, n_exp)
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
    print(f"moe_gemm_bf16 T={T} N={N} K={K} rel-L2 {err:.2e}", flush=True)
    assert err <= 2e-3


def test_moe_prefill_config4_pipeline(gpu):
    """2048 tokens, hidden 2048, 512 Q4_K experts + shared, top-10 with the Zipf
    bias.  Device pipeline: route -> sort -> gate, up -> silu -> down -> combine; 12 sampled tokens
    against the oracle's bf16 path (bf16 weights and activations, double accumulation)."""
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
    g = torch.zeros((NS, F), device="cuda"); u = torch.zeros((NS, F), device="cuda")
    qmm.moe_gemm_bf16(synth.Q4_K, synth.Q4_K, Wg, Sg, Wg_h[0].nbytes, tiles, counts, cap, rowtok, x, g, F, H)
    qmm.moe_gemm_bf16(synth.Q4_K, synth.Q4_K, Wu, Su, Wu_h[0].nbytes, tiles, counts, cap, rowtok, x, u, F, H)
    h = torch.zeros((NS, F), dtype=torch.bfloat16, device="cuda")
    qmm.moe_silu_bf16(g, u, h, NS * F)
    dn = torch.zeros((NS, H), device="cuda")
    qmm.moe_gemm_bf16(synth.Q4_K, synth.Q4_K, Wd, Sd, Wd_h[0].nbytes, tiles, counts, cap, None, h, dn, H, F)
    y = torch.zeros((T, H), device="cuda")
    qmm.moe_combine_sorted(dn, w, kpos, y, T, NE, H)
    ids_h, w_h = host(ids), host(w)
    toks = np.array([0, 1, 2, 100, 511, 777, 1000, 1024, 1500, 2000, 2046, 2047], np.int32)
    y_ref = oracle.moe_prefill_tokens(synth.Q4_K, Wg_h, Wu_h, Wd_h, Sg_h, Su_h, Sd_h, x_bits, ids_h, w_h, H, F, toks)
    err = rel_l2(host(y)[toks], y_ref)
    print(f"config-4 MoE prefill, sampled tokens rel-L2 {err:.2e}", flush=True)
    assert err <= 2e-3
