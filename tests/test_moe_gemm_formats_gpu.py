"""GPU parity of the prefill grouped expert GEMM (qmm_moe_gemm_bf16) for the reference's other expert
formats (engine/kernels/gemv.hip:954-969,1377-1381: Q4_K, Q5_K, Q5_1_SOA, Q8_0_SOA, the routed and the
shared expert formats independent; IQ4_XS too), including the engine's expert FF 640 (qwen4exp.h:22):
down projections with K = 640 in the 32-weight formats.

Bar (bf16 MFMA path): rel-L2 <= 2e-3 against a torch float32 product of the
same bf16 activations and the exactly dequantised bf16 experts (the dequantisation itself is pinned bit
for bit: qmm_dequant_bf16 against the oracle, which the reference's own quant.h pins).  Measured
errors are ~1e-7 (f32 accumulation of exact bf16 products); the test prints them.
"""
import numpy as np
import pytest
import torch

import oracle
from hipster_amd import qmm, synth
from tests.gpu_util import dev, host, rel_l2
from tests.test_moe_prefill_gpu import bf16_dev, sort_on_gpu

pytestmark = pytest.mark.gpu
NE = 11


def dequant_dev(fmt, W, N, K):
    """bf16 [N][K] on the device via qmm_dequant_bf16 (bit-exact), as float32."""
    out = torch.zeros((N, K), dtype=torch.int16, device="cuda")
    qmm.dequant_bf16(fmt, W, out, N, K)
    return out.view(torch.bfloat16).float()


@pytest.mark.parametrize("fmt,sfmt,N,K,gather", [
    (synth.Q5_1_SOA, synth.Q5_1_SOA, 512, 640, False),     # the engine's down projection shape, scaled
    (synth.Q8_0_SOA, synth.Q5_1_SOA, 512, 640, False),
    (synth.Q5_1_SOA, synth.Q8_0_SOA, 640, 512, True),
    (synth.Q5_K, synth.Q5_K, 640, 512, True),
    (synth.Q5_K, synth.Q8_0_SOA, 640, 512, True),
    (synth.Q4_K, synth.Q8_0_SOA, 384, 512, True),
    (synth.Q8_0_SOA, synth.Q4_K, 256, 512, False),
    (synth.IQ4_XS, synth.IQ4_XS, 200, 256, True),
    (synth.Q5_1_SOA, synth.Q5_1_SOA, 130, 96, True),
])
def test_moe_gemm_formats_match_torch(gpu, fmt, sfmt, N, K, gather):
    n_exp, T = 24, 150
    W_h = synth.experts(1600 + fmt, fmt, n_exp, N, K)
    S_h = synth.matrix(1601 + sfmt, sfmt, N, K)
    ids_h, _ = oracle.moe_route(synth.router_logits(1602 + T, T, n_exp, 1.1), n_exp, 10)
    kpos, rowtok, tiles, counts, cap = sort_on_gpu(ids_h, n_exp, 128)
    NS = T * NE
    rows_a = T if gather else NS
    A = bf16_dev(synth.to_bf16_bits(synth.normal_f32(1603, (rows_a, K))))
    D = torch.full((NS, N), float("nan"), device="cuda")
    Wd, Sd = dev(W_h), dev(S_h)
    qmm.moe_gemm_bf16(fmt, sfmt, Wd, Sd, W_h[0].nbytes, tiles, counts, cap, rowtok if gather else None, A, D, N, K)
    Wf = [dequant_dev(fmt, Wd[e], N, K) for e in range(n_exp)]
    Sf = dequant_dev(sfmt, Sd, N, K)
    rt, kp = host(rowtok), host(kpos)
    Af = A.float()
    ref = torch.zeros((NS, N), device="cuda")
    for te in range(NS):
        e = ids_h.reshape(-1)[te]
        k = kp[te]
        ref[k] = torch.mv(Wf[e] if e >= 0 else Sf, Af[rt[k]] if gather else Af[k])
    got = host(D)
    assert not np.isnan(got).any()
    err = rel_l2(got, host(ref))
    print(f"moe_gemm fmt={fmt} shared={sfmt} N={N} K={K} rel-L2 {err:.2e}", flush=True)
    assert err <= 2e-3


def test_dequant_bf16_soa_k_granules(gpu):
    """qmm_dequant_bf16 at the SoA formats' own K granules (K = 640, 96) against the oracle, bit for bit."""
    for fmt, N, K in ((synth.Q5_1_SOA, 33, 640), (synth.Q8_0_SOA, 17, 640), (synth.Q5_1_SOA, 9, 96), (synth.Q8_0_SOA, 5, 192)):
        W = synth.matrix(1610 + K + fmt, fmt, N, K)
        out = torch.zeros((N, K), dtype=torch.int16, device="cuda")
        qmm.dequant_bf16(fmt, dev(W), out, N, K)
        assert np.array_equal(host(out).view(np.uint16), oracle.dequant_rows_bf16(fmt, W, K)), (fmt, K)
