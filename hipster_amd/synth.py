"""Seeded synthetic GGUF tensors and activations for the BASELINE configurations.

All randomness comes from ``numpy.random.Generator(PCG64(seed))`` so the bytes are identical
on every host running the same numpy.  Distributions:

* Q4_K block (engine/src/quant.h:22): d, dmin = fp16(|N(0, 0.01)|) (some fp16 subnormals
  appear), the 12 scale bytes and the 128 quant bytes uniform random bytes, which makes the 6-bit
  scales/mins and the 4-bit quants exactly uniform.
* Q6_K block (quant.h:24): ql, qh and the int8 scales uniform random bytes, d = fp16(|N(0, 0.01)|).
* The other formats of the call surface (quant.h:23,26-30), same recipe: every scale fp16(|N(0, 0.01)|)
  (the Q5_1 offset m fp16(N(0, 0.01)), signed), every other byte uniform random -- Q5_K (176 B / 256),
  IQ4_XS (136 B / 256), Q8_0 (34 B / 32), Q5_1 (24 B / 32), Q5_0 (22 B / 32), and the row-SoA
  repacks the engine makes of Q8_0 and Q5_1 / Q5_0 rows at load time.
* activations N(0, 1) f32 (or bf16 for the prefill configs).
* router logits N(0, 1); for the prefill MoE config plus a Zipf(s=1.1) bias
  b_e = -1.1 * ln(rank_e) with ranks a seeded permutation of 1..n_exp.
"""
import numpy as np

Q4K_BYTES = 144
Q6K_BYTES = 210
QK = 256

# format ids (include/hipster_qmm.h); 8, 9, 10 are the GGUF-native 32-weight block rows that the
# engine repacks into Q8_0_SOA / Q5_1_SOA (they are not weight formats of the C ABI)
Q4_K, Q5_K, IQ4_XS, Q6_K_SOA, Q8_0_SOA, Q5_1_SOA, Q6_K = 0, 1, 2, 3, 4, 5, 6
Q8_0, Q5_1, Q5_0 = 8, 9, 10
BLOCK = {Q4_K: (256, 144), Q5_K: (256, 176), IQ4_XS: (256, 136), Q6_K: (256, 210), Q6_K_SOA: (256, 210),
         Q8_0: (32, 34), Q5_1: (32, 24), Q5_0: (32, 22), Q8_0_SOA: (32, 34), Q5_1_SOA: (32, 24)}


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def _f16_abs_normal(g, n, sigma=0.01):
    return np.abs(g.normal(0.0, sigma, n)).astype(np.float16).view(np.uint16)


def q4k_blocks(g, nblocks):
    """nblocks Q4_K blocks as uint8 [nblocks, 144]."""
    out = np.empty((nblocks, Q4K_BYTES), dtype=np.uint8)
    out[:, 0:2] = _f16_abs_normal(g, nblocks).view(np.uint8).reshape(nblocks, 2)
    out[:, 2:4] = _f16_abs_normal(g, nblocks).view(np.uint8).reshape(nblocks, 2)
    out[:, 4:] = g.integers(0, 256, (nblocks, Q4K_BYTES - 4), dtype=np.uint8)
    return out


def q6k_blocks(g, nblocks):
    """nblocks GGUF Q6_K blocks as uint8 [nblocks, 210]."""
    out = np.empty((nblocks, Q6K_BYTES), dtype=np.uint8)
    out[:, :208] = g.integers(0, 256, (nblocks, 208), dtype=np.uint8)
    out[:, 208:210] = _f16_abs_normal(g, nblocks).view(np.uint8).reshape(nblocks, 2)
    return out


def blocks(g, fmt, nblocks):
    """nblocks GGUF blocks of fmt (Q4_K, Q5_K, IQ4_XS, Q6_K, Q8_0, Q5_1, Q5_0) as uint8 [nblocks, bytes]."""
    if fmt == Q4_K:
        return q4k_blocks(g, nblocks)
    if fmt == Q6_K:
        return q6k_blocks(g, nblocks)
    nbytes = BLOCK[fmt][1]
    out = g.integers(0, 256, (nblocks, nbytes), dtype=np.uint8)
    if fmt in (Q5_K, Q8_0, Q5_0, IQ4_XS):        # d (and Q5_K's dmin) at bytes 0..1 (2..3)
        out[:, 0:2] = _f16_abs_normal(g, nblocks).view(np.uint8).reshape(nblocks, 2)
        if fmt == Q5_K:
            out[:, 2:4] = _f16_abs_normal(g, nblocks).view(np.uint8).reshape(nblocks, 2)
    elif fmt == Q5_1:                              # d, then the signed offset m
        out[:, 0:2] = _f16_abs_normal(g, nblocks).view(np.uint8).reshape(nblocks, 2)
        out[:, 2:4] = g.normal(0.0, 0.01, nblocks).astype(np.float16).view(np.uint8).reshape(nblocks, 2)
    else:
        raise ValueError(f"format {fmt}")
    return out


def row_bytes(fmt, K):
    per, nbytes = BLOCK[fmt]
    assert K % per == 0
    if fmt == Q8_0_SOA:
        return K + K // 16
    return K // per * nbytes


def matrix(seed, fmt, N, K):
    """A [N][K] weight in format fmt as uint8 [N, row_bytes].  The SoA formats are the repacks of
    the GGUF matrix drawn with the same seed (Q6_K -> Q6_K_SOA, Q8_0 -> Q8_0_SOA, Q5_1 -> Q5_1_SOA)."""
    g = rng(seed)
    src = {Q6_K_SOA: Q6_K, Q8_0_SOA: Q8_0, Q5_1_SOA: Q5_1}.get(fmt, fmt)
    per, nbytes = BLOCK[src]
    nb = K // per
    W = blocks(g, src, N * nb).reshape(N, nb * nbytes)
    if fmt == Q6_K_SOA:
        return repack_q6k_soa(W, K)
    if fmt == Q8_0_SOA:
        return repack_q8_0_soa(W, K)
    if fmt == Q5_1_SOA:
        return repack_q5_1_soa(W, K)
    return W


def repack_q6k_soa(W, K):
    """GGUF Q6_K rows -> [ql K/2][qh K/4][sc K/16][d K/128] per row (engine/kernels/gemv.hip:1341-1350)."""
    N = W.shape[0]
    nb = K // QK
    b = W.reshape(N, nb, Q6K_BYTES)
    return np.concatenate([b[:, :, :128].reshape(N, -1), b[:, :, 128:192].reshape(N, -1),
                           b[:, :, 192:208].reshape(N, -1), b[:, :, 208:210].reshape(N, -1)], axis=1)


def repack_q8_0_soa(W, K):
    """GGUF Q8_0 rows -> [qs K][d (K/32) x f16] per row (engine/kernels/gemv.hip:1351-1354)."""
    N = W.shape[0]
    b = W.reshape(N, K // 32, 34)
    return np.concatenate([b[:, :, 2:].reshape(N, -1), b[:, :, :2].reshape(N, -1)], axis=1)


def repack_q5_1_soa(W, K):
    """GGUF Q5_1 rows -> [qs K/2][qh K/8][d (K/32) x f16][m (K/32) x f16] (gemv.hip:1458-1465)."""
    N = W.shape[0]
    b = W.reshape(N, K // 32, 24)
    return np.concatenate([b[:, :, 8:24].reshape(N, -1), b[:, :, 4:8].reshape(N, -1), b[:, :, 0:2].reshape(N, -1),
                           b[:, :, 2:4].reshape(N, -1)], axis=1)


def experts(seed, fmt, n_exp, N, K):
    """n_exp expert matrices [N][K], contiguous (expert e at e * N * row_bytes)."""
    return matrix(seed, fmt, n_exp * N, K).reshape(n_exp, N, row_bytes(fmt, K))


def normal_f32(seed, shape):
    return rng(seed).standard_normal(shape, dtype=np.float32)


def to_bf16_bits(x):
    """f32 -> bf16 bits, round-to-nearest-even (engine/kernels/gemm.hip:12)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def router_logits(seed, T, n_exp=512, zipf_s=None):
    """[T][n_exp + 1] f32: N(0,1) logits for the experts plus the shared-expert gate logit (the
    reference router has n_exp + 1 rows, fn.hip:170,203).  With zipf_s, expert e gets the bias
    -zipf_s * ln(rank_e), ranks a seeded permutation of 1..n_exp."""
    g = rng(seed)
    logits = g.standard_normal((T, n_exp + 1), dtype=np.float32)
    if zipf_s is not None:
        ranks = g.permutation(n_exp) + 1
        bias = (-zipf_s * np.log(ranks.astype(np.float64))).astype(np.float32)
        logits[:, :n_exp] += bias[None, :]
    return logits


# ---- the BASELINE.json configurations ----
SEEDS = {"cfg0": 1000, "cfg1": 1100, "cfg2": 1200, "cfg3": 1300, "cfg4": 1400}

CFG0 = dict(N=17408, K=5120)                         # Q4_K GEMV M=1
CFG1 = dict(hidden=5120, ffn=17408, qkv=6144 + 1024 + 1024, o_in=6144, M=(1, 4, 8))
CFG2 = dict(hidden=2048, ffn=512, n_exp=512, topk=10, T=(1, 4, 8))
CFG3 = dict(M=2048, N=17408, K=5120, verify_M=(3, 4, 5, 6))
CFG4 = dict(T=2048, hidden=2048, ffn=512, n_exp=512, topk=10, zipf_s=1.1)
