// q4k_pair.hpp -- the Q4_K "pair" decomposition shared by the decode GEMV (gemv.hip) and the MoE
// expert GEMVs (moe.hip): per-lane weight loads, branch-free scale decode, int8 dot products and the
// transposed LDS layout of q8 activations.  Device code only; nothing here allocates.
#pragma once
#include "qmm_common.hpp"

namespace qmm {

constexpr int kPairBlock = 256;   // threads per workgroup of the kernels that stage x with XStage

// Q4_K x int8 GEMV ("pair" mapping).
//
// A Q4_K block is {d, dmin, scales[12]} + qs[128]; qs bytes 32j..32j+31 carry sub-block 2j in
// their low nibbles and sub-block 2j+1 in their high nibbles (engine/src/quant.h:43-53).  One
// lane owns one such 32-byte "pair" (64 weights): it loads the two 16-byte halves plus the
// 16-byte block header, decodes only the two scales and two mins it needs, and finishes both
// sub-block dot products itself.  LPR lanes cover a row (lane t takes pairs t, t+LPR, ... of the
// row, so pair index j = t & 3 is fixed per lane); the decode GEMV uses LPR = 16 (4 rows per
// wave, 16 rows per 256-thread workgroup), the short-K expert GEMVs LPR = 8.  Each wave issues the loads of its whole row group (up to 6 pair iterations) before
// it computes anything; longer rows are streamed in chunks of 4 iterations with the next chunk's
// loads in flight while the current one is computed.  The loads are unconditional (indices past
// the row end are clamped and their results masked), which keeps them straight-line code so the
// compiler waits for one buffer with a partial vmcnt instead of draining all loads.
//
// x (int8 per 32, scale d, d*sum) is staged per workgroup in LDS, transposed at 16-byte
// granularity so that the 16-byte reads of consecutive lanes (consecutive pairs) hit consecutive
// banks: unit q of pair p (x[64p + 16q .. +15]) sits at ((q * K/64) + p) * 16, and the four
// scalars {d(2p), d(2p+1), s(2p), s(2p+1)} of pair p at (K + 16p).
// Per lane the sums accumulate in pair order; the 16 lanes of a row reduce with a fixed butterfly.
// Neither depends on NCOL, so a column's result is bitwise the same whatever ncol the call has.
template <int I>
struct Q4kPairs { uint4 q0[I], q1[I], h[I]; };

template <int I, int LPR = 16>
__device__ __forceinline__ void q4k_load_pairs(const uint8_t* __restrict__ rp, int t, int j, int ntask, int it0,
                                               Q4kPairs<I>& B) {
#pragma unroll
    for (int i = 0; i < I; ++i) {
        const int task = min(t + LPR * (it0 + i), ntask - 1);
        const uint8_t* bp = rp + (size_t)(task >> 2) * 144;
        B.h[i] = ld16(bp);
        B.q0[i] = ld16(bp + 16 + 32 * j);
        B.q1[i] = ld16(bp + 32 + 32 * j);
    }
}

// x operand of one column, either from the transposed LDS copy or from global memory
template <bool XLDS>
struct XPairSrc {
    const uint8_t* q;     // LDS: transposed xq of this column; global: xq row of this column
    const float* d;       // global only
    const float* s;       // global only
    int K;
    __device__ __forceinline__ void get(int task, uint4& u0, uint4& u1, uint4& u2, uint4& u3, float4& ds) const {
        if constexpr (XLDS) {
            const int kq = K >> 6;
            u0 = ld16(q + (size_t)(task) * 16);
            u1 = ld16(q + (size_t)(kq + task) * 16);
            u2 = ld16(q + (size_t)(2 * kq + task) * 16);
            u3 = ld16(q + (size_t)(3 * kq + task) * 16);
            ds = *(const float4*)(q + (size_t)K + (size_t)task * 16);
        } else {
            const uint8_t* p = q + (size_t)task * 64;
            u0 = ld16(p); u1 = ld16(p + 16); u2 = ld16(p + 32); u3 = ld16(p + 48);
            const float2 dd = *(const float2*)(d + 2 * task), ss = *(const float2*)(s + 2 * task);
            ds = make_float4(dd.x, dd.y, ss.x, ss.y);
        }
    }
};

// Lane-constant pieces of the scale/min decode for pair j (engine/src/quant.h:37-40).  The 6-bit
// scales of sub-blocks 2j, 2j+1 are bytes (2j)&3, (2j+1)&3 of
//   j < 2:  s[0..3] & 63                          (mins: s[4..7] & 63)
//   j >= 2: (s[8..11] & 15) | ((s[0..3] >> 6) << 4) (mins: (s[8..11] >> 4) | ((s[4..7] >> 6) << 4))
// written branch-free as ((s0 >> sh0) & m0) | ((s2 >> sh2) & m2).
struct Q4kPairDecode {
    uint32_t sh0, m0, m2, bsh;
    __device__ __forceinline__ explicit Q4kPairDecode(int j) {
        const bool lo = j < 2;
        sh0 = lo ? 0u : 2u;
        m0 = lo ? 0x3f3f3f3fu : 0x30303030u;
        m2 = lo ? 0u : 0x0f0f0f0fu;
        bsh = (uint32_t)(j & 1) * 16u;
    }
};

// The scales of pair j of a block header: dA, dB = d * sc[2j], d * sc[2j+1]; mA, mB = dmin * m[2j],
// dmin * m[2j+1] (quant.h:37-40 decode).
struct Q4kPairScales { float dA, dB, mA, mB; };
__device__ __forceinline__ Q4kPairScales q4k_pair_scales(const uint4 hd, const Q4kPairDecode& dc) {
    const uint32_t scw = (((hd.y >> dc.sh0) & dc.m0) | (hd.w & dc.m2)) >> dc.bsh;
    const uint32_t mw = (((hd.z >> dc.sh0) & dc.m0) | ((hd.w >> 4) & dc.m2)) >> dc.bsh;
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    return {d * (float)(scw & 0xffu), d * (float)((scw >> 8) & 0xffu), dmin * (float)(mw & 0xffu),
            dmin * (float)((mw >> 8) & 0xffu)};
}

// One pair's contribution to one column, ds = {dx[2p], dx[2p+1], sx[2p], sx[2p+1]} of x and ia, ib the
// exact integer dots of sub-blocks 2j, 2j+1.  Evaluated in a fixed order (explicit fma, no contraction
// left to the compiler), so every kernel that adds a row's pair values in the same order -- the dot4
// kernels here, the matrix-core kernel of gemv_mfma.hip -- gets the same bits.
__device__ __forceinline__ float q4k_pair_value(const Q4kPairScales& s, const float4 ds, int ia, int ib) {
#pragma clang fp contract(off)
    const float t = __builtin_fmaf(s.dB, ds.y * (float)ib, s.dA * (ds.x * (float)ia));
    return t - __builtin_fmaf(s.mB, ds.w, s.mA * ds.z);
}

template <int NCOL, int I, bool XLDS, bool EXACT, int LPR = 16>
__device__ __forceinline__ void q4k_pairs_compute(const Q4kPairs<I>& B, const Q4kPairDecode& dc, int t, int ntask, int it0,
                                                  const XPairSrc<XLDS>* xs, float* acc) {
#pragma unroll
    for (int i = 0; i < I; ++i) {
        const int task = t + LPR * (it0 + i);
        const uint4 hd = B.h[i], w0 = B.q0[i], w1 = B.q1[i];
        const Q4kPairScales sc = q4k_pair_scales(hd, dc);
        const uint32_t a0 = w0.x & 0x0f0f0f0fu, a1 = w0.y & 0x0f0f0f0fu, a2 = w0.z & 0x0f0f0f0fu, a3 = w0.w & 0x0f0f0f0fu;
        const uint32_t a4 = w1.x & 0x0f0f0f0fu, a5 = w1.y & 0x0f0f0f0fu, a6 = w1.z & 0x0f0f0f0fu, a7 = w1.w & 0x0f0f0f0fu;
        const uint32_t b0 = (w0.x >> 4) & 0x0f0f0f0fu, b1 = (w0.y >> 4) & 0x0f0f0f0fu, b2 = (w0.z >> 4) & 0x0f0f0f0fu, b3 = (w0.w >> 4) & 0x0f0f0f0fu;
        const uint32_t b4 = (w1.x >> 4) & 0x0f0f0f0fu, b5 = (w1.y >> 4) & 0x0f0f0f0fu, b6 = (w1.z >> 4) & 0x0f0f0f0fu, b7 = (w1.w >> 4) & 0x0f0f0f0fu;
        const int tk = EXACT ? task : min(task, ntask - 1);
#pragma unroll
        for (int c = 0; c < NCOL; ++c) {
            uint4 u0, u1, u2, u3; float4 ds;
            xs[c].get(tk, u0, u1, u2, u3, ds);
            int ia = sdot4(a0, u0.x, 0); ia = sdot4(a1, u0.y, ia); ia = sdot4(a2, u0.z, ia); ia = sdot4(a3, u0.w, ia);
            ia = sdot4(a4, u1.x, ia); ia = sdot4(a5, u1.y, ia); ia = sdot4(a6, u1.z, ia); ia = sdot4(a7, u1.w, ia);
            int ib = sdot4(b0, u2.x, 0); ib = sdot4(b1, u2.y, ib); ib = sdot4(b2, u2.z, ib); ib = sdot4(b3, u2.w, ib);
            ib = sdot4(b4, u3.x, ib); ib = sdot4(b5, u3.y, ib); ib = sdot4(b6, u3.z, ib); ib = sdot4(b7, u3.w, ib);
            const float v = q4k_pair_value(sc, ds, ia, ib);
            acc[c] += (EXACT || task < ntask) ? v : 0.f;
        }
    }
}

// Stage NCOL columns of q8 x into LDS in the transposed pair layout described above; column c
// occupies [c * 5K/4, (c+1) * 5K/4).  The staging is split in two so that a caller can issue the
// x loads (L2 hits) before its weight loads: vmcnt retires loads in issue order, so x can then be
// waited for without waiting for the weights.  Unit v < NCOL*K/16 is 16 bytes of xq; unit
// NCOL*K/16 + w is the {d, d, s, s} quadruple of pair w.  Each thread takes units
// threadIdx.x + 256*u, u < U (U * 256 >= NCOL * 5K/64).
template <int NCOL, int U>
struct XStage { uint4 v[U]; };

template <int NCOL, int U>
__device__ __forceinline__ void stage_pairs_load(const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                 const float* __restrict__ xs, int K, XStage<NCOL, U>& S) {
    const int nq = NCOL * (K >> 4), nt = nq + NCOL * (K >> 6), kq = K >> 6, nsb = K >> 5;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int v = min((int)threadIdx.x + kPairBlock * u, nt - 1);
        if (v < nq) {
            S.v[u] = ld16(xq + (size_t)v * 16);
        } else {
            const int w = v - nq, c = w / kq, p = w - c * kq;
            const float2 dd = *(const float2*)(xd + (size_t)c * nsb + 2 * p), ss = *(const float2*)(xs + (size_t)c * nsb + 2 * p);
            S.v[u] = make_uint4(__float_as_uint(dd.x), __float_as_uint(dd.y), __float_as_uint(ss.x), __float_as_uint(ss.y));
        }
    }
}

template <int NCOL, int U>
__device__ __forceinline__ void stage_pairs_store(uint8_t* lds, int K, const XStage<NCOL, U>& S) {
    const int nu = K >> 4, nq = NCOL * nu, nt = nq + NCOL * (K >> 6), kq = K >> 6;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int v = (int)threadIdx.x + kPairBlock * u;
        if (v >= nt) continue;
        size_t off;
        if (v < nq) {
            const int c = v / nu, un = v - c * nu;
            off = (size_t)c * (K + (K >> 2)) + (size_t)((un & 3) * kq + (un >> 2)) * 16;
        } else {
            const int w = v - nq, c = w / kq, p = w - c * kq;
            off = (size_t)c * (K + (K >> 2)) + (size_t)K + (size_t)p * 16;
        }
        *(uint4*)(lds + off) = S.v[u];
    }
}

// The same layout filled from f32 x: a quad of lanes holds the 32 values of one q8 block (lane k of
// the quad: values 8k..8k+7, two float4) and quantises them with the arithmetic of the q8 quantiser
// (gemv.hip:36-51 semantics: d = amax/127, q = rne(x * 127/amax), s = d * sum(q)), so q, d and s
// are bit-identical to staging its output; the quad reductions are DPP lane permutations.  Thread
// slot e = threadIdx.x + BS*u (BS = threads of the workgroup) covers floats 8e..8e+7 of the
// column-major [NCOL][K] array; U * BS >= NCOL * K/8.
template <int NCOL, int U>
struct XStageF { float4 v[U][2]; };

template <int NCOL, int U, int BS = kPairBlock>
__device__ __forceinline__ void stagef_load(const float* __restrict__ x, int K, XStageF<NCOL, U>& S) {
    const int n8 = NCOL * (K >> 3);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const float4* p = (const float4*)x + 2 * min((int)threadIdx.x + BS * u, n8 - 1);
        S.v[u][0] = p[0];
        S.v[u][1] = p[1];
    }
}

// value of the lane `xor m` within the quad (m = 1 or 2), by DPP quad permutation
template <int M>
__device__ __forceinline__ int quad_xor(int v) {
    return __builtin_amdgcn_mov_dpp(v, M == 1 ? 0xB1 : 0x4E, 0xf, 0xf, false);
}

// One slot of the staging below: the 8 values {a, b} are floats 8e..8e+7 of the column-major [ncol][K]
// array; the 4 lanes of a quad hold one 32-value q8 block.  All 4 lanes of a quad must be active (the
// quad reductions are DPP permutations); e >= n8 computes and stores nothing.
__device__ __forceinline__ void stagef_store_one(uint8_t* lds, int K, float4 a, float4 b, int e, int n8) {
    const int k8 = K >> 3, kq = K >> 6;
    float amax = fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                       fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
    amax = fmaxf(amax, __int_as_float(quad_xor<1>(__float_as_int(amax))));
    amax = fmaxf(amax, __int_as_float(quad_xor<2>(__float_as_int(amax))));
    const float dd = amax / 127.f, id = amax > 0.f ? 127.f / amax : 0.f;
    const int q0 = __float2int_rn(a.x * id), q1 = __float2int_rn(a.y * id), q2 = __float2int_rn(a.z * id);
    const int q3 = __float2int_rn(a.w * id), q4 = __float2int_rn(b.x * id), q5 = __float2int_rn(b.y * id);
    const int q6 = __float2int_rn(b.z * id), q7 = __float2int_rn(b.w * id);
    int sum = ((q0 + q1) + (q2 + q3)) + ((q4 + q5) + (q6 + q7));
    sum += quad_xor<1>(sum);
    sum += quad_xor<2>(sum);
    if (e < n8) {
        const int c = e / k8, f = e - c * k8, un = f >> 1;   // 16-byte unit un, half f & 1
        uint8_t* base = lds + (size_t)c * (K + (K >> 2));
        const uint32_t lo = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)q3 << 24);
        const uint32_t hi = (uint32_t)(q4 & 0xff) | ((uint32_t)(q5 & 0xff) << 8) | ((uint32_t)(q6 & 0xff) << 16) | ((uint32_t)q7 << 24);
        *(uint2*)(base + (size_t)((un & 3) * kq + (un >> 2)) * 16 + (f & 1) * 8) = make_uint2(lo, hi);
        if ((f & 3) == 0) {
            const int sb = f >> 2;
            float* dsq = (float*)(base + (size_t)K + (size_t)(sb >> 1) * 16);
            dsq[sb & 1] = dd;
            dsq[2 + (sb & 1)] = dd * (float)sum;
        }
    }
}

template <int NCOL, int U, int BS = kPairBlock>
__device__ __forceinline__ void stagef_store(uint8_t* lds, int K, const XStageF<NCOL, U>& S) {
    const int n8 = NCOL * (K >> 3);
#pragma unroll
    for (int u = 0; u < U; ++u)                               // n8 is a multiple of 4: quads share e < n8
        stagef_store_one(lds, K, S.v[u][0], S.v[u][1], (int)threadIdx.x + BS * u, n8);
}

// Same layout, loop form for any K (used when the whole x does not fit the register batch).
template <int NCOL>
__device__ __forceinline__ void stage_xq8_pairs(uint8_t* lds, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                const float* __restrict__ xs, int K) {
    const int nu = K >> 4, kq = K >> 6, nsb = K >> 5;
    for (int v = threadIdx.x; v < NCOL * nu; v += blockDim.x) {
        const int c = v / nu, u = v - c * nu;          // unit u = x[16u .. 16u+15] of column c
        const int p = u >> 2, q = u & 3;
        *(uint4*)(lds + (size_t)c * (K + (K >> 2)) + (size_t)(q * kq + p) * 16) = ld16(xq + (size_t)c * K + (size_t)u * 16);
    }
    for (int v = threadIdx.x; v < NCOL * kq; v += blockDim.x) {
        const int c = v / kq, p = v - c * kq;
        const float2 dd = *(const float2*)(xd + (size_t)c * nsb + 2 * p), ss = *(const float2*)(xs + (size_t)c * nsb + 2 * p);
        *(float4*)(lds + (size_t)c * (K + (K >> 2)) + (size_t)K + (size_t)p * 16) = make_float4(dd.x, dd.y, ss.x, ss.y);
    }
    __syncthreads();
}

}  // namespace qmm
