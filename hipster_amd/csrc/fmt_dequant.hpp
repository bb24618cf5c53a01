// fmt_dequant.hpp -- exact f32 dequantisation of one 32-weight sub-block of a weight row, for every
// format of the call surface except Q6_K (engine/src/quant.h:37-100 and the SoA repacks of
// engine/kernels/gemv.hip:1341-1354,1448-1465).  Every product here is exact in f32 (at most 24
// significant bits: an f16 scale times a 6-bit scale, an 8-bit level or a <= 8-bit quant), so a
// contracted d*q - m rounds exactly like the reference's separately rounded operations.
#pragma once
#include "qmm_common.hpp"

namespace qmm {

// bytes of one weight row of K weights
__host__ __device__ __forceinline__ size_t fmt_row_bytes_rt(int fmt, int K) {
    switch (fmt) {
        case QMM_Q4_K: return (size_t)(K >> 8) * 144;
        case QMM_Q5_K: return (size_t)(K >> 8) * 176;
        case QMM_IQ4_XS: return (size_t)(K >> 8) * 136;
        case QMM_Q8_0_SOA: return (size_t)K + (size_t)(K >> 4);
        default: return (size_t)(K >> 5) * 24;          // QMM_Q5_1_SOA
    }
}

template <int F>
__device__ __forceinline__ void dq_sub32(const uint8_t* __restrict__ rp, int K, int sb, float (&w)[32]) {
    if constexpr (F == QMM_Q4_K) {                      // y = (d sc) q - (dmin m), quant.h:44-53
        const uint8_t* blk = rp + (size_t)(sb >> 3) * 144;
        const int s = sb & 7, j = s >> 1;
        const uint4 hd = ld16(blk);
        const uint4 q0 = ld16(blk + 16 + 32 * j), q1 = ld16(blk + 32 + 32 * j);
        const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
        const Q4kScaleBytes sc = q4k_scale_bytes(hd.y, hd.z, hd.w);
        const float dl = d * (float)byte8(sc.sc_lo, sc.sc_hi, s), ml = dmin * (float)byte8(sc.m_lo, sc.m_hi, s);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const uint32_t qb = (q[l >> 2] >> (8 * (l & 3))) & 0xffu;
            w[l] = dl * (float)((s & 1) ? qb >> 4 : qb & 15u) - ml;
        }
    } else if constexpr (F == QMM_Q5_K) {
        const uint8_t* blk = rp + (size_t)(sb >> 3) * 176;
        const int s = sb & 7, j = s >> 1;
        const uint4 hd = ld16(blk), h0 = ld16(blk + 16), h1 = ld16(blk + 32);
        const uint4 q0 = ld16(blk + 48 + 32 * j), q1 = ld16(blk + 64 + 32 * j);
        const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
        const Q4kScaleBytes sc = q4k_scale_bytes(hd.y, hd.z, hd.w);
        const float dl = d * (float)byte8(sc.sc_lo, sc.sc_hi, s), ml = dmin * (float)byte8(sc.m_lo, sc.m_hi, s);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t hb[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const uint32_t qb = (q[l >> 2] >> (8 * (l & 3))) & 0xffu, hbit = (hb[l >> 2] >> (8 * (l & 3) + s)) & 1u;
            w[l] = dl * (float)(((s & 1) ? qb >> 4 : qb & 15u) + 16u * hbit) - ml;
        }
    } else if constexpr (F == QMM_IQ4_XS) {
        const uint8_t* blk = rp + (size_t)(sb >> 3) * 136;
        const int ib = sb & 7;
        const uint2 hd = *(const uint2*)blk;
        const uint4 qs = ld16_a4(blk + 8 + 16 * ib);
        const int ls = (int)((hd.y >> (4 * ib)) & 0xfu) | (int)(((hd.x >> (16 + 2 * ib)) & 3u) << 4);
        const float dl = h2f(hd.x) * (float)(ls - 32);
        const int8_t lv[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
        for (int l = 0; l < 16; ++l) {
            const uint32_t qb = (q[l >> 2] >> (8 * (l & 3))) & 0xffu;
            w[l] = dl * (float)lv[qb & 15u];
            w[l + 16] = dl * (float)lv[qb >> 4];
        }
    } else if constexpr (F == QMM_Q8_0_SOA) {          // rows dword aligned (K % 64)
        const uint4 a = ld16_a4(rp + 32 * (size_t)sb), b = ld16_a4(rp + 32 * (size_t)sb + 16);
        const float d = h2f(*(const uint16_t*)(rp + K + 2 * sb));
        const uint32_t q[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int l = 0; l < 32; ++l) w[l] = (float)(int8_t)((q[l >> 2] >> (8 * (l & 3))) & 0xffu) * d;
    } else {                                            // QMM_Q5_1_SOA, rows 8-byte aligned
        const uint4 qs = ld16_a4(rp + 16 * (size_t)sb);
        const uint32_t qh = *(const uint32_t*)(rp + (K >> 1) + 4 * sb);
        const float d = h2f(*(const uint16_t*)(rp + (K >> 1) + (K >> 3) + 2 * sb));
        const float m = h2f(*(const uint16_t*)(rp + (K >> 1) + (K >> 3) + (K >> 4) + 2 * sb));
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
        for (int l = 0; l < 16; ++l) {
            const uint32_t qb = (q[l >> 2] >> (8 * (l & 3))) & 0xffu;
            w[l] = (float)((qb & 15u) | (((qh >> l) & 1u) << 4)) * d + m;
            w[l + 16] = (float)((qb >> 4) | (((qh >> (l + 16)) & 1u) << 4)) * d + m;
        }
    }
}

// the same with the format chosen at run time (a uniform branch)
__device__ __forceinline__ void dq_sub32_rt(int fmt, const uint8_t* __restrict__ rp, int K, int sb, float (&w)[32]) {
    switch (fmt) {
        case QMM_Q4_K: dq_sub32<QMM_Q4_K>(rp, K, sb, w); break;
        case QMM_Q5_K: dq_sub32<QMM_Q5_K>(rp, K, sb, w); break;
        case QMM_IQ4_XS: dq_sub32<QMM_IQ4_XS>(rp, K, sb, w); break;
        case QMM_Q8_0_SOA: dq_sub32<QMM_Q8_0_SOA>(rp, K, sb, w); break;
        default: dq_sub32<QMM_Q5_1_SOA>(rp, K, sb, w); break;
    }
}

}  // namespace qmm
