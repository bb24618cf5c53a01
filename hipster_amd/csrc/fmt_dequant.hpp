// fmt_dequant.hpp -- exact f32 dequantisation of one 32-weight sub-block of a weight row, for every
// format of the call surface (engine/src/quant.h:37-100 and the SoA repacks of
// engine/kernels/gemv.hip:1341-1354,1448-1465; Q6_K in its row-SoA repack, the engine's only form).  Every product here is exact in f32 (at most 24
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
        case QMM_Q6_K_SOA: return (size_t)(K >> 8) * 210;
        default: return (size_t)(K >> 5) * 24;          // QMM_Q5_1_SOA
    }
}

// The raw bytes of one sub-block (at most 80: a Q5_K block header, its qh and a qs pair), loaded
// apart from their decode so that a pipeline can issue the loads a step ahead.
struct SubRaw { uint4 v[5]; };

template <int F>
__device__ __forceinline__ void sub_load(const uint8_t* __restrict__ rp, int K, int sb, SubRaw& r) {
    if constexpr (F == QMM_Q4_K) {
        const uint8_t* blk = rp + (size_t)(sb >> 3) * 144;
        const int j = (sb & 7) >> 1;
        r.v[0] = ld16(blk);
        r.v[1] = ld16(blk + 16 + 32 * j);
        r.v[2] = ld16(blk + 32 + 32 * j);
    } else if constexpr (F == QMM_Q5_K) {
        const uint8_t* blk = rp + (size_t)(sb >> 3) * 176;
        const int j = (sb & 7) >> 1;
        r.v[0] = ld16(blk);
        r.v[1] = ld16(blk + 16);
        r.v[2] = ld16(blk + 32);
        r.v[3] = ld16(blk + 48 + 32 * j);
        r.v[4] = ld16(blk + 64 + 32 * j);
    } else if constexpr (F == QMM_IQ4_XS) {
        const uint8_t* blk = rp + (size_t)(sb >> 3) * 136;
        const uint2 hd = *(const uint2*)blk;
        r.v[0] = make_uint4(hd.x, hd.y, 0u, 0u);
        r.v[1] = ld16_a4(blk + 8 + 16 * (sb & 7));
    } else if constexpr (F == QMM_Q6_K_SOA) {          // streams [ql][qh][scales][d], rows dword aligned (K % 512)
        const int nb = K >> 8, b = sb >> 3, s = sb & 7, n = s >> 2, g = s & 3;
        const uint8_t* ql = rp + (size_t)b * 128 + 64 * n + 32 * (g & 1);
        const uint8_t* qh = rp + (size_t)nb * 128 + (size_t)b * 64 + 32 * n;
        r.v[0] = ld16_a4(ql);
        r.v[1] = ld16_a4(ql + 16);
        r.v[2] = ld16_a4(qh);
        r.v[3] = ld16_a4(qh + 16);
        r.v[4].x = *(const uint16_t*)(rp + (size_t)nb * 192 + (size_t)b * 16 + 8 * n + 2 * g);   // the two scales
        r.v[4].y = *(const uint16_t*)(rp + (size_t)nb * 208 + 2 * (size_t)b);                  // d
    } else if constexpr (F == QMM_Q8_0_SOA) {          // rows dword aligned (K % 64)
        r.v[0] = ld16_a4(rp + 32 * (size_t)sb);
        r.v[1] = ld16_a4(rp + 32 * (size_t)sb + 16);
        r.v[2].x = *(const uint16_t*)(rp + K + 2 * sb);
    } else {                                            // QMM_Q5_1_SOA, rows 8-byte aligned
        r.v[0] = ld16_a4(rp + 16 * (size_t)sb);
        r.v[1].x = *(const uint32_t*)(rp + (K >> 1) + 4 * sb);
        r.v[1].y = *(const uint16_t*)(rp + (K >> 1) + (K >> 3) + 2 * sb);
        r.v[1].z = *(const uint16_t*)(rp + (K >> 1) + (K >> 3) + (K >> 4) + 2 * sb);
    }
}

template <int F>
__device__ __forceinline__ void sub_decode(const SubRaw& r, int sb, float (&w)[32]) {
    if constexpr (F == QMM_Q4_K) {                      // y = (d sc) q - (dmin m), quant.h:44-53
        const int s = sb & 7;
        const uint4 hd = r.v[0], q0 = r.v[1], q1 = r.v[2];
        const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
        const Q4kScaleBytes sc = q4k_scale_bytes(hd.y, hd.z, hd.w);
        const float dl = d * (float)byte8(sc.sc_lo, sc.sc_hi, s), ml = dmin * (float)byte8(sc.m_lo, sc.m_hi, s);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const uint32_t qb = (q[l >> 2] >> (8 * (l & 3))) & 0xffu;
            w[l] = dl * (float)((s & 1) ? qb >> 4 : qb & 15u) - ml;
        }
    } else if constexpr (F == QMM_Q5_K) {               // quant.h:54-64
        const int s = sb & 7;
        const uint4 hd = r.v[0], h0 = r.v[1], h1 = r.v[2], q0 = r.v[3], q1 = r.v[4];
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
    } else if constexpr (F == QMM_IQ4_XS) {             // quant.h:92-100
        const int ib = sb & 7;
        const uint32_t hx = r.v[0].x, hy = r.v[0].y;
        const int ls = (int)((hy >> (4 * ib)) & 0xfu) | (int)(((hx >> (16 + 2 * ib)) & 3u) << 4);
        const float dl = h2f(hx) * (float)(ls - 32);
        const uint32_t q[4] = {r.v[1].x, r.v[1].y, r.v[1].z, r.v[1].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {           // weights 4k..4k+3 (low nibbles) and 16+4k.. (high)
            const uint32_t lo = iq4_levels4(q[k] & 0x0f0f0f0fu), hi = iq4_levels4((q[k] >> 4) & 0x0f0f0f0fu);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                w[4 * k + b] = dl * (float)(int8_t)(lo >> (8 * b));
                w[16 + 4 * k + b] = dl * (float)(int8_t)(hi >> (8 * b));
            }
        }
    } else if constexpr (F == QMM_Q6_K_SOA) {          // quant.h:65-75: weight 32g + l of half n
        // (sub-block 4n + g) = d sc[8n + 2g + l/16] ((ql nibble) | (qh bits 2g, 2g+1) << 4) - 32)
        const int g = sb & 3;
        const float d = h2f(r.v[4].y);
        const float ds0 = d * (float)(int8_t)(r.v[4].x & 0xffu), ds1 = d * (float)(int8_t)((r.v[4].x >> 8) & 0xffu);
        const uint32_t ql[8] = {r.v[0].x, r.v[0].y, r.v[0].z, r.v[0].w, r.v[1].x, r.v[1].y, r.v[1].z, r.v[1].w};
        const uint32_t qh[8] = {r.v[2].x, r.v[2].y, r.v[2].z, r.v[2].w, r.v[3].x, r.v[3].y, r.v[3].z, r.v[3].w};
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const uint32_t lo = (ql[l >> 2] >> (8 * (l & 3))) & 0xffu, hi = (qh[l >> 2] >> (8 * (l & 3))) & 0xffu;
            const int q = (int)((g < 2 ? (lo & 15u) : (lo >> 4)) | (((hi >> (2 * g)) & 3u) << 4)) - 32;
            w[l] = (l < 16 ? ds0 : ds1) * (float)q;
        }
    } else if constexpr (F == QMM_Q8_0_SOA) {          // quant.h:76-80 (SoA: gemv.hip:1351-1354)
        const float d = h2f(r.v[2].x);
        const uint32_t q[8] = {r.v[0].x, r.v[0].y, r.v[0].z, r.v[0].w, r.v[1].x, r.v[1].y, r.v[1].z, r.v[1].w};
#pragma unroll
        for (int l = 0; l < 32; ++l) w[l] = (float)(int8_t)((q[l >> 2] >> (8 * (l & 3))) & 0xffu) * d;
    } else {                                            // QMM_Q5_1_SOA, quant.h:82-88 (SoA: gemv.hip:1458-1465)
        const uint32_t qh = r.v[1].x;
        const float d = h2f(r.v[1].y), m = h2f(r.v[1].z);
        const uint32_t q[4] = {r.v[0].x, r.v[0].y, r.v[0].z, r.v[0].w};
#pragma unroll
        for (int l = 0; l < 16; ++l) {
            const uint32_t qb = (q[l >> 2] >> (8 * (l & 3))) & 0xffu;
            w[l] = (float)((qb & 15u) | (((qh >> l) & 1u) << 4)) * d + m;
            w[l + 16] = (float)((qb >> 4) | (((qh >> (l + 16)) & 1u) << 4)) * d + m;
        }
    }
}

template <int F>
__device__ __forceinline__ void dq_sub32(const uint8_t* __restrict__ rp, int K, int sb, float (&w)[32]) {
    SubRaw r;
    sub_load<F>(rp, K, sb, r);
    sub_decode<F>(r, sb, w);
}

// load and decode with the format chosen at run time (a uniform branch)
__device__ __forceinline__ void sub_load_rt(int fmt, const uint8_t* __restrict__ rp, int K, int sb, SubRaw& r) {
    switch (fmt) {
        case QMM_Q4_K: sub_load<QMM_Q4_K>(rp, K, sb, r); break;
        case QMM_Q5_K: sub_load<QMM_Q5_K>(rp, K, sb, r); break;
        case QMM_IQ4_XS: sub_load<QMM_IQ4_XS>(rp, K, sb, r); break;
        case QMM_Q8_0_SOA: sub_load<QMM_Q8_0_SOA>(rp, K, sb, r); break;
        default: sub_load<QMM_Q5_1_SOA>(rp, K, sb, r); break;
    }
}
__device__ __forceinline__ void sub_decode_rt(int fmt, const SubRaw& r, int sb, float (&w)[32]) {
    switch (fmt) {
        case QMM_Q4_K: sub_decode<QMM_Q4_K>(r, sb, w); break;
        case QMM_Q5_K: sub_decode<QMM_Q5_K>(r, sb, w); break;
        case QMM_IQ4_XS: sub_decode<QMM_IQ4_XS>(r, sb, w); break;
        case QMM_Q8_0_SOA: sub_decode<QMM_Q8_0_SOA>(r, sb, w); break;
        default: sub_decode<QMM_Q5_1_SOA>(r, sb, w); break;
    }
}

// the same in one call
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
