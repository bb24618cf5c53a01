/*
 * qmm_oracle.c -- CPU restatement of the reference's quantized-matmul path.
 * TEST INFRASTRUCTURE ONLY (see qmm_oracle.h): never linked into the product.
 *
 * Build: gcc -O3 -ffp-contract=off (oracle/Makefile).  Contraction must stay off: the
 * reference's dequantisers round d*sc and d*sc*q - dmin*m as separate operations
 * (quant.h:47-50), and the fixtures compare those floats bit for bit.
 */
#include "qmm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------ */
/* small parallel-for over [0, n) with static chunks                                           */
typedef void (*qo_body_fn)(void* ctx, int lo, int hi);
typedef struct { qo_body_fn fn; void* ctx; int lo, hi; } qo_job;
static void* qo_job_run(void* p) { qo_job* j = (qo_job*)p; j->fn(j->ctx, j->lo, j->hi); return NULL; }
static void qo_parallel(int n, int nthreads, qo_body_fn fn, void* ctx) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > n) nthreads = n > 0 ? n : 1;
    if (nthreads == 1) { fn(ctx, 0, n); return; }
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
    qo_job* jobs = (qo_job*)malloc(sizeof(qo_job) * (size_t)nthreads);
    for (int i = 0; i < nthreads; ++i) {
        jobs[i].fn = fn; jobs[i].ctx = ctx;
        jobs[i].lo = (int)((long long)n * i / nthreads); jobs[i].hi = (int)((long long)n * (i + 1) / nthreads);
        pthread_create(&th[i], NULL, qo_job_run, &jobs[i]);
    }
    for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
    free(th); free(jobs);
}

/* ------------------------------------------------------------------------------------------ */
/* number formats                                                                              */

/* quant.h:11-17: IEEE half -> float, exact.  Subnormal halves are renormalised by shifting the
 * mantissa up until the implicit bit appears. */
float qo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (exp == 0) {
        if (man == 0) bits = sign;
        else {
            int e = 1;
            while (!(man & 0x400u)) { man <<= 1; --e; }
            bits = sign | ((uint32_t)(e + 112) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 31) bits = sign | 0x7f800000u | (man << 13);
    else bits = sign | ((exp + 112) << 23) | (man << 13);
    float f; memcpy(&f, &bits, 4); return f;
}
/* float -> IEEE half, round to nearest even (the conversion `(_Float16)x` of gemv.hip:1453);
 * overflow gives infinity, tiny values become subnormal halves.  NaN is not needed here. */
uint16_t qo_f32_to_f16(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const float a = fabsf(f);
    if (!(a < 65520.f)) return (uint16_t)(sign | 0x7c00u);               /* rounds to infinity */
    if (a < 6.103515625e-05f) {                                          /* subnormal half: steps of 2^-24 */
        const float q = nearbyintf(a * 16777216.f);                     /* exact scaling, RNE */
        return (uint16_t)(sign | (uint32_t)q);
    }
    uint32_t v; memcpy(&v, &a, 4);
    const uint32_t mant = v & 0x7fffffu, exp = (v >> 23) - 112u;         /* rebias 127 -> 15 */
    uint32_t h = (exp << 10) | (mant >> 13);
    const uint32_t rest = mant & 0x1fffu;                                /* 13 dropped bits */
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;            /* RNE; a carry bumps the exponent */
    return (uint16_t)(sign | h);
}
/* gemm.hip:12: bf16 = round-to-nearest-even of the top 16 bits (no NaN special case) */
uint16_t qo_f32_to_bf16(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float qo_bf16_to_f32(uint16_t b) { uint32_t u = (uint32_t)b << 16; float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------------------------ */
/* weight blocks                                                                               */

/* quant.h:37-40: 6-bit scale and min of sub-block j from the 12 packed bytes.  j<4: low 6 bits of
 * bytes j and j+4; j>=4: low/high nibble of byte j+4 plus the top two bits of bytes j-4 / j. */
void qo_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) { *sc = q[j] & 63; *m = q[j + 4] & 63; }
    else {
        *sc = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* quant.h:22,43-53.  Block = {f16 d, f16 dmin, u8 scales[12], u8 qs[128]}.  Weights 64j..64j+31
 * are the low nibbles of qs[32j..32j+31] (sub-block 2j), 64j+32..64j+63 the high nibbles
 * (sub-block 2j+1).  w = (d*sc)*q - (dmin*m), every product rounded on its own. */
void qo_dequant_q4_K_block(const uint8_t* blk, float* y) {
    uint16_t hd, hm; memcpy(&hd, blk, 2); memcpy(&hm, blk + 2, 2);
    const float d = qo_f16_to_f32(hd), dmin = qo_f16_to_f32(hm);
    const uint8_t* scales = blk + 4; const uint8_t* qs = blk + 16;
    for (int j = 0; j < 4; ++j) {
        uint8_t sc, m;
        qo_scale_min_k4(2 * j, scales, &sc, &m);
        const float dl = d * (float)sc, ml = dmin * (float)m;
        qo_scale_min_k4(2 * j + 1, scales, &sc, &m);
        const float dh = d * (float)sc, mh = dmin * (float)m;
        for (int l = 0; l < 32; ++l) y[64 * j + l] = dl * (float)(qs[32 * j + l] & 0x0f) - ml;
        for (int l = 0; l < 32; ++l) y[64 * j + 32 + l] = dh * (float)(qs[32 * j + l] >> 4) - mh;
    }
}

/* quant.h:24,65-80.  Block = {u8 ql[128], u8 qh[64], i8 scales[16], f16 d}.  For half n (128
 * weights) and l in 0..31: the four 6-bit values at l, l+32, l+64, l+96 take low/high nibbles of
 * ql[64n+l], ql[64n+l+32] and bit pairs 0-1, 2-3, 4-5, 6-7 of qh[32n+l]; minus 32.
 * w = (d*scale)*q with the scale of 16-element group l/16 (+2 per 32-column). */
void qo_dequant_q6_K_block(const uint8_t* blk, float* y) {
    const uint8_t* ql = blk; const uint8_t* qh = blk + 128; const int8_t* sc = (const int8_t*)(blk + 192);
    uint16_t hd; memcpy(&hd, blk + 208, 2);
    const float d = qo_f16_to_f32(hd);
    for (int n = 0; n < 2; ++n) {
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = (int)((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = (int)((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l + 0] = d * (float)sc[is + 0] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        y += 128; ql += 64; qh += 32; sc += 8;
    }
}

/* gemv.hip:1341-1350: one GGUF Q6_K row -> row-SoA [ql K/2][qh K/4][scales K/16][d (K/256)*2] */
void qo_repack_row_q6_K(const uint8_t* src, uint8_t* dst, int K) {
    const int nb = K / 256;
    for (int b = 0; b < nb; ++b) {
        const uint8_t* blk = src + (size_t)b * 210;
        memcpy(dst + (size_t)b * 128, blk, 128);
        memcpy(dst + (size_t)nb * 128 + (size_t)b * 64, blk + 128, 64);
        memcpy(dst + (size_t)nb * 192 + (size_t)b * 16, blk + 192, 16);
        memcpy(dst + (size_t)nb * 208 + (size_t)b * 2, blk + 208, 2);
    }
}

/* quant.h:23,54-64.  Block = {f16 d, f16 dmin, u8 scales[12], u8 qh[32], u8 qs[128]}.  Like Q4_K,
 * with a fifth bit per weight: weight 64j+l (l < 32) adds 16 when bit 2j of qh[l] is set, weight
 * 64j+32+l when bit 2j+1 is.  w = (d*sc)*q - (dmin*m). */
void qo_dequant_q5_K_block(const uint8_t* blk, float* y) {
    uint16_t hd, hm; memcpy(&hd, blk, 2); memcpy(&hm, blk + 2, 2);
    const float d = qo_f16_to_f32(hd), dmin = qo_f16_to_f32(hm);
    const uint8_t* scales = blk + 4; const uint8_t* qh = blk + 16; const uint8_t* qs = blk + 48;
    for (int j = 0; j < 4; ++j) {
        uint8_t sc, m;
        qo_scale_min_k4(2 * j, scales, &sc, &m);
        const float dl = d * (float)sc, ml = dmin * (float)m;
        qo_scale_min_k4(2 * j + 1, scales, &sc, &m);
        const float dh = d * (float)sc, mh = dmin * (float)m;
        for (int l = 0; l < 32; ++l) {
            const int lo = (qs[32 * j + l] & 0x0f) + (((qh[l] >> (2 * j)) & 1) ? 16 : 0);
            const int hi = (qs[32 * j + l] >> 4) + (((qh[l] >> (2 * j + 1)) & 1) ? 16 : 0);
            y[64 * j + l] = dl * (float)lo - ml;
            y[64 * j + 32 + l] = dh * (float)hi - mh;
        }
    }
}

/* The 16 non-linear 4-bit levels of IQ4_NL / IQ4_XS (quant.h:35; GGUF's kvalues_iq4nl). */
const int8_t qo_iq4nl_levels[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* quant.h:30,93-100.  Block = {f16 d, u16 scales_h, u8 scales_l[4], u8 qs[128]}.  Sub-block ib (32
 * weights) has the 6-bit scale ls = nibble ib of scales_l | bits 2ib..2ib+1 of scales_h << 4 and
 * dl = d*(ls - 32); its weights j and j+16 are the low and high nibbles of qs[16ib + j], mapped
 * through the level table.  w = dl * level. */
void qo_dequant_iq4_xs_block(const uint8_t* blk, float* y) {
    uint16_t hd, sh; memcpy(&hd, blk, 2); memcpy(&sh, blk + 2, 2);
    const float d = qo_f16_to_f32(hd);
    const uint8_t* sl = blk + 4; const uint8_t* qs = blk + 8;
    for (int ib = 0; ib < 8; ++ib) {
        const int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 0x0f) | (((sh >> (2 * ib)) & 3) << 4);
        const float dl = d * (float)(ls - 32);
        for (int j = 0; j < 16; ++j) {
            y[32 * ib + j] = dl * (float)qo_iq4nl_levels[qs[16 * ib + j] & 0x0f];
            y[32 * ib + j + 16] = dl * (float)qo_iq4nl_levels[qs[16 * ib + j] >> 4];
        }
    }
}

/* quant.h:26,81.  Block = {f16 d, i8 qs[32]}: w = q*d. */
void qo_dequant_q8_0_block(const uint8_t* blk, float* y) {
    uint16_t hd; memcpy(&hd, blk, 2);
    const float d = qo_f16_to_f32(hd);
    for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)blk[2 + j] * d;
}

/* quant.h:27,82-88.  Block = {f16 d, f16 m, u8 qh[4], u8 qs[16]}: weight j (j < 16) is the low nibble
 * of qs[j] plus 16 when bit j of the little-endian qh word is set, weight j+16 the high nibble plus
 * 16 when bit j+16 is.  w = q*d + m. */
void qo_dequant_q5_1_block(const uint8_t* blk, float* y) {
    uint16_t hd, hm; uint32_t qh; memcpy(&hd, blk, 2); memcpy(&hm, blk + 2, 2); memcpy(&qh, blk + 4, 4);
    const float d = qo_f16_to_f32(hd), m = qo_f16_to_f32(hm);
    const uint8_t* qs = blk + 8;
    for (int j = 0; j < 16; ++j) {
        const int lo = (qs[j] & 0x0f) | (int)(((qh >> j) & 1u) << 4);
        const int hi = (qs[j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
        y[j] = (float)lo * d + m;
        y[j + 16] = (float)hi * d + m;
    }
}

/* GGUF Q5_0 block = {f16 d, u8 qh[4], u8 qs[16]} (22 B): w = (q - 16)*d, q as in Q5_1.  The engine
 * never dequantises it directly: it repacks Q5_0 rows into the Q5_1 row-SoA layout with m = -16d
 * (gemv.hip:1448-1457).  This restatement is the format's definition, used to check that repack. */
void qo_dequant_q5_0_block(const uint8_t* blk, float* y) {
    uint16_t hd; uint32_t qh; memcpy(&hd, blk, 2); memcpy(&qh, blk + 2, 4);
    const float d = qo_f16_to_f32(hd);
    const uint8_t* qs = blk + 6;
    for (int j = 0; j < 16; ++j) {
        const int lo = (qs[j] & 0x0f) | (int)(((qh >> j) & 1u) << 4);
        const int hi = (qs[j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
        y[j] = (float)(lo - 16) * d;
        y[j + 16] = (float)(hi - 16) * d;
    }
}

/* gemv.hip:1351-1354: Q8_0 row -> row-SoA [qs K][d (K/32) x f16] */
void qo_repack_row_q8_0(const uint8_t* src, uint8_t* dst, int K) {
    for (int b = 0; b < K / 32; ++b) {
        memcpy(dst + (size_t)b * 32, src + (size_t)b * 34 + 2, 32);
        memcpy(dst + (size_t)K + (size_t)b * 2, src + (size_t)b * 34, 2);
    }
}
/* gemv.hip:1458-1465: Q5_1 row -> row-SoA [qs K/2][qh K/8][d (K/32) x f16][m (K/32) x f16] */
void qo_repack_row_q5_1(const uint8_t* src, uint8_t* dst, int K) {
    for (int b = 0; b < K / 32; ++b) {
        const uint8_t* blk = src + (size_t)b * 24;
        memcpy(dst + (size_t)b * 16, blk + 8, 16);
        memcpy(dst + (size_t)K / 2 + (size_t)b * 4, blk + 4, 4);
        memcpy(dst + (size_t)K / 2 + K / 8 + (size_t)b * 2, blk, 2);
        memcpy(dst + (size_t)K / 2 + K / 8 + K / 16 + (size_t)b * 2, blk + 2, 2);
    }
}
/* gemv.hip:1448-1457: Q5_0 row -> the Q5_1 row-SoA layout with m = f16(-16*d) (exact: a power-of-two
 * multiple of an f16 value, rounded to f16 -- exact unless it overflows) */
void qo_repack_row_q5_0(const uint8_t* src, uint8_t* dst, int K) {
    for (int b = 0; b < K / 32; ++b) {
        const uint8_t* blk = src + (size_t)b * 22;
        uint16_t hd; memcpy(&hd, blk, 2);
        const uint16_t hm = qo_f32_to_f16(-16.f * qo_f16_to_f32(hd));
        memcpy(dst + (size_t)b * 16, blk + 6, 16);
        memcpy(dst + (size_t)K / 2 + (size_t)b * 4, blk + 2, 4);
        memcpy(dst + (size_t)K / 2 + K / 8 + (size_t)b * 2, &hd, 2);
        memcpy(dst + (size_t)K / 2 + K / 8 + K / 16 + (size_t)b * 2, &hm, 2);
    }
}

size_t qo_row_bytes(int wfmt, int K) {
    switch (wfmt) {
        case QO_Q4_K: return (size_t)K / 256 * 144;
        case QO_Q5_K: return (size_t)K / 256 * 176;
        case QO_IQ4_XS: return (size_t)K / 256 * 136;
        case QO_Q6_K_SOA: case QO_Q6_K: return (size_t)K / 256 * 210;
        case QO_Q8_0_SOA: return (size_t)K + (size_t)K / 16;
        case QO_Q5_1_SOA: return (size_t)K / 32 * 24;
        case QO_Q8_0: return (size_t)K / 32 * 34;
        case QO_Q5_1: return (size_t)K / 32 * 24;
        case QO_Q5_0: return (size_t)K / 32 * 22;
        default: return 0;
    }
}
/* K granularity of a format: 256 for the super-block formats, 32 for the 32-weight block ones */
int qo_k_granule(int wfmt) {
    return (wfmt == QO_Q8_0_SOA || wfmt == QO_Q5_1_SOA || wfmt == QO_Q8_0 || wfmt == QO_Q5_1 || wfmt == QO_Q5_0) ? 32 : 256;
}

int qo_dequant_row(int wfmt, const uint8_t* row, float* y, int K) {
    const int nb = K / 256, n32 = K / 32;
    if (!qo_row_bytes(wfmt, K) || K % qo_k_granule(wfmt) != 0) return -1;
    switch (wfmt) {
        case QO_Q4_K: for (int b = 0; b < nb; ++b) qo_dequant_q4_K_block(row + (size_t)b * 144, y + (size_t)b * 256); return 0;
        case QO_Q5_K: for (int b = 0; b < nb; ++b) qo_dequant_q5_K_block(row + (size_t)b * 176, y + (size_t)b * 256); return 0;
        case QO_IQ4_XS: for (int b = 0; b < nb; ++b) qo_dequant_iq4_xs_block(row + (size_t)b * 136, y + (size_t)b * 256); return 0;
        case QO_Q8_0: for (int b = 0; b < n32; ++b) qo_dequant_q8_0_block(row + (size_t)b * 34, y + (size_t)b * 32); return 0;
        case QO_Q5_1: for (int b = 0; b < n32; ++b) qo_dequant_q5_1_block(row + (size_t)b * 24, y + (size_t)b * 32); return 0;
        case QO_Q5_0: for (int b = 0; b < n32; ++b) qo_dequant_q5_0_block(row + (size_t)b * 22, y + (size_t)b * 32); return 0;
        case QO_Q8_0_SOA: {     /* gather block b back from the SoA streams, then decode as a GGUF block */
            uint8_t blk[34];
            for (int b = 0; b < n32; ++b) {
                memcpy(blk, row + (size_t)K + (size_t)b * 2, 2);
                memcpy(blk + 2, row + (size_t)b * 32, 32);
                qo_dequant_q8_0_block(blk, y + (size_t)b * 32);
            }
            return 0;
        }
        case QO_Q5_1_SOA: {
            uint8_t blk[24];
            for (int b = 0; b < n32; ++b) {
                memcpy(blk, row + (size_t)K / 2 + K / 8 + (size_t)b * 2, 2);
                memcpy(blk + 2, row + (size_t)K / 2 + K / 8 + K / 16 + (size_t)b * 2, 2);
                memcpy(blk + 4, row + (size_t)K / 2 + (size_t)b * 4, 4);
                memcpy(blk + 8, row + (size_t)b * 16, 16);
                qo_dequant_q5_1_block(blk, y + (size_t)b * 32);
            }
            return 0;
        }
        case QO_Q6_K: for (int b = 0; b < nb; ++b) qo_dequant_q6_K_block(row + (size_t)b * 210, y + (size_t)b * 256); return 0;
        case QO_Q6_K_SOA: {
            /* gather block b back from the SoA streams, then decode as a GGUF block */
            uint8_t blk[210];
            for (int b = 0; b < nb; ++b) {
                memcpy(blk, row + (size_t)b * 128, 128);
                memcpy(blk + 128, row + (size_t)nb * 128 + (size_t)b * 64, 64);
                memcpy(blk + 192, row + (size_t)nb * 192 + (size_t)b * 16, 16);
                memcpy(blk + 208, row + (size_t)nb * 208 + (size_t)b * 2, 2);
                qo_dequant_q6_K_block(blk, y + (size_t)b * 256);
            }
            return 0;
        }
        default: return -1;
    }
}

typedef struct { int wfmt; const uint8_t* W; int K; size_t rb; float* outf; uint16_t* outb; } dq_ctx;
static void dq_body(void* p, int lo, int hi) {
    dq_ctx* c = (dq_ctx*)p;
    float* tmp = c->outb ? (float*)malloc(sizeof(float) * (size_t)c->K) : NULL;
    for (int r = lo; r < hi; ++r) {
        if (c->outf) qo_dequant_row(c->wfmt, c->W + (size_t)r * c->rb, c->outf + (size_t)r * c->K, c->K);
        else {
            qo_dequant_row(c->wfmt, c->W + (size_t)r * c->rb, tmp, c->K);
            for (int k = 0; k < c->K; ++k) c->outb[(size_t)r * c->K + k] = qo_f32_to_bf16(tmp[k]);
        }
    }
    free(tmp);
}
int qo_dequant_matrix(int wfmt, const uint8_t* W, int N, int K, float* out, int nthreads) {
    if (!qo_row_bytes(wfmt, K) || K % qo_k_granule(wfmt)) return -1;
    dq_ctx c = {wfmt, W, K, qo_row_bytes(wfmt, K), out, NULL};
    qo_parallel(N, nthreads, dq_body, &c); return 0;
}
int qo_dequant_matrix_bf16(int wfmt, const uint8_t* W, int N, int K, uint16_t* out, int nthreads) {
    if (!qo_row_bytes(wfmt, K) || K % qo_k_granule(wfmt)) return -1;
    dq_ctx c = {wfmt, W, K, qo_row_bytes(wfmt, K), NULL, out};
    qo_parallel(N, nthreads, dq_body, &c); return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* activations                                                                                 */

/* bench_gemv.cpp:17-25 (== the device quantiser gemv.hip:36-51): per 32 values amax, d=amax/127,
 * id = 127/amax (0 when amax == 0), q = round-half-even(x*id), s = d*sum(q). */
void qo_quantize_x_q8(const float* x, int K, int8_t* q, float* d, float* s) {
    for (int b = 0; b < K / 32; ++b) {
        float amax = 0.f;
        for (int l = 0; l < 32; ++l) amax = fmaxf(amax, fabsf(x[b * 32 + l]));
        const float dd = amax / 127.f, id = amax > 0 ? 127.f / amax : 0.f;
        int sum = 0;
        for (int l = 0; l < 32; ++l) {
            const int qi = (int)nearbyintf(x[b * 32 + l] * id);
            q[b * 32 + l] = (int8_t)qi; sum += qi;
        }
        d[b] = dd; s[b] = dd * (float)sum;
    }
}
/* gemv.hip:686-705 (quantize_x_q8k): one scale per 256 values, d = amax/127 over the 256, q = rne(x * 127/amax)
 * (0 when amax == 0), bs = the int16 sum of each 32 q.  Column c of ncol <= 16: q at q + c*K, d[b*16 + c],
 * bs[(b*16 + c)*8 + j] (the reference's XQ8K layout, gemv.h:33). */
void qo_quantize_x_q8k(const float* x, int K, int ncol, int8_t* q, float* d, int16_t* bs) {
    for (int c = 0; c < ncol; ++c)
        for (int b = 0; b < K / 256; ++b) {
            const float* xb = x + (size_t)c * K + (size_t)b * 256;
            float amax = 0.f;
            for (int l = 0; l < 256; ++l) amax = fmaxf(amax, fabsf(xb[l]));
            const float dd = amax / 127.f, id = amax > 0 ? 127.f / amax : 0.f;
            for (int j = 0; j < 8; ++j) {
                int sum = 0;
                for (int l = 0; l < 32; ++l) {
                    const int qi = (int)nearbyintf(xb[32 * j + l] * id);
                    q[(size_t)c * K + (size_t)b * 256 + 32 * j + l] = (int8_t)qi; sum += qi;
                }
                bs[((size_t)b * 16 + c) * 8 + j] = (int16_t)sum;
            }
            d[(size_t)b * 16 + c] = dd;
        }
}
void qo_q8_to_f32(const int8_t* q, const float* d, int K, float* xr) {
    for (int k = 0; k < K; ++k) xr[k] = (float)q[k] * d[k / 32];
}
/* fn.hip:8,206-211: silu(g) = g / (1 + exp(-g)), times u */
void qo_silu_mul(const float* g, const float* u, size_t n, float* h) {
    for (size_t i = 0; i < n; ++i) h[i] = g[i] / (1.f + expf(-g[i])) * u[i];
}

/* ops.hip:64-78 (block_sum1024): 1024 per-thread partials folded by the xor butterfly of
 * __shfl_xor(v, o, 32), o = 16..1, inside each group of 32 threads, then the same butterfly over the
 * 32 group sums.  Lane l adds lane l^o; both partners form the same sum, so it is a pairwise tree. */
float qo_block_sum1024(const float* part) {
    float g[32];
    for (int w = 0; w < 32; ++w) {
        float a[32], b[32];
        for (int l = 0; l < 32; ++l) a[l] = part[w * 32 + l];
        for (int o = 16; o > 0; o >>= 1) {
            for (int l = 0; l < 32; ++l) b[l] = a[l] + a[l ^ o];
            for (int l = 0; l < 32; ++l) a[l] = b[l];
        }
        g[w] = a[0];
    }
    for (int o = 16; o > 0; o >>= 1) {
        float b[32];
        for (int l = 0; l < 32; ++l) b[l] = g[l] + g[l ^ o];
        for (int l = 0; l < 32; ++l) g[l] = b[l];
    }
    return g[0];
}

/* one row of ops.hip:79-98 / 111-120: x += y (when y), the scale 1/sqrt(ss/n + eps) with ss the sum
 * of squares of 1024 threads (thread t: fma over elements t, t+1024, ... in that order, then
 * block_sum1024).  The reference's rsqrtf is replaced by the correctly rounded value (1/sqrt in
 * double, rounded once), which the library computes the same way. */
static float rms_row(float* x, const float* y, int n, float eps) {
    float part[1024];
    for (int t = 0; t < 1024; ++t) {
        float ss = 0.f;
        for (int i = t; i < n; i += 1024) {
            float a = x[i];
            if (y) { a += y[i]; x[i] = a; }
            ss = fmaf(a, a, ss);
        }
        part[t] = ss;
    }
    const float tot = qo_block_sum1024(part);
    return (float)(1.0 / sqrt((double)(tot / (float)n + eps)));
}

/* ops.hip:79-98: per row, x += y, xn = x * sc * w ((x*sc)*w, two roundings), q8 of xn per 32 */
int qo_add_rmsnorm_quant(float* x, const float* y, const float* w, float* xn, int8_t* q, float* d, float* s, int T, int n,
                         float eps) {
    if (n <= 0 || n % 32 != 0 || n > 32768) return -1;
    for (int t = 0; t < T; ++t) {
        float* xr = x + (size_t)t * n;
        float* on = xn + (size_t)t * n;
        const float sc = rms_row(xr, y ? y + (size_t)t * n : NULL, n, eps);
        for (int i = 0; i < n; ++i) on[i] = xr[i] * sc * w[i];
        qo_quantize_x_q8(on, n, q + (size_t)t * n, d + (size_t)t * (n / 32), s + (size_t)t * (n / 32));
    }
    return 0;
}

/* ops.hip:111-120: per row, x += y, xb = bf16(x * sc * w) */
int qo_add_rmsnorm_bf16(float* x, const float* y, const float* w, uint16_t* xb, int T, int n, float eps) {
    if (n <= 0 || n > 32768) return -1;
    for (int t = 0; t < T; ++t) {
        float* xr = x + (size_t)t * n;
        const float sc = rms_row(xr, y ? y + (size_t)t * n : NULL, n, eps);
        for (int i = 0; i < n; ++i) xb[(size_t)t * n + i] = qo_f32_to_bf16(xr[i] * sc * w[i]);
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* GEMV references                                                                             */

typedef struct {
    int wfmt; const uint8_t* W; int N, K; const float* x; int ncol; size_t rb;
    double* y; double* mag; float* yf; const int* rows;
} gv_ctx;
static void gv_ref_body(void* p, int lo, int hi) {
    gv_ctx* c = (gv_ctx*)p;
    float* w = (float*)malloc(sizeof(float) * (size_t)c->K);
    for (int i = lo; i < hi; ++i) {
        const int r = c->rows ? c->rows[i] : i;
        qo_dequant_row(c->wfmt, c->W + (size_t)r * c->rb, w, c->K);
        for (int col = 0; col < c->ncol; ++col) {
            const float* xc = c->x + (size_t)col * c->K;
            double acc = 0, mg = 0;
            for (int k = 0; k < c->K; ++k) { const double v = (double)w[k] * (double)xc[k]; acc += v; mg += fabs(v); }
            /* c->N is the row count of y: N for a full GEMV, nrows for a sampled-row one */
            c->y[(size_t)col * c->N + i] = acc;
            if (c->mag) c->mag[(size_t)col * c->N + i] = mg;
        }
    }
    free(w);
}
int qo_gemv_ref(int wfmt, const uint8_t* W, int N, int K, const float* x, int ncol,
                double* y, double* mag, int nthreads) {
    if (!qo_row_bytes(wfmt, K) || K % qo_k_granule(wfmt)) return -1;
    gv_ctx c = {wfmt, W, N, K, x, ncol, qo_row_bytes(wfmt, K), y, mag, NULL, NULL};
    qo_parallel(N, nthreads, gv_ref_body, &c); return 0;
}
int qo_gemv_ref_rows(int wfmt, const uint8_t* W, int N, int K, const float* x, int ncol,
                     const int* rows, int nrows, double* y, double* mag) {
    if (!qo_row_bytes(wfmt, K) || K % qo_k_granule(wfmt)) return -1;
    for (int i = 0; i < nrows; ++i) if (rows[i] < 0 || rows[i] >= N) return -2;
    /* y/mag are [ncol][nrows]: reuse the body with N := nrows as the output stride */
    gv_ctx c = {wfmt, W, nrows, K, x, ncol, qo_row_bytes(wfmt, K), y, mag, NULL, rows};
    gv_ref_body(&c, 0, nrows); return 0;
}

/* CPU baseline: the reference's host scalar path (dequant a row, fp32 dot), one row per step */
static void gv_f32_body(void* p, int lo, int hi) {
    gv_ctx* c = (gv_ctx*)p;
    float* w = (float*)malloc(sizeof(float) * (size_t)c->K);
    for (int r = lo; r < hi; ++r) {
        qo_dequant_row(c->wfmt, c->W + (size_t)r * c->rb, w, c->K);
        for (int col = 0; col < c->ncol; ++col) {
            const float* xc = c->x + (size_t)col * c->K;
            float acc = 0.f;
            for (int k = 0; k < c->K; ++k) acc += w[k] * xc[k];
            c->yf[(size_t)col * c->N + r] = acc;
        }
    }
    free(w);
}
int qo_gemv_f32(int wfmt, const uint8_t* W, int N, int K, const float* x, int ncol, float* y, int nthreads) {
    if (!qo_row_bytes(wfmt, K) || K % qo_k_granule(wfmt)) return -1;
    gv_ctx c = {wfmt, W, N, K, x, ncol, qo_row_bytes(wfmt, K), NULL, NULL, y, NULL};
    qo_parallel(N, nthreads, gv_f32_body, &c); return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* MoE routing, sort, decode and prefill references                                            */

/* fn.hip:157-205 (k_moe_route), for nexp experts (the reference: 512) and top-k (the reference: 10):
 *   mx = max of the logits; e_i = exp(l_i - mx);
 *   sum = S_0 + S_1 + ... in that order, S_g the xor-butterfly sum (lane l with l^16, then l^8, ..., l^1;
 *         a pairwise tree) of e over experts 32g .. 32g+31 (experts past nexp add nothing);
 *   p_i = e_i / sum; the top-k by p, ties to the lower id (k rounds of argmax); w_r = p_r / wsum with
 *   wsum the sum of the selected p in selection order; slot k: id -1, w = sigmoid(l[nexp]).
 * The device exp (__expf) and the host libm's expf may differ in the last ulp. */
static float tree32(const float* e) {
    float a[32], b[32];
    for (int l = 0; l < 32; ++l) a[l] = e[l];
    for (int o = 16; o > 0; o >>= 1) {
        for (int l = 0; l < 32; ++l) b[l] = a[l] + a[l ^ o];
        for (int l = 0; l < 32; ++l) a[l] = b[l];
    }
    return a[0];
}
void qo_moe_route(const float* logits, int T, int nexp, int stride, int topk, int* ids, float* w) {
    const int ng = (nexp + 31) / 32;
    float* e = (float*)calloc((size_t)ng * 32, sizeof(float));
    float* p = (float*)malloc(sizeof(float) * (size_t)nexp);
    char* used = (char*)malloc((size_t)nexp);
    for (int t = 0; t < T; ++t) {
        const float* l = logits + (size_t)t * stride;
        float mx = l[0];
        for (int i = 1; i < nexp; ++i) mx = fmaxf(mx, l[i]);
        for (int i = 0; i < nexp; ++i) e[i] = expf(l[i] - mx);
        float sum = 0.f;
        for (int g = 0; g < ng; ++g) sum += tree32(e + 32 * g);
        for (int i = 0; i < nexp; ++i) p[i] = e[i] / sum;
        memset(used, 0, (size_t)nexp);
        float wsum = 0.f;
        int* id = ids + (size_t)t * (topk + 1); float* ww = w + (size_t)t * (topk + 1);
        for (int r = 0; r < topk; ++r) {
            int bi = -1;
            for (int i = 0; i < nexp; ++i) if (!used[i] && (bi < 0 || p[i] > p[bi])) bi = i;
            used[bi] = 1; id[r] = bi; ww[r] = p[bi]; wsum += p[bi];
        }
        for (int r = 0; r < topk; ++r) ww[r] /= wsum;
        id[topk] = -1; ww[topk] = 1.f / (1.f + expf(-l[nexp]));
    }
    free(e); free(p); free(used);
}

/* fn.hip:251-277 (k_f32_gemv), y[t][n] = W[n] . x[t]: 32 lanes per row, lane l summing the float4 steps
 * i = 4l + 128k in order, each step t = fma(a.w,b.w, fma(a.z,b.z, fma(a.x,b.x, a.y*b.y))) and
 * acc = acc + t -- the contraction the reference's own hipcc build (-O3) makes of
 * `acc += a.x*b.x + a.y*b.y + a.z*b.z + a.w*b.w` (v_mul, then three v_fmac, then v_add) -- and the
 * 32 partial sums folded by the xor butterfly.  K % 4 == 0. */
int qo_f32_gemv(const float* W, const float* x, float* y, int N, int K, int T) {
    if (K <= 0 || K % 4 != 0) return -1;
    for (int t = 0; t < T; ++t)
        for (int n = 0; n < N; ++n) {
            const float* a = W + (size_t)n * K;
            const float* b = x + (size_t)t * K;
            float acc[32];
            for (int l = 0; l < 32; ++l) {
                float s = 0.f;
                for (int i = 4 * l; i < K; i += 128) {
                    const float u = fmaf(a[i + 3], b[i + 3], fmaf(a[i + 2], b[i + 2], fmaf(a[i], b[i], a[i + 1] * b[i + 1])));
                    s = s + u;
                }
                acc[l] = s;
            }
            y[(size_t)t * N + n] = tree32(acc);
        }
    return 0;
}

/* qwen4exp.cpp:628-641.  Sorting by (eid, te) is a stable counting sort over the slots taken in
 * te order; -1 (shared) sorts first. */
int qo_moe_sort(const int* eid, int T, int NE, int maxc, int* kpos, int* rowtok, int* tiles, int* nstiles) {
    const int NS = T * NE;
    int maxe = -1;
    for (int i = 0; i < NS; ++i) if (eid[i] > maxe) maxe = eid[i];
    const int nb = maxe + 2;   /* bucket 0 = shared (-1), bucket e+1 = expert e */
    int* cnt = (int*)calloc((size_t)nb + 1, sizeof(int));
    for (int i = 0; i < NS; ++i) cnt[eid[i] + 1 + 1]++;
    for (int b = 1; b <= nb; ++b) cnt[b] += cnt[b - 1];
    int* order = (int*)malloc(sizeof(int) * (size_t)NS);
    for (int te = 0; te < NS; ++te) order[cnt[eid[te] + 1]++] = te;
    int nt = 0, ns = 0;
    int* st = (int*)malloc(sizeof(int) * 3 * (size_t)(NS + 1));
    for (int k = 0; k < NS; ++k) {
        const int te = order[k];
        kpos[te] = k; rowtok[k] = te / NE;
        const int e = eid[te];
        int* lst = e < 0 ? st : tiles; int* n = e < 0 ? &ns : &nt;
        if (*n == 0 || (k > 0 && e != eid[order[k - 1]]) || lst[3 * (*n - 1) + 2] == maxc) {
            lst[3 * *n] = e; lst[3 * *n + 1] = k; lst[3 * *n + 2] = 1; ++*n;
        } else lst[3 * (*n - 1) + 2]++;
    }
    memcpy(tiles + 3 * nt, st, sizeof(int) * 3 * (size_t)ns);
    *nstiles = ns;
    free(cnt); free(order); free(st);
    return nt;
}

/* y = W_row . xr in double, W given as a dequantised f32 row (helper for the MoE references) */
static double dot_fd(const float* w, const float* x, int K) {
    double a = 0; for (int k = 0; k < K; ++k) a += (double)w[k] * (double)x[k]; return a;
}

/* gemv.hip:1075-1114 (per-slot gate/up on the token's q8 row, down on the slot's q8 h row,
 * combine sum_e slotw[te] * dot in slot order) + fn.hip:206-211 (h = silu(g)*u, q8 per 32). */
int qo_moe_decode(int wfmt, const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd,
                  size_t ebytes_gu, size_t ebytes_d, const uint8_t* Sg, const uint8_t* Su,
                  const uint8_t* Sd, const float* x, const int* ids, const float* w, int T, int NE,
                  int H, int F, float* g, float* u, float* dn, float* y) {
    const size_t rb_gu = qo_row_bytes(wfmt, H), rb_d = qo_row_bytes(wfmt, F);
    if (!rb_gu || !rb_d) return -1;
    float* wrow = (float*)malloc(sizeof(float) * (size_t)(H > F ? H : F));
    float* xr = (float*)malloc(sizeof(float) * (size_t)H);
    int8_t* q = (int8_t*)malloc((size_t)(H > F ? H : F));
    float* qd = (float*)malloc(sizeof(float) * (size_t)(H > F ? H : F) / 32 + 4);
    float* qs = (float*)malloc(sizeof(float) * (size_t)(H > F ? H : F) / 32 + 4);
    float* h = (float*)malloc(sizeof(float) * (size_t)F);
    float* hr = (float*)malloc(sizeof(float) * (size_t)F);
    for (int t = 0; t < T; ++t) {
        qo_quantize_x_q8(x + (size_t)t * H, H, q, qd, qs);
        qo_q8_to_f32(q, qd, H, xr);
        for (int e = 0; e < NE; ++e) {
            const int te = t * NE + e, id = ids[te];
            const uint8_t* wg = id >= 0 ? Wg + (size_t)id * ebytes_gu : Sg;
            const uint8_t* wu = id >= 0 ? Wu + (size_t)id * ebytes_gu : Su;
            for (int n = 0; n < F; ++n) {
                qo_dequant_row(wfmt, wg + (size_t)n * rb_gu, wrow, H); g[(size_t)te * F + n] = (float)dot_fd(wrow, xr, H);
                qo_dequant_row(wfmt, wu + (size_t)n * rb_gu, wrow, H); u[(size_t)te * F + n] = (float)dot_fd(wrow, xr, H);
            }
        }
    }
    for (int t = 0; t < T; ++t) {
        for (int n = 0; n < H; ++n) y[(size_t)t * H + n] = 0.f;
        double* acc = (double*)calloc((size_t)H, sizeof(double));
        for (int e = 0; e < NE; ++e) {
            const int te = t * NE + e, id = ids[te];
            qo_silu_mul(g + (size_t)te * F, u + (size_t)te * F, (size_t)F, h);
            qo_quantize_x_q8(h, F, q, qd, qs);
            qo_q8_to_f32(q, qd, F, hr);
            const uint8_t* wd = id >= 0 ? Wd + (size_t)id * ebytes_d : Sd;
            for (int n = 0; n < H; ++n) {
                qo_dequant_row(wfmt, wd + (size_t)n * rb_d, wrow, F);
                const double v = dot_fd(wrow, hr, F);
                dn[(size_t)te * H + n] = (float)v;
                acc[n] += (double)w[te] * v;
            }
        }
        for (int n = 0; n < H; ++n) y[(size_t)t * H + n] = (float)acc[n];
        free(acc);
    }
    free(wrow); free(xr); free(q); free(qd); free(qs); free(h); free(hr);
    return 0;
}

int qo_moe_down_q8(int wfmt, const uint8_t* Wd, size_t ebytes_d, const uint8_t* Sd,
                   const int8_t* hq, const float* hd, const int* ids, const float* w, int T,
                   int NE, int H, int F, float* dn, float* y) {
    const size_t rb_d = qo_row_bytes(wfmt, F);
    if (!rb_d) return -1;
    float* wrow = (float*)malloc(sizeof(float) * (size_t)F);
    float* hr = (float*)malloc(sizeof(float) * (size_t)F);
    double* acc = (double*)malloc(sizeof(double) * (size_t)H);
    for (int t = 0; t < T; ++t) {
        for (int n = 0; n < H; ++n) acc[n] = 0;
        for (int e = 0; e < NE; ++e) {
            const int te = t * NE + e, id = ids[te];
            qo_q8_to_f32(hq + (size_t)te * F, hd + (size_t)te * (F / 32), F, hr);
            const uint8_t* wd = id >= 0 ? Wd + (size_t)id * ebytes_d : Sd;
            for (int n = 0; n < H; ++n) {
                qo_dequant_row(wfmt, wd + (size_t)n * rb_d, wrow, F);
                const double v = dot_fd(wrow, hr, F);
                if (dn) dn[(size_t)te * H + n] = (float)v;
                acc[n] += (double)w[te] * v;
            }
        }
        for (int n = 0; n < H; ++n) y[(size_t)t * H + n] = (float)acc[n];
    }
    free(wrow); free(hr); free(acc);
    return 0;
}

typedef struct {
    int wfmt; const uint8_t *Wg, *Wu, *Wd; size_t eb_gu, eb_d; const uint8_t *Sg, *Su, *Sd;
    const uint16_t* xb; const int* ids; const float* w; int NE, H, F; const int* toks; float* y;
} mp_ctx;
static void mp_body(void* p, int lo, int hi) {
    mp_ctx* c = (mp_ctx*)p;
    const int H = c->H, F = c->F;
    const size_t rb_gu = qo_row_bytes(c->wfmt, H), rb_d = qo_row_bytes(c->wfmt, F);
    float* wrow = (float*)malloc(sizeof(float) * (size_t)(H > F ? H : F));
    float* x = (float*)malloc(sizeof(float) * (size_t)H);
    float* h = (float*)malloc(sizeof(float) * (size_t)F);
    double* acc = (double*)malloc(sizeof(double) * (size_t)H);
    for (int i = lo; i < hi; ++i) {
        const int t = c->toks[i];
        for (int k = 0; k < H; ++k) x[k] = qo_bf16_to_f32(c->xb[(size_t)t * H + k]);
        for (int n = 0; n < H; ++n) acc[n] = 0;
        for (int e = 0; e < c->NE; ++e) {
            const int te = t * c->NE + e, id = c->ids[te];
            const uint8_t* wg = id >= 0 ? c->Wg + (size_t)id * c->eb_gu : c->Sg;
            const uint8_t* wu = id >= 0 ? c->Wu + (size_t)id * c->eb_gu : c->Su;
            const uint8_t* wd = id >= 0 ? c->Wd + (size_t)id * c->eb_d : c->Sd;
            for (int n = 0; n < F; ++n) {
                double gv = 0, uv = 0;
                qo_dequant_row(c->wfmt, wg + (size_t)n * rb_gu, wrow, H);
                for (int k = 0; k < H; ++k) gv += (double)qo_bf16_to_f32(qo_f32_to_bf16(wrow[k])) * x[k];
                qo_dequant_row(c->wfmt, wu + (size_t)n * rb_gu, wrow, H);
                for (int k = 0; k < H; ++k) uv += (double)qo_bf16_to_f32(qo_f32_to_bf16(wrow[k])) * x[k];
                const float gf = (float)gv, uf = (float)uv;
                h[n] = qo_bf16_to_f32(qo_f32_to_bf16(gf / (1.f + expf(-gf)) * uf));
            }
            for (int n = 0; n < H; ++n) {
                qo_dequant_row(c->wfmt, wd + (size_t)n * rb_d, wrow, F);
                double dv = 0;
                for (int k = 0; k < F; ++k) dv += (double)qo_bf16_to_f32(qo_f32_to_bf16(wrow[k])) * h[k];
                acc[n] += (double)c->w[te] * (double)(float)dv;
            }
        }
        for (int n = 0; n < H; ++n) c->y[(size_t)i * H + n] = (float)acc[n];
    }
    free(wrow); free(x); free(h); free(acc);
}
int qo_moe_prefill_tokens(int wfmt, const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd,
                          size_t ebytes_gu, size_t ebytes_d, const uint8_t* Sg, const uint8_t* Su,
                          const uint8_t* Sd, const uint16_t* xb, const int* ids, const float* w,
                          int NE, int H, int F, const int* toks, int ntok, float* y, int nthreads) {
    if (!qo_row_bytes(wfmt, H) || !qo_row_bytes(wfmt, F)) return -1;
    mp_ctx c = {wfmt, Wg, Wu, Wd, ebytes_gu, ebytes_d, Sg, Su, Sd, xb, ids, w, NE, H, F, toks, y};
    qo_parallel(ntok, nthreads, mp_body, &c);
    return 0;
}

int qo_gemm_wq_ref(int wfmt, const uint8_t* W, const uint16_t* A, int M, int N, int K,
                   const int* ms, const int* ns, int npairs, double* out) {
    const size_t rb = qo_row_bytes(wfmt, K);
    if (!rb || K % 256) return -1;
    float* w = (float*)malloc(sizeof(float) * (size_t)K);
    int last = -1;
    for (int i = 0; i < npairs; ++i) {
        if (ms[i] < 0 || ms[i] >= M || ns[i] < 0 || ns[i] >= N) { free(w); return -2; }
        if (ns[i] != last) { qo_dequant_row(wfmt, W + (size_t)ns[i] * rb, w, K); last = ns[i]; }
        double acc = 0;
        for (int k = 0; k < K; ++k)
            acc += (double)qo_bf16_to_f32(qo_f32_to_bf16(w[k])) * (double)qo_bf16_to_f32(A[(size_t)ms[i] * K + k]);
        out[i] = acc;
    }
    free(w);
    return 0;
}
