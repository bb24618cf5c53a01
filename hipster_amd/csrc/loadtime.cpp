// loadtime.cpp -- the engine's load-time choice of the layout the kernels read for a GGUF weight, and the
// row repacks / requantisation that produce it.  Host code only (no GPU calls).
//
//   qmm_weight_format,
//   qmm_prepare_weight     to_lin / upload_lin  engine/src/qwen4exp.cpp:34-65, qwen35.cpp:31-58
//
// Block formats the kernels read as they are (Q4_K, Q5_K, IQ4_XS) are copied; Q6_K, Q8_0, Q5_1 and Q5_0
// rows take the row repacks of capi.cpp; F32 / F16 / BF16 rows are requantised to Q8_0 row-SoA with the
// reference's own f32 -> f16 rounding of the scale (quant.h:150-183), so the bytes equal the reference's.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <thread>
#include <vector>

#include "../../include/hipster_qmm.h"

namespace {

// f32 -> f16 as quant.h:150-155 does it: truncate the mantissa and add one when the first dropped bit
// is set (round half away from zero in magnitude), subnormals alike; tiny values -> signed zero,
// large ones -> infinity
uint16_t f32_to_f16_loadtime(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t s = (x >> 16) & 0x8000u;
    const int e = (int)((x >> 23) & 0xffu) - 127 + 15;
    uint32_t m = x & 0x7fffffu;
    if (e <= 0) {
        if (e < -10) return (uint16_t)s;
        m |= 0x800000u;
        const uint32_t t = (uint32_t)(14 - e);
        uint32_t r = m >> t;
        if ((m >> (t - 1)) & 1u) r++;
        return (uint16_t)(s | r);
    }
    if (e >= 31) return (uint16_t)(s | 0x7c00u);
    uint32_t r = s | ((uint32_t)e << 10) | (m >> 13);
    if (m & 0x1000u) r++;
    return (uint16_t)r;
}
float f16_to_f32_host(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) bits = sign;
        else {
            const float v = ldexpf((float)m, -24);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) bits = sign | 0x7f800000u | (m << 13);
    else bits = sign | ((e + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// one row of F32 / F16 / BF16 -> f32 (quant.h:197-199)
void float_row(int type, const uint8_t* src, float* dst, int K) {
    if (type == QMM_GGML_F32) memcpy(dst, src, (size_t)K * 4);
    else if (type == QMM_GGML_F16) for (int i = 0; i < K; ++i) { uint16_t h; memcpy(&h, src + 2 * i, 2); dst[i] = f16_to_f32_host(h); }
    else for (int i = 0; i < K; ++i) { uint16_t b; memcpy(&b, src + 2 * i, 2); const uint32_t u = (uint32_t)b << 16; memcpy(dst + i, &u, 4); }
}

// f32 row -> Q8_0 row-SoA [q K int8][d K/32 f16] (quant.h:174-183): d = f16(amax/127), q = rint(x / d)
void quantize_row_q8_0_soa(const float* x, uint8_t* dst, int K) {
    int8_t* q = (int8_t*)dst;
    uint8_t* dd = dst + K;
    for (int b = 0; b < K / 32; ++b) {
        float amax = 0.f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[b * 32 + j]));
        const uint16_t h = f32_to_f16_loadtime(amax / 127.f);
        memcpy(dd + 2 * b, &h, 2);
        const float dq = f16_to_f32_host(h), idq = dq != 0.f ? 1.f / dq : 0.f;
        for (int j = 0; j < 32; ++j) q[b * 32 + j] = (int8_t)nearbyintf(x[b * 32 + j] * idq);
    }
}

template <class F>
void parallel_rows(int N, int nthreads, F fn) {
    if (nthreads <= 1 || N < 2) {
        for (int r = 0; r < N; ++r) fn(r);
        return;
    }
    std::vector<std::thread> th;
    for (int i = 0; i < nthreads; ++i) th.emplace_back([=] { for (int r = i; r < N; r += nthreads) fn(r); });
    for (auto& t : th) t.join();
}

}  // namespace

extern "C" {

int qmm_weight_format(int gtype, int K, int* wfmt, size_t* row_bytes) {
    if (!wfmt || !row_bytes) return QMM_ERR_NULL;
    int f;
    switch (gtype) {
        case QMM_GGML_Q4_K: f = QMM_Q4_K; break;
        case QMM_GGML_Q5_K: f = QMM_Q5_K; break;
        case QMM_GGML_IQ4_XS: f = QMM_IQ4_XS; break;
        case QMM_GGML_Q6_K: f = QMM_Q6_K_SOA; break;
        case QMM_GGML_Q8_0: f = QMM_Q8_0_SOA; break;
        case QMM_GGML_Q5_0: case QMM_GGML_Q5_1: f = QMM_Q5_1_SOA; break;
        case QMM_GGML_F32: case QMM_GGML_F16: case QMM_GGML_BF16: f = QMM_Q8_0_SOA; break;   // requantised at load
        default: return QMM_ERR_FORMAT;
    }
    const size_t rb = qmm_wfmt_row_bytes(f, K);
    if (rb == 0) return QMM_ERR_SHAPE;
    *wfmt = f;
    *row_bytes = rb;
    return QMM_OK;
}

int qmm_prepare_weight(int gtype, const uint8_t* src, int N, int K, uint8_t* dst, int nthreads) {
    if (!src || !dst) return QMM_ERR_NULL;
    int f;
    size_t rb;
    if (int e = qmm_weight_format(gtype, K, &f, &rb)) return e;
    if (N <= 0) return QMM_ERR_SHAPE;
    uint32_t bs, tb;
    if (qmm_gtype_block(gtype, &bs, &tb) != QMM_OK || K % (int)bs != 0) return QMM_ERR_SHAPE;
    const size_t rs = (size_t)(K / (int)bs) * tb;             // source row bytes
    nthreads = nthreads < 1 ? 1 : (nthreads > 64 ? 64 : nthreads);
    int rc = QMM_OK;
    switch (gtype) {
        case QMM_GGML_Q4_K: case QMM_GGML_Q5_K: case QMM_GGML_IQ4_XS:
            memcpy(dst, src, rs * (size_t)N);
            break;
        case QMM_GGML_Q6_K:
            parallel_rows(N, nthreads, [&](int r) { qmm_repack_row_q6_K(src + (size_t)r * rs, dst + (size_t)r * rb, K); });
            break;
        case QMM_GGML_Q8_0:
            parallel_rows(N, nthreads, [&](int r) { qmm_repack_row_q8_0(src + (size_t)r * rs, dst + (size_t)r * rb, K); });
            break;
        case QMM_GGML_Q5_1:
            parallel_rows(N, nthreads, [&](int r) { qmm_repack_row_q5_1(src + (size_t)r * rs, dst + (size_t)r * rb, K); });
            break;
        case QMM_GGML_Q5_0:
            parallel_rows(N, nthreads, [&](int r) { qmm_repack_row_q5_0(src + (size_t)r * rs, dst + (size_t)r * rb, K); });
            break;
        default:                                               // F32 / F16 / BF16 -> Q8_0_SOA
            parallel_rows(N, nthreads, [&](int r) {
                std::vector<float> row((size_t)K);
                float_row(gtype, src + (size_t)r * rs, row.data(), K);
                quantize_row_q8_0_soa(row.data(), dst + (size_t)r * rb, K);
            });
            break;
    }
    return rc;
}

}  // extern "C"
