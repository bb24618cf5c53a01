// capi.cpp -- host-only entry points of the C ABI (no kernels): version, status strings and the
// row-layout helpers of the reference (engine/kernels/gemv.hip:1337-1354,1448-1465).
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../../include/hipster_qmm.h"

namespace {
// IEEE half <-> float for the host repacks (g++ here has no _Float16).  f2h rounds to nearest
// even, overflow gives infinity; NaN keeps its sign and becomes a quiet NaN.
float h2f_host(uint16_t h) {
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
uint16_t f2h_host(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const float a = fabsf(f);
    if (a != a) return (uint16_t)(sign | 0x7e00u);
    if (!(a < 65520.f)) return (uint16_t)(sign | 0x7c00u);
    if (a < 6.103515625e-05f) return (uint16_t)(sign | (uint16_t)nearbyintf(a * 16777216.f));
    uint32_t v;
    memcpy(&v, &a, 4);
    const uint32_t mant = v & 0x7fffffu, exp = (v >> 23) - 112u, rest = mant & 0x1fffu;
    uint32_t h = (exp << 10) | (mant >> 13);
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}
}  // namespace

extern "C" {

const char* qmm_version(void) { return "hipster_qmm 0.1 (gfx950)"; }

const char* qmm_status_string(int status) {
    switch (status) {
        case QMM_OK: return "ok";
        case QMM_ERR_FORMAT: return "unsupported weight format";
        case QMM_ERR_SHAPE: return "invalid shape";
        case QMM_ERR_NULL: return "null pointer";
        case QMM_ERR_LAUNCH: return "kernel launch failed";
        case QMM_ERR_WORKSPACE: return "workspace missing or too small";
        case QMM_ERR_ARG: return "invalid argument";
        case QMM_ERR_LAYOUT: return "weight layout not supported (the reference's experimental interleaved layouts)";
        case QMM_ERR_IO: return "GGUF file missing, truncated, not GGUF v3, or a tensor past its end";
        case QMM_ERR_NOT_FOUND: return "tensor or key not found";
        case QMM_ERR_UNSUPPORTED: return "entry point off the quantized matmul path (not provided by this library)";
        default: return "unknown status";
    }
}

// gemv.hip:1337-1340
size_t qmm_wfmt_row_bytes(int fmt, int K) {
    if (K <= 0) return 0;
    const bool b32 = fmt == QMM_Q8_0_SOA || fmt == QMM_Q5_1_SOA;
    if (K % (b32 ? 32 : 256) != 0) return 0;
    switch (fmt) {
        case QMM_Q4_K: return (size_t)K / 256 * 144;
        case QMM_Q5_K: return (size_t)K / 256 * 176;
        case QMM_IQ4_XS: return (size_t)K / 256 * 136;
        case QMM_Q6_K: case QMM_Q6_K_SOA: return (size_t)K / 256 * 210;
        case QMM_Q8_0_SOA: return (size_t)K + (size_t)K / 16;
        case QMM_Q5_1_SOA: return (size_t)K / 32 * 24;
        default: return 0;
    }
}

// gemv.hip:1341-1350: GGUF Q6_K row -> [ql K/2][qh K/4][scales K/16][d (K/256)*2]
int qmm_repack_row_q6_K(const uint8_t* src, uint8_t* dst, int K) {
    if (!src || !dst) return QMM_ERR_NULL;
    if (K <= 0 || K % 256 != 0) return QMM_ERR_SHAPE;
    const size_t nb = (size_t)K / 256;
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* blk = src + b * 210;
        memcpy(dst + b * 128, blk, 128);
        memcpy(dst + nb * 128 + b * 64, blk + 128, 64);
        memcpy(dst + nb * 192 + b * 16, blk + 192, 16);
        memcpy(dst + nb * 208 + b * 2, blk + 208, 2);
    }
    return QMM_OK;
}

// gemv.hip:1351-1354: GGUF Q8_0 row {f16 d, i8 qs[32]} x K/32 -> [qs K][d (K/32) x f16]
int qmm_repack_row_q8_0(const uint8_t* src, uint8_t* dst, int K) {
    if (!src || !dst) return QMM_ERR_NULL;
    if (K <= 0 || K % 32 != 0) return QMM_ERR_SHAPE;
    for (size_t b = 0; b < (size_t)K / 32; ++b) {
        memcpy(dst + b * 32, src + b * 34 + 2, 32);
        memcpy(dst + (size_t)K + b * 2, src + b * 34, 2);
    }
    return QMM_OK;
}

// gemv.hip:1458-1465: GGUF Q5_1 row {f16 d, f16 m, u8 qh[4], u8 qs[16]} x K/32 ->
// [qs K/2][qh K/8][d (K/32) x f16][m (K/32) x f16]
int qmm_repack_row_q5_1(const uint8_t* src, uint8_t* dst, int K) {
    if (!src || !dst) return QMM_ERR_NULL;
    if (K <= 0 || K % 32 != 0) return QMM_ERR_SHAPE;
    const size_t qh = (size_t)K / 2, dd = qh + (size_t)K / 8, mm = dd + (size_t)K / 16;
    for (size_t b = 0; b < (size_t)K / 32; ++b) {
        const uint8_t* blk = src + b * 24;
        memcpy(dst + b * 16, blk + 8, 16);
        memcpy(dst + qh + b * 4, blk + 4, 4);
        memcpy(dst + dd + b * 2, blk, 2);
        memcpy(dst + mm + b * 2, blk + 2, 2);
    }
    return QMM_OK;
}

// gemv.hip:1448-1457: GGUF Q5_0 row {f16 d, u8 qh[4], u8 qs[16]} x K/32 -> the Q5_1 SoA layout with
// m = f16(-16 d): w = q d - 16 d = (q - 16) d, exactly
int qmm_repack_row_q5_0(const uint8_t* src, uint8_t* dst, int K) {
    if (!src || !dst) return QMM_ERR_NULL;
    if (K <= 0 || K % 32 != 0) return QMM_ERR_SHAPE;
    const size_t qh = (size_t)K / 2, dd = qh + (size_t)K / 8, mm = dd + (size_t)K / 16;
    for (size_t b = 0; b < (size_t)K / 32; ++b) {
        const uint8_t* blk = src + b * 22;
        uint16_t d;
        memcpy(&d, blk, 2);
        const uint16_t m = f2h_host(-16.0f * h2f_host(d));
        memcpy(dst + b * 16, blk + 6, 16);
        memcpy(dst + qh + b * 4, blk + 2, 4);
        memcpy(dst + dd + b * 2, &d, 2);
        memcpy(dst + mm + b * 2, &m, 2);
    }
    return QMM_OK;
}

}  // extern "C"

namespace {
int block_bytes_il(int fmt) {
    switch (fmt) {
        case QMM_Q4_K: return 144;
        case QMM_Q5_K: return 176;
        case QMM_IQ4_XS: return 136;
        case QMM_Q6_K_SOA: return 210;
        case QMM_Q8_0_SOA: return 272;
        default: return 0;
    }
}
}  // namespace

extern "C" {

// gemv.hip:1442-1447: groups of 8 rows, block b of row r at block index (r/8)*8*nb + b*8 + r%8
int qmm_repack_interleave8(int fmt, const uint8_t* src, uint8_t* dst, int N, int K) {
    if (!src || !dst) return QMM_ERR_NULL;
    if (fmt != QMM_Q4_K && fmt != QMM_Q5_K && fmt != QMM_IQ4_XS) return QMM_ERR_FORMAT;
    if (N <= 0 || N % 8 != 0 || K <= 0 || K % 256 != 0) return QMM_ERR_SHAPE;
    const size_t bb = (size_t)block_bytes_il(fmt), nb = (size_t)K / 256;
    for (size_t r = 0; r < (size_t)N; ++r)
        for (size_t b = 0; b < nb; ++b) memcpy(dst + ((r / 8) * 8 * nb + b * 8 + r % 8) * bb, src + (r * nb + b) * bb, bb);
    return QMM_OK;
}

// gemv.hip:1280
size_t qmm_wmma_il_bytes(int fmt, int N, int K) {
    const int bb = block_bytes_il(fmt);
    if (bb == 0 || N <= 0 || K <= 0 || K % 256 != 0) return 0;
    return (size_t)((N + 15) / 16) * (size_t)(K / 256) * 16 * (size_t)bb;
}

// gemv.hip:1281-1303: rows in groups of 16 (N padded with zero rows); per group and 256-weight block the
// 16 rows' bytes are stored piece-major, [piece][row][piece bytes]: 16-byte pieces for Q4_K and Q5_K,
// 8-byte pieces for IQ4_XS, Q6_K_SOA as [ql 8 x 16 B][qh 4 x 16 B][scales 16 B][d 2 B] per row,
// Q8_0_SOA as [q 16 x 16 B][d 16 B] per row
int qmm_repack_wmma_il(int fmt, const uint8_t* src, uint8_t* dst, int N, int K) {
    if (!src || !dst) return QMM_ERR_NULL;
    const size_t total = qmm_wmma_il_bytes(fmt, N, K);
    if (block_bytes_il(fmt) == 0) return QMM_ERR_FORMAT;
    if (total == 0) return QMM_ERR_SHAPE;
    const size_t nb = (size_t)K / 256, BB = (size_t)block_bytes_il(fmt), gb = 16 * BB;
    memset(dst, 0, total);
    for (size_t r = 0; r < (size_t)N; ++r) {
        const size_t g = r / 16, r16 = r % 16;
        uint8_t* gbase = dst + g * nb * gb;
        for (size_t b = 0; b < nb; ++b) {
            uint8_t* d = gbase + b * gb;
            if (fmt == QMM_Q4_K || fmt == QMM_Q5_K) {
                const uint8_t* blk = src + (r * nb + b) * BB;
                for (size_t i = 0; i < BB / 16; ++i) memcpy(d + i * 256 + r16 * 16, blk + i * 16, 16);
            } else if (fmt == QMM_IQ4_XS) {
                const uint8_t* blk = src + (r * nb + b) * 136;
                for (size_t i = 0; i < 17; ++i) memcpy(d + i * 128 + r16 * 8, blk + i * 8, 8);
            } else if (fmt == QMM_Q6_K_SOA) {
                const uint8_t* rp = src + r * ((size_t)K * 210 / 256);
                for (size_t i = 0; i < 8; ++i) memcpy(d + i * 256 + r16 * 16, rp + b * 128 + i * 16, 16);
                for (size_t i = 0; i < 4; ++i) memcpy(d + 2048 + i * 256 + r16 * 16, rp + nb * 128 + b * 64 + i * 16, 16);
                memcpy(d + 3072 + r16 * 16, rp + nb * 192 + b * 16, 16);
                memcpy(d + 3328 + r16 * 2, rp + nb * 208 + b * 2, 2);
            } else {                                  // Q8_0_SOA
                const uint8_t* rp = src + r * ((size_t)K + (size_t)K / 16);
                for (size_t i = 0; i < 16; ++i) memcpy(d + i * 256 + r16 * 16, rp + b * 256 + i * 16, 16);
                memcpy(d + 4096 + r16 * 16, rp + (size_t)K + b * 16, 16);
            }
        }
    }
    return QMM_OK;
}

}  // extern "C"
