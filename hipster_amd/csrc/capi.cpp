// capi.cpp -- host-only entry points of the C ABI (no kernels): version, status strings and the
// row-layout helpers of the reference (engine/kernels/gemv.hip:1337-1350).
#include <string.h>

#include "../../include/hipster_qmm.h"

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
        default: return "unknown status";
    }
}

// gemv.hip:1337-1340, for the formats this build reads
size_t qmm_wfmt_row_bytes(int fmt, int K) {
    if (K <= 0 || K % 256 != 0) return 0;
    switch (fmt) {
        case QMM_Q4_K: return (size_t)K / 256 * 144;
        case QMM_Q6_K: case QMM_Q6_K_SOA: return (size_t)K / 256 * 210;
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

}  // extern "C"
