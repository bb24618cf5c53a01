// gemv_fmt.hip -- q8-activation GEMV on gfx950 for the other weight formats of the call surface:
// Q5_K and IQ4_XS (GGUF blocks) and Q8_0_SOA / Q5_1_SOA (the engine's load-time row-SoA repacks of
// Q8_0 and Q5_1 / Q5_0 rows).  Reached through qmm_gemv_q8 / qmm_gemv_multi (gemv.hip), which is
// the reference's gemv_q8 / gemv_multi (engine/kernels/gemv.h:25,28) for these formats; the
// per-format arithmetic is the reference's (block decoders gemv.hip:90-163,214-268).
//
// RPW rows per wave (4; 2 for Q5_K).  A unit is one scale's worth of weights -- 32 (one sub-block) for IQ4_XS,
// Q8_0_SOA and Q5_1_SOA, 64 for Q5_K (the two sub-blocks sharing one 32-byte qs pair) -- and lane l
// takes units l, l + 64, ... of the row, NIT at a time, with all of a pass's weight loads issued
// before its compute.  The q8 x of a unit (32 bytes per sub-block, its d and s) is read from
// global memory (L1) once per wave and used for all of the wave's rows.  Per sub-block the
// weights become int8 lanes of a dword, the integer dot with the q8 x uses v_dot4_i32_i8, and the
// reference's fix-up follows:
//   Q5_K    acc += (d sc) xd isum - (dmin m) xs          (q = nibble | fifth bit << 4, 0..31)
//   IQ4_XS  acc += (d (ls - 32)) xd isum                 (q = level[nibble], signed)
//   Q8_0    acc += d xd isum
//   Q5_1    acc += d xd isum + m xs                      (q = nibble | fifth bit << 4)
// A lane accumulates its units in a fixed order and the wave reduces with a fixed butterfly, so a
// column's result does not depend on ncol (T-invariant).  K % 256 == 0 for the block formats, K % 64
// (Q8_0_SOA) or K % 32 (Q5_1_SOA) for the row-SoA ones (checked by the caller).
#include "fmt_unit.hpp"
#include "qmm_common.hpp"

#include <hip/hip_runtime.h>

namespace qmm {
namespace {

constexpr int kFmtBlock = 256, kFmtWaves = kFmtBlock / 64;

template <int F, int NCOL, int NIT, int RPW>
__global__ void __launch_bounds__(kFmtBlock) k_gemv_fmt(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                        const float* __restrict__ xd, const float* __restrict__ xs,
                                                        float* __restrict__ y, int N, int K) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kFmtWaves + wave) * RPW;
    const int nsb = K / 32;
    XSrcQ8 xsrc[NCOL];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) xsrc[c] = XSrcQ8{xq + (size_t)c * K, xd + (size_t)c * nsb, xs + (size_t)c * nsb};
    float acc[RPW][NCOL];
    fmt_rows<F, NCOL, NIT, RPW>(W, row0, N, K, xsrc, acc, 0, fmt_units<F>(K));
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int c = 0; c < NCOL; ++c) acc[r][c] = wave_sum(acc[r][c]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r)
            if (row0 + r < N) {
#pragma unroll
                for (int c = 0; c < NCOL; ++c) y[(size_t)c * N + row0 + r] = acc[r][c];
            }
    }
}

// ---- MoE decode for the formats above (reference: gemv_moe, gemv.h:44, gemv.hip:1385-1394) ----
// Routed experts in format F, the shared expert in FS (F, or Q8_0_SOA as the reference allows).  A
// slot's rows are computed by fmt_rows like the plain GEMV of its expert (same per-row order, so
// the same bits as qmm_gemv_q8 on that expert), two rows per wave.
constexpr int kMoeRpw = 2, kMoeCols = 8;

template <int F, int FS, int NIT, int NC>
__device__ __forceinline__ void moe_fmt_pass(const uint8_t* wbase, bool shared, int row0, int N, int K, const int8_t* xq,
                                             const float* xd, const float* xs, const int* cols, int nc, int nexp,
                                             int xrow_te, float* __restrict__ y) {
    const int nsb = K / 32, lane = threadIdx.x & 63;
    XSrcQ8 xsrc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int sl = cols[min(c, nc - 1)];
        const size_t xr = (size_t)(xrow_te ? sl : sl / nexp);
        xsrc[c] = XSrcQ8{xq + xr * K, xd + xr * nsb, xs + xr * nsb};
    }
    float acc[kMoeRpw][NC];
    if (shared) fmt_rows<FS, NC, NIT, kMoeRpw>(wbase, row0, N, K, xsrc, acc, 0, fmt_units<FS>(K));
    else fmt_rows<F, NC, NIT, kMoeRpw>(wbase, row0, N, K, xsrc, acc, 0, fmt_units<F>(K));
#pragma unroll
    for (int r = 0; r < kMoeRpw; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = wave_sum(acc[r][c]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < kMoeRpw; ++r)
            if (row0 + r < N) {
#pragma unroll
                for (int c = 0; c < NC; ++c)
                    if (c < nc) y[(size_t)cols[c] * N + row0 + r] = acc[r][c];
            }
    }
}

// gather (gate|up): grid = (row blocks of 4 waves x 2 rows, slots, segments).
template <int F, int FS, int NIT>
__global__ void __launch_bounds__(kFmtBlock) k_gemv_moe_fmt(qmm_moe_segs a, const int* __restrict__ ids, int nexp,
                                                            const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                            const float* __restrict__ xs, int N, int K, int nslot,
                                                            int xrow_te) {
    __shared__ int s_cols[64 + kMoeCols];
    __shared__ int s_n, s_dup;
    const int te = blockIdx.y, seg = blockIdx.z;
    const int id = ids[te];
    if (threadIdx.x < 64) moe_slot_columns(ids, nslot, te, id, s_cols, &s_n, &s_dup);
    __syncthreads();
    if (s_dup) return;
    const int ncols = s_n, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kFmtWaves + wave) * kMoeRpw;
    const uint8_t* wbase = id >= 0 ? (const uint8_t*)a.w[seg] + (size_t)id * a.ebytes : (const uint8_t*)a.shared[seg];
    float* y = a.y[seg];
    for (int c0 = 0; c0 < ncols; c0 += kMoeCols) {
        const int nc = min(kMoeCols, ncols - c0);
        const int* cols = s_cols + c0;
        if (nc == 1) moe_fmt_pass<F, FS, NIT, 1>(wbase, id < 0, row0, N, K, xq, xd, xs, cols, nc, nexp, xrow_te, y);
        else if (nc == 2) moe_fmt_pass<F, FS, NIT, 2>(wbase, id < 0, row0, N, K, xq, xd, xs, cols, nc, nexp, xrow_te, y);
        else if (nc <= 4) moe_fmt_pass<F, FS, NIT, 4>(wbase, id < 0, row0, N, K, xq, xd, xs, cols, nc, nexp, xrow_te, y);
        else moe_fmt_pass<F, FS, NIT, 8>(wbase, id < 0, row0, N, K, xq, xd, xs, cols, nc, nexp, xrow_te, y);
    }
}

// down projection + weighted combine: grid = (row blocks of 2 rows, tokens); wave w takes the slots
// e = w, w + 4, ... of the token; lane r < 2 then sums row r over the slots in order (the combine of
// the Q4_K kernel, the same expression).
template <int F, int FS, int NIT>
__global__ void __launch_bounds__(kFmtBlock) k_gemv_moe_down_fmt(qmm_moe_segs a, const int* __restrict__ ids, int nexp,
                                                                 const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                                 const float* __restrict__ xs, int N, int K) {
    __shared__ float vres[kMoeMaxSlots][kMoeRpw];
    const int tok = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int row0 = blockIdx.x * kMoeRpw, nsb = K / 32;
    for (int e = wave; e < nexp; e += kFmtWaves) {
        const int id = ids[tok * nexp + e];
        const uint8_t* wbase = id >= 0 ? (const uint8_t*)a.w[0] + (size_t)id * a.ebytes : (const uint8_t*)a.shared[0];
        const size_t xr = (size_t)tok * nexp + e;
        const XSrcQ8 xsrc[1] = {XSrcQ8{xq + xr * K, xd + xr * nsb, xs + xr * nsb}};
        float acc[kMoeRpw][1];
        if (id < 0) fmt_rows<FS, 1, NIT, kMoeRpw>(wbase, row0, N, K, xsrc, acc, 0, fmt_units<FS>(K));
        else fmt_rows<F, 1, NIT, kMoeRpw>(wbase, row0, N, K, xsrc, acc, 0, fmt_units<F>(K));
#pragma unroll
        for (int r = 0; r < kMoeRpw; ++r) {
            const float v = wave_sum(acc[r][0]);
            if (lane == 0) vres[e][r] = v;
        }
    }
    __syncthreads();
    if (tid < kMoeRpw && row0 + tid < N) {
        float acc = 0.f;
        for (int e = 0; e < nexp; ++e) acc += a.slotw[tok * nexp + e] * vres[e][tid];
        a.y[0][(size_t)tok * N + row0 + tid] = acc;
    }
}

template <int F, int FS>
int launch_moe_fmt(const qmm_moe_segs& a, int nseg, const int* ids, int nexp, qmm_xq8 x, int N, int K, int T, int xrow_te,
                   hipStream_t s) {
    const int per_lane = (max(fmt_units<F>(K), fmt_units<FS>(K)) + 63) / 64;
    if (a.slotw) {
        const dim3 grid((unsigned)((N + kMoeRpw - 1) / kMoeRpw), (unsigned)T);
        if (per_lane <= 1) hipLaunchKernelGGL((k_gemv_moe_down_fmt<F, FS, 1>), grid, dim3(kFmtBlock), 0, s, a, ids, nexp, x.q, x.d, x.s, N, K);
        else hipLaunchKernelGGL((k_gemv_moe_down_fmt<F, FS, 2>), grid, dim3(kFmtBlock), 0, s, a, ids, nexp, x.q, x.d, x.s, N, K);
    } else {
        const dim3 grid((unsigned)((N + kFmtWaves * kMoeRpw - 1) / (kFmtWaves * kMoeRpw)), (unsigned)(T * nexp), (unsigned)nseg);
        if (per_lane <= 1)
            hipLaunchKernelGGL((k_gemv_moe_fmt<F, FS, 1>), grid, dim3(kFmtBlock), 0, s, a, ids, nexp, x.q, x.d, x.s, N, K, T * nexp, xrow_te);
        else
            hipLaunchKernelGGL((k_gemv_moe_fmt<F, FS, 2>), grid, dim3(kFmtBlock), 0, s, a, ids, nexp, x.q, x.d, x.s, N, K, T * nexp, xrow_te);
    }
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

template <int F, int NCOL>
int launch_fmt(const void* W, qmm_xq8 x, float* y, int N, int K, hipStream_t s) {
    // rows per wave: 2 at one column (more waves in flight), 4 above (the shared x pays more), 2 for
    // Q5_K (its units hold 20 registers of raw weights)
    constexpr int RPW = (F == QMM_Q5_K || NCOL == 1) ? 2 : 4;
    const int grid = (N + kFmtWaves * RPW - 1) / (kFmtWaves * RPW);
    const int per_lane = (fmt_units<F>(K) + 63) / 64;
#define QMM_FMTL(IV) hipLaunchKernelGGL((k_gemv_fmt<F, NCOL, IV, RPW>), dim3(grid), dim3(kFmtBlock), 0, s, (const uint8_t*)W, x.q, x.d, x.s, y, N, K)
    // units per lane and pass: all of them when they are few, else passes of two (registers: RPW
    // rows x NIT units of raw weights are live at once)
    if (per_lane <= 1) QMM_FMTL(1);
    else if (per_lane == 3 && F != QMM_Q5_K) QMM_FMTL(3);
    else QMM_FMTL(2);
#undef QMM_FMTL
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

template <int NCOL>
int launch_fmt_ncol(int fmt, const void* W, qmm_xq8 x, float* y, int N, int K, hipStream_t s) {
    switch (fmt) {
        case QMM_Q5_K: return launch_fmt<QMM_Q5_K, NCOL>(W, x, y, N, K, s);
        case QMM_IQ4_XS: return launch_fmt<QMM_IQ4_XS, NCOL>(W, x, y, N, K, s);
        case QMM_Q8_0_SOA: return launch_fmt<QMM_Q8_0_SOA, NCOL>(W, x, y, N, K, s);
        case QMM_Q5_1_SOA: return launch_fmt<QMM_Q5_1_SOA, NCOL>(W, x, y, N, K, s);
        default: return QMM_ERR_FORMAT;
    }
}

}  // namespace

int gemv_fmt_dispatch(int fmt, const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, hipStream_t s) {
    switch (ncol) {
        case 1: return launch_fmt_ncol<1>(fmt, W, x, y, N, K, s);
        case 2: return launch_fmt_ncol<2>(fmt, W, x, y, N, K, s);
        case 3: return launch_fmt_ncol<3>(fmt, W, x, y, N, K, s);
        case 4: return launch_fmt_ncol<4>(fmt, W, x, y, N, K, s);
        case 5: return launch_fmt_ncol<5>(fmt, W, x, y, N, K, s);
        case 6: return launch_fmt_ncol<6>(fmt, W, x, y, N, K, s);
        case 7: return launch_fmt_ncol<7>(fmt, W, x, y, N, K, s);
        case 8: return launch_fmt_ncol<8>(fmt, W, x, y, N, K, s);
        default: return QMM_ERR_SHAPE;
    }
}

// routed format fmt, shared format sfmt (fmt, or Q8_0_SOA); fmt may be Q4_K only with a Q8_0_SOA
// shared expert (the all-Q4_K case has its own kernels).
int moe_fmt_dispatch(int fmt, int sfmt, const qmm_moe_segs* a, int nseg, const int* ids, int nexp, qmm_xq8 x, int N, int K,
                     int T, int xrow_te, hipStream_t s) {
#define QMM_MF(F)                                                                                                    \
    case F:                                                                                                          \
        return sfmt == QMM_Q8_0_SOA ? launch_moe_fmt<F, QMM_Q8_0_SOA>(*a, nseg, ids, nexp, x, N, K, T, xrow_te, s) \
                                    : launch_moe_fmt<F, F>(*a, nseg, ids, nexp, x, N, K, T, xrow_te, s);
    if (sfmt != fmt && sfmt != QMM_Q8_0_SOA) return QMM_ERR_FORMAT;
    switch (fmt) {
        case QMM_Q4_K:
            if (sfmt != QMM_Q8_0_SOA) return QMM_ERR_FORMAT;
            return launch_moe_fmt<QMM_Q4_K, QMM_Q8_0_SOA>(*a, nseg, ids, nexp, x, N, K, T, xrow_te, s);
        QMM_MF(QMM_Q5_K)
        QMM_MF(QMM_IQ4_XS)
        QMM_MF(QMM_Q5_1_SOA)
        case QMM_Q8_0_SOA:
            return launch_moe_fmt<QMM_Q8_0_SOA, QMM_Q8_0_SOA>(*a, nseg, ids, nexp, x, N, K, T, xrow_te, s);
        default:
            return QMM_ERR_FORMAT;
    }
#undef QMM_MF
}

}  // namespace qmm
