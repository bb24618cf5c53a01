// gemv_fmt.hip -- q8-activation GEMV on gfx950 for the other weight formats of the call surface:
// Q5_K and IQ4_XS (GGUF blocks) and Q8_0_SOA / Q5_1_SOA (the engine's load-time row-SoA repacks of
// Q8_0 and Q5_1 / Q5_0 rows).  Reached through qmm_gemv_q8 / qmm_gemv_multi (gemv.hip), which is
// the reference's gemv_q8 / gemv_multi (engine/kernels/gemv.h:25,28) for these formats; the
// per-format arithmetic is the reference's (block decoders gemv.hip:90-163,214-268).
//
// RPW rows per wave (4; 2 for Q5_K).  A unit is one scale's worth of weights -- 32 (one sub-block) for IQ4_XS,
// Q8_0_SOA and Q5_1_SOA, 64 for Q5_K (the two sub-blocks sharing one 32-byte qs pair) -- and lane l
// takes units l, l + 64, ... of the row, NIT at a time, with all of a pass's weight loads issued
// before its compute.  The q8 x of a unit (32 bytes per sub-block, its d and s) is read once per
// wave and used for all of the wave's rows, from LDS (x staged once per workgroup) or from global
// memory (L1), whichever the format and width measured faster.  Per sub-block the
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
extern int g_fmt_xlds;
namespace {

constexpr int kFmtBlock = 256, kFmtWaves = kFmtBlock / 64, kFmtMaxSeg = 4;
constexpr size_t kFmtXLds = 64 * 1024;   // bytes of LDS the plain GEMV may use for staged x

// x of NCOL columns staged in LDS as [xq NCOL*K][xd NCOL*K/32][xs NCOL*K/32] (the layout of
// stage_xq8), read ahead of the weights: load() issues the thread's 16-byte pieces (element e =
// threadIdx.x + 256u, clamped to the last element, so every store is unconditional and duplicates
// write the same bytes), the weight loads follow, and operator() -- called by fmt_rows once they
// are issued -- stores the pieces (waiting for the x loads only: loads retire in issue order) and
// meets the workgroup at an LDS-only barrier.
constexpr int kXFirstU = 4;                    // pieces per thread: 16 KiB of staged x
template <int NU>
struct FmtXFirst {
    static constexpr bool active = true;
    uint4 v[NU];
    uint4* lds;
    int n;
    __device__ __forceinline__ void load(const int8_t* xq, const float* xd, const float* xs, int ncol, int K) {
        const int nq = ncol * K / 16, ns = ncol * (K / 32) / 4;
        n = nq + 2 * ns;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int e = min((int)threadIdx.x + kFmtBlock * u, n - 1);
            const void* src = e < nq ? (const void*)(xq + (size_t)e * 16)
                            : e < nq + ns ? (const void*)(xd + (size_t)(e - nq) * 4) : (const void*)(xs + (size_t)(e - nq - ns) * 4);
            v[u] = ld16(src);
        }
    }
    __device__ __forceinline__ void operator()() const {
#pragma unroll
        for (int u = 0; u < NU; ++u) lds[min((int)threadIdx.x + kFmtBlock * u, n - 1)] = v[u];
        lds_barrier();
    }
};

// Up to four weights of one format sharing x (the reference's gemv_multi / gemv_wmma segments): the
// workgroups of segment i are t0[i] .. t0[i+1]-1, each RPW rows per wave of that segment.
struct FSegs {
    const uint8_t* w[kFmtMaxSeg];
    float* y[kFmtMaxSeg];
    int N[kFmtMaxSeg];
    int t0[kFmtMaxSeg + 1];
    int nseg;
};

// XS: 0 = x read from global memory (L1) by every wave, 1 = staged in LDS before the weights are
// loaded, 2 = staged in LDS from registers loaded ahead of the first weight loads (FmtXFirst).
// The arithmetic is the same in all three, so are the results; a row's arithmetic does not depend on
// its segment or the other segments of the launch.
template <int F, int NCOL, int NIT, int RPW, int XS>
__global__ void __launch_bounds__(kFmtBlock) k_gemv_fmt(FSegs sg, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                        const float* __restrict__ xs, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    int si = 0;
#pragma unroll
    for (int i = 1; i < kFmtMaxSeg; ++i)
        if (i < sg.nseg && (int)blockIdx.x >= sg.t0[i]) si = i;
    const uint8_t* __restrict__ W = sg.w[si];
    float* __restrict__ y = sg.y[si];
    const int N = sg.N[si];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (((int)blockIdx.x - sg.t0[si]) * kFmtWaves + wave) * RPW;
    const int nsb = K / 32;
    XSrcQ8 xsrc[NCOL];
    float acc[RPW][NCOL];
    if constexpr (XS > 0) {
        const float* sd = (const float*)(smem + (size_t)NCOL * K);
#pragma unroll
        for (int c = 0; c < NCOL; ++c) xsrc[c] = XSrcQ8{(const int8_t*)smem + (size_t)c * K, sd + (size_t)c * nsb, sd + (size_t)(NCOL + c) * nsb};
    } else {
#pragma unroll
        for (int c = 0; c < NCOL; ++c) xsrc[c] = XSrcQ8{xq + (size_t)c * K, xd + (size_t)c * nsb, xs + (size_t)c * nsb};
    }
    if constexpr (XS == 2) {
        FmtXFirst<kXFirstU> st;
        st.lds = (uint4*)smem;
        st.load(xq, xd, xs, NCOL, K);
        fmt_rows<F, NCOL, NIT, RPW>(W, row0, N, K, xsrc, acc, 0, fmt_units<F>(K), 0, st);
    } else {
        if constexpr (XS == 1) stage_xq8<NCOL>(smem, xq, xd, xs, K);
        fmt_rows<F, NCOL, NIT, RPW>(W, row0, N, K, xsrc, acc, 0, fmt_units<F>(K));
    }
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

// ---- the reference's interleaved weight layouts (its gemv_q8 rpt 5, and rpt 4 with tpr 3) ----
// The format's own per-row arithmetic (fmt_rows), the loads placed by the layout's loader LD: two rows
// per wave, x from global memory, NCOL columns per launch.
template <int F, class LD, int NCOL>
__global__ void __launch_bounds__(kFmtBlock) k_gemv_il(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                       const float* __restrict__ xd, const float* __restrict__ xs,
                                                       float* __restrict__ y, int N, int K) {
    constexpr int RPW = 2, NIT = 2;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = ((int)blockIdx.x * kFmtWaves + wave) * RPW;
    const int nsb = K / 32;
    XSrcQ8 xsrc[NCOL];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) xsrc[c] = XSrcQ8{xq + (size_t)c * K, xd + (size_t)c * nsb, xs + (size_t)c * nsb};
    float acc[RPW][NCOL];
    fmt_rows<F, NCOL, NIT, RPW, XSrcQ8, FmtNoPre, LD>(W, row0, N, K, xsrc, acc, 0, fmt_units<F>(K));
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

// columns in launches of 8, then 4, then the 1..3 left
template <int F, class LD>
int launch_il(const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, hipStream_t s) {
    const dim3 grid((unsigned)((N + kFmtWaves * 2 - 1) / (kFmtWaves * 2)));
    const int nsb = K / 32;
    for (int c0 = 0; c0 < ncol;) {
        const int left = ncol - c0, nc = left >= 8 ? 8 : left >= 4 ? 4 : left;
        const uint8_t* w = (const uint8_t*)W;
        const int8_t* q = x.q + (size_t)c0 * K;
        const float *d = x.d + (size_t)c0 * nsb, *sm = x.s + (size_t)c0 * nsb;
        float* yc = y + (size_t)c0 * N;
        switch (nc) {
            case 1: hipLaunchKernelGGL((k_gemv_il<F, LD, 1>), grid, dim3(kFmtBlock), 0, s, w, q, d, sm, yc, N, K); break;
            case 2: hipLaunchKernelGGL((k_gemv_il<F, LD, 2>), grid, dim3(kFmtBlock), 0, s, w, q, d, sm, yc, N, K); break;
            case 3: hipLaunchKernelGGL((k_gemv_il<F, LD, 3>), grid, dim3(kFmtBlock), 0, s, w, q, d, sm, yc, N, K); break;
            case 4: hipLaunchKernelGGL((k_gemv_il<F, LD, 4>), grid, dim3(kFmtBlock), 0, s, w, q, d, sm, yc, N, K); break;
            default: hipLaunchKernelGGL((k_gemv_il<F, LD, 8>), grid, dim3(kFmtBlock), 0, s, w, q, d, sm, yc, N, K); break;
        }
        QMM_LAUNCH_CHECK();
        c0 += nc;
    }
    return QMM_OK;
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
int launch_fmt(const qmm_gemv_seg* segs, int nseg, qmm_xq8 x, int K, hipStream_t s) {
    // rows per wave: 2 at one column (more waves in flight), 4 above (the shared x pays more), 2 for
    // Q5_K (its units hold 20 registers of raw weights)
    constexpr int RPW = (F == QMM_Q5_K || NCOL == 1) ? 2 : 4;
    FSegs sg = {};
    sg.nseg = nseg;
    for (int i = 0; i < nseg; ++i) {
        sg.w[i] = (const uint8_t*)segs[i].w;
        sg.y[i] = segs[i].y;
        sg.N[i] = segs[i].N;
        sg.t0[i + 1] = sg.t0[i] + (segs[i].N + kFmtWaves * RPW - 1) / (kFmtWaves * RPW);
    }
    const int grid = sg.t0[nseg];
    const int per_lane = (fmt_units<F>(K) + 63) / 64;
    // Where x comes from (measured at 17408 x 5120, M = 1..8): staged once per workgroup in LDS for
    // Q5_K and Q5_1_SOA at every width (Q5_K M = 4: 30.6 -> 23.6 us, M = 8: 52.5 -> 35.2 us), for
    // IQ4_XS at 2..4 columns and Q8_0_SOA at 1..2; read from global memory otherwise (there each wave's
    // L1 reads cost less than the staging).  Staged x is loaded ahead of the weights into registers
    // when it is at most 16 KiB and the kernel is one column or a row-SoA format (M = 1: Q5_K 17.7 ->
    // 16.8 us), else copied before them.  Needs K % 128 == 0 (the float4 copy of the scales).
    constexpr bool lds_pays = F == QMM_Q5_K || F == QMM_Q5_1_SOA || (F == QMM_IQ4_XS && NCOL >= 2 && NCOL <= 4) ||
                              (F == QMM_Q8_0_SOA && NCOL <= 2);
    constexpr bool xfirst_pays = NCOL == 1 || F == QMM_Q8_0_SOA || F == QMM_Q5_1_SOA;
    const size_t xl = (size_t)NCOL * (K + K / 4);
    const int xmode = !g_fmt_xlds || !lds_pays || K % 128 != 0 || xl > kFmtXLds ? 0
                    : xfirst_pays && xl <= (size_t)kXFirstU * kFmtBlock * 16 ? 2 : 1;
#define QMM_FMTL(IV)                                                                                                     \
    do {                                                                                                                \
        if (xmode == 2) hipLaunchKernelGGL((k_gemv_fmt<F, NCOL, IV, RPW, 2>), dim3(grid), dim3(kFmtBlock), xl, s,       \
                                           sg, x.q, x.d, x.s, K);                                  \
        else if (xmode == 1) hipLaunchKernelGGL((k_gemv_fmt<F, NCOL, IV, RPW, 1>), dim3(grid), dim3(kFmtBlock), xl, s,  \
                                                sg, x.q, x.d, x.s, K);                             \
        else hipLaunchKernelGGL((k_gemv_fmt<F, NCOL, IV, RPW, 0>), dim3(grid), dim3(kFmtBlock), 0, s,                   \
                                sg, x.q, x.d, x.s, K);                                            \
    } while (0)
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
int launch_fmt_ncol(int fmt, const qmm_gemv_seg* segs, int nseg, qmm_xq8 x, int K, hipStream_t s) {
    switch (fmt) {
        case QMM_Q5_K: return launch_fmt<QMM_Q5_K, NCOL>(segs, nseg, x, K, s);
        case QMM_IQ4_XS: return launch_fmt<QMM_IQ4_XS, NCOL>(segs, nseg, x, K, s);
        case QMM_Q8_0_SOA: return launch_fmt<QMM_Q8_0_SOA, NCOL>(segs, nseg, x, K, s);
        case QMM_Q5_1_SOA: return launch_fmt<QMM_Q5_1_SOA, NCOL>(segs, nseg, x, K, s);
        default: return QMM_ERR_FORMAT;
    }
}

}  // namespace

int g_fmt_xlds = 1;

// one launch for nseg (<= 4) segments of format fmt sharing x, ncol <= 8 columns
int gemv_fmt_dispatch_segs(int fmt, const qmm_gemv_seg* segs, int nseg, qmm_xq8 x, int K, int ncol, hipStream_t s) {
    if (nseg < 1 || nseg > kFmtMaxSeg) return QMM_ERR_SHAPE;
    switch (ncol) {
        case 1: return launch_fmt_ncol<1>(fmt, segs, nseg, x, K, s);
        case 2: return launch_fmt_ncol<2>(fmt, segs, nseg, x, K, s);
        case 3: return launch_fmt_ncol<3>(fmt, segs, nseg, x, K, s);
        case 4: return launch_fmt_ncol<4>(fmt, segs, nseg, x, K, s);
        case 5: return launch_fmt_ncol<5>(fmt, segs, nseg, x, K, s);
        case 6: return launch_fmt_ncol<6>(fmt, segs, nseg, x, K, s);
        case 7: return launch_fmt_ncol<7>(fmt, segs, nseg, x, K, s);
        case 8: return launch_fmt_ncol<8>(fmt, segs, nseg, x, K, s);
        default: return QMM_ERR_SHAPE;
    }
}

int gemv_fmt_dispatch(int fmt, const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, hipStream_t s) {
    const qmm_gemv_seg seg = {fmt, W, y, N, K};
    return gemv_fmt_dispatch_segs(fmt, &seg, 1, x, K, ncol, s);
}

// rows interleaved by 8 (rows = 8: Q4_K, Q5_K, IQ4_XS) or 16 (rows = 16: also Q6_K_SOA, Q8_0_SOA); shapes
// checked by the caller (K % 256 == 0; N % 8 == 0 for 8)
int gemv_il_dispatch(int rows, int fmt, const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, hipStream_t s) {
    if (rows == 8) {
        switch (fmt) {
            case QMM_Q4_K: return launch_il<QMM_Q4_K, FmtIl8Load<QMM_Q4_K>>(W, x, y, N, K, ncol, s);
            case QMM_Q5_K: return launch_il<QMM_Q5_K, FmtIl8Load<QMM_Q5_K>>(W, x, y, N, K, ncol, s);
            case QMM_IQ4_XS: return launch_il<QMM_IQ4_XS, FmtIl8Load<QMM_IQ4_XS>>(W, x, y, N, K, ncol, s);
            default: return QMM_ERR_FORMAT;
        }
    }
    switch (fmt) {
        case QMM_Q4_K: return launch_il<QMM_Q4_K, FmtIl16Load<QMM_Q4_K>>(W, x, y, N, K, ncol, s);
        case QMM_Q5_K: return launch_il<QMM_Q5_K, FmtIl16Load<QMM_Q5_K>>(W, x, y, N, K, ncol, s);
        case QMM_IQ4_XS: return launch_il<QMM_IQ4_XS, FmtIl16Load<QMM_IQ4_XS>>(W, x, y, N, K, ncol, s);
        case QMM_Q6_K_SOA: return launch_il<QMM_Q6_K_SOA, FmtIl16Load<QMM_Q6_K_SOA>>(W, x, y, N, K, ncol, s);
        case QMM_Q8_0_SOA: return launch_il<QMM_Q8_0_SOA, FmtIl16Load<QMM_Q8_0_SOA>>(W, x, y, N, K, ncol, s);
        default: return QMM_ERR_FORMAT;
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

extern "C" int qmm_set_gemv_fmt_xlds(int on) {
    const int prev = qmm::g_fmt_xlds;
    qmm::g_fmt_xlds = on != 0;
    return prev;
}
