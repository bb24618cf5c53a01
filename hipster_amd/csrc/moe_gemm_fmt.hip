// moe_gemm_fmt.hip -- the prefill grouped expert GEMM (qmm_moe_gemm_bf16) for the expert formats other
// than all-Q4_K, as the reference's moe_gemm takes them (engine/kernels/gemv.h:49-50,
// gemv.hip:954-969,1377-1381: Q4_K, Q5_K, Q5_1_SOA, Q8_0_SOA, the routed and the shared expert formats
// independent; IQ4_XS as well): over the device tile list of qmm_moe_sort,
//   D[k0 + r][n] = sum_k A[rowtab[k0 + r]][k] * bf16(W_e[n][k])      (f32 out, sorted row order)
// with W_e dequantised exactly (the arithmetic of qmm_dequant_bf16) and bf16 MFMA, f32 accumulation.
//
// Workgroup = (tile, 128 weight rows), 256 threads = 4 waves.  Wave w owns the block's weight rows
// 32w..32w+31 (one v_mfma_f32_32x32x16_bf16 column block) and the tile's NRB row blocks of 32.  The K
// loop steps by 32 -- one sub-block, the scale granule of every format: threads 0-127 dequantise
// their weight row's sub-block to bf16 and threads 128-255 copy the tile's 128 A rows of the step,
// both into the LDS stage that the next step's MFMAs read, while this step's MFMAs run from the
// other stage (one barrier per step); the raw bytes are loaded a step before that.  Stage rows are
// 80 bytes apart (32 bf16 + 16 bytes of padding: the 16-byte fragment reads of a half-wave's 32 rows
// spread over the banks).
#include "fmt_dequant.hpp"
#include "qmm_common.hpp"

namespace qmm {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int FBM = 128, FBN = 128, FBK = 32, FROW = 40;   // FROW: bf16 per stage row (32 + 8 of padding)
constexpr int kFStage = (FBM + FBN) * FROW;                // bf16 per stage: A rows, then weight rows

struct FArgs {
    const uint8_t* w;       // routed experts, expert e at w + e * ebytes
    const uint8_t* wsh;     // shared expert
    size_t ebytes;
    int fmt, sfmt;
    const qmm_moe_tile* tiles;
    const int* counts;      // [routed tiles, shared tiles], on the device
    int nimp;               // capacity of tiles
    const int* rowtab;      // sorted row -> A row, or null (A rows in sorted order)
    const uint16_t* A;
    float* D;
    int N, K, nb;           // nb = 128-row weight blocks
};

template <int NRB, int F>
__device__ __forceinline__ void fmt_tile(const FArgs& a, const qmm_moe_tile tl, int n0, uint16_t* st, const int* rows) {
    const int tid = threadIdx.x, lane = tid & 63, fr = lane & 31, h = lane >> 5, wave = tid >> 6;
    const uint8_t* wb = tl.expert < 0 ? a.wsh : a.w + (size_t)tl.expert * a.ebytes;
    const size_t rb = fmt_row_bytes_rt(F, a.K);
    const int nsteps = a.K / FBK;
    // step t's raw bytes (a weight row's sub-block, or 64 bytes of an A row) are loaded two steps
    // ahead of their MFMAs and decoded / stored into the LDS stage one step ahead
    const int wrow = min(n0 + tid, a.N - 1);
    const uint8_t* wrp = wb + (size_t)wrow * rb;
    const uint16_t* arow = a.A + (size_t)rows[tid & (FBM - 1)] * a.K;
    SubRaw wraw, araw;                      // araw.v[0..3]: 64 bytes of the A row
    auto load = [&](int t) {
        if (tid < FBN) {
            sub_load<F>(wrp, a.K, t, wraw);
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) araw.v[c] = ld16(arow + (size_t)t * FBK + 8 * c);
        }
    };
    auto store = [&](int t, uint16_t* stg) {
        if (tid < FBN) {                    // exact dequantisation, then RNE to bf16
            float w[32];
            sub_decode<F>(wraw, t, w);
            uint16_t* dst = stg + (FBM + tid) * FROW;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                uint32_t o[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) o[k] = f2bf_bits(w[8 * v + 2 * k]) | (f2bf_bits(w[8 * v + 2 * k + 1]) << 16);
                *(uint4*)(dst + 8 * v) = make_uint4(o[0], o[1], o[2], o[3]);
            }
        } else {
            uint16_t* dst = stg + (tid - FBN) * FROW;
#pragma unroll
            for (int c = 0; c < 4; ++c) *(uint4*)(dst + 8 * c) = araw.v[c];
        }
    };
    f32x16_t acc[NRB];
#pragma unroll
    for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
    load(0);
    store(0, st);
    if (nsteps > 1) load(1);
    lds_barrier();           // LDS-only: the prefetched global loads stay in flight across it
    for (int t = 0; t < nsteps; ++t) {
        const uint16_t* cur = st + (t & 1) * kFStage;
#pragma unroll
        for (int s = 0; s < 2; ++s) {       // two 16-wide K slices; lane: row l%32, k = 16s + 8h .. +7
            const bf16x8_t wf = *(const bf16x8_t*)(cur + (FBM + 32 * wave + fr) * FROW + 16 * s + 8 * h);
#pragma unroll
            for (int i = 0; i < NRB; ++i) {
                const bf16x8_t af = *(const bf16x8_t*)(cur + (32 * i + fr) * FROW + 16 * s + 8 * h);
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, wf, acc[i], 0, 0, 0);
            }
        }
        if (t + 1 < nsteps) {
            store(t + 1, st + ((t + 1) & 1) * kFStage);
            if (t + 2 < nsteps) load(t + 2);
        }
        lds_barrier();
    }
    // acc[i][e] = output row 32i + 8(e/4) + 4h + e%4 of the tile, weight row n0 + 32w + fr
    const int n = n0 + 32 * wave + fr;
#pragma unroll
    for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int r = 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
            if (r < tl.ncols && n < a.N) a.D[(size_t)(tl.k0 + r) * a.N + n] = acc[i][e];
        }
}

// One workgroup per (tile, weight-row block); workgroup i runs on XCD i % 8, which takes tiles x, x+8,
// ... with all their blocks (the blocks of a tile share its A rows in one L2).  One launch per
// format, as the reference launches its routed and shared tiles apart: part 0 takes the routed
// tiles [0, counts[0]), part 1 the shared ones [counts[0], counts[0] + counts[1]), part 2 both
// (one format for all).  Tiles past the device count (clamped to the capacity) exit at once.
template <int F>
__global__ void __launch_bounds__(256) k_moe_gemm_fmt(FArgs a, int part) {
    __shared__ __align__(16) uint16_t st[2 * kFStage];
    __shared__ int rows[FBM];
    const int id = blockIdx.x, sid = id >> 3;
    const int local = 8 * (sid / a.nb) + (id & 7), nbi = sid % a.nb;
    const int c0 = a.counts[0], c1 = a.counts[1];
    const int first = part == 1 ? c0 : 0, count = part == 0 ? c0 : part == 1 ? c1 : c0 + c1;
    const int tix = first + local;
    if (local >= count || tix >= a.nimp) return;
    qmm_moe_tile tl = a.tiles[tix];
    tl.ncols = max(1, min(tl.ncols, FBM));
    if (threadIdx.x < FBM) {
        const int k = tl.k0 + min((int)threadIdx.x, tl.ncols - 1);
        rows[threadIdx.x] = a.rowtab ? a.rowtab[k] : k;
    }
    __syncthreads();
    const int n0 = nbi * FBN;
    switch ((tl.ncols + 31) >> 5) {
        case 1: fmt_tile<1, F>(a, tl, n0, st, rows); break;
        case 2: fmt_tile<2, F>(a, tl, n0, st, rows); break;
        case 3: fmt_tile<3, F>(a, tl, n0, st, rows); break;
        default: fmt_tile<4, F>(a, tl, n0, st, rows); break;
    }
}

int launch_fmt_part(int fmt, const FArgs& a, int part, int grid, hipStream_t s) {
    switch (fmt) {
        case QMM_Q4_K: hipLaunchKernelGGL(k_moe_gemm_fmt<QMM_Q4_K>, dim3(grid), dim3(256), 0, s, a, part); break;
        case QMM_Q5_K: hipLaunchKernelGGL(k_moe_gemm_fmt<QMM_Q5_K>, dim3(grid), dim3(256), 0, s, a, part); break;
        case QMM_IQ4_XS: hipLaunchKernelGGL(k_moe_gemm_fmt<QMM_IQ4_XS>, dim3(grid), dim3(256), 0, s, a, part); break;
        case QMM_Q8_0_SOA: hipLaunchKernelGGL(k_moe_gemm_fmt<QMM_Q8_0_SOA>, dim3(grid), dim3(256), 0, s, a, part); break;
        default: hipLaunchKernelGGL(k_moe_gemm_fmt<QMM_Q5_1_SOA>, dim3(grid), dim3(256), 0, s, a, part); break;
    }
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

}  // namespace

// formats and K already checked by the caller (qmm_moe_gemm_bf16)
int launch_moe_gemm_fmt(int fmt, int sfmt, const void* W, const void* Wsh, size_t ebytes, const qmm_moe_tile* tiles,
                        const int* counts, int max_tiles, const int* rowtab, const uint16_t* A, float* D, int N, int K,
                        hipStream_t s) {
    FArgs a{(const uint8_t*)W, (const uint8_t*)Wsh, ebytes, fmt, sfmt, tiles, counts, max_tiles, rowtab, A, D, N, K,
            (N + FBN - 1) / FBN};
    const int grid = 8 * ((max_tiles + 7) / 8) * a.nb;
    if (fmt == sfmt) return launch_fmt_part(fmt, a, 2, grid, s);
    if (int e = launch_fmt_part(fmt, a, 0, grid, s)) return e;
    return launch_fmt_part(sfmt, a, 1, grid, s);
}

}  // namespace qmm
