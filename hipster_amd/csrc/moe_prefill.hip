// moe_prefill.hip -- MoE prefill on gfx950: device-side expert sort (histogram, prefix scan, stable
// scatter, tiles), the grouped expert GEMM over the sorted rows (Q4_K experts dequantised to bf16 in
// LDS, bf16 MFMA), and silu(g)*u -> bf16.
//
// Entry points (C ABI, include/hipster_qmm.h) and what they replace in the reference:
//   qmm_moe_sort        the host path of engine/src/qwen4exp.cpp:628-645 (blocking device->host
//                       copy of the ids, std::sort by (expert, slot), tile building, three
//                       host->device copies) -- here one workgroup on the device, no host sync
//   qmm_moe_gemm_bf16   moe_gemm (engine/kernels/gemv.h:49-50, gemv.hip:909-969,1377-1381) with
//                       bf16 activations; the tile count is read on the device
//   qmm_moe_silu_bf16   moe_silu_quant (fn.hip:206-211) for the bf16 path: h = bf16(silu(g) * u)
#include "qmm_common.hpp"

#include <hip/hip_runtime.h>

namespace qmm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------------------------------------
// Expert sort.  Slots te = t*nslot + e are ordered by key = id + 1 (0 = shared expert, id -1, then
// the experts ascending), stable in te: the reference's std::sort by (expert id, te)
// (qwen4exp.cpp:631-632).  One workgroup of 16 waves; wave w owns a contiguous slot range.
// Pass 1 counts keys per wave; pass 2 turns the counts into per-(key, wave) start offsets, key-major
// then wave order; pass 3 scatters each wave's range in order, a lane's rank among equal keys of
// its 64-slot chunk coming from ballot peer masks over the key bits -- deterministic and stable.
// Tiles: per key, ceil(count / maxc) tiles of consecutive sorted positions (the reference cuts a
// tile at each expert change and every maxc positions, qwen4exp.cpp:636-641); routed-expert tiles
// first in expert order, then the shared-expert tiles.  counts = {routed tiles, shared tiles}.
constexpr int kSortThreads = 1024, kSortWaves = kSortThreads / 64, kMaxKeys = 1025;

// exclusive scan over the workgroup of one int per thread; *total gets the sum
__device__ __forceinline__ int block_exscan(int v, int* wsum, int* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(x, o, 64);
        if (lane >= o) x += u;
    }
    __syncthreads();
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    if (wave == 0) {
        int y = lane < kSortWaves ? wsum[lane] : 0;
#pragma unroll
        for (int o = 1; o < kSortWaves; o <<= 1) {
            const int u = __shfl_up(y, o, 64);
            if (lane >= o) y += u;
        }
        if (lane < kSortWaves) wsum[lane] = y;
    }
    __syncthreads();
    *total = wsum[kSortWaves - 1];
    return x - v + (wave > 0 ? wsum[wave - 1] : 0);
}

__global__ void __launch_bounds__(kSortThreads) k_moe_sort(const int* __restrict__ ids, int ns, int nslot, int nkeys, int maxc,
                                                           int* __restrict__ kpos, int* __restrict__ rowtok,
                                                           qmm_moe_tile* __restrict__ tiles, int* __restrict__ counts) {
    extern __shared__ int sm[];
    int* cnt = sm;                                   // [kSortWaves][nkeys]: per-wave counts, then running offsets
    int* tot = cnt + kSortWaves * nkeys;             // [nkeys]
    __shared__ int wsum[kSortWaves];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int i = tid; i < kSortWaves * nkeys; i += kSortThreads) cnt[i] = 0;
    __syncthreads();
    const int per = ((ns + kSortWaves - 1) / kSortWaves + 63) & ~63;
    const int lo = min(ns, wave * per), hi = min(ns, lo + per);
    // pass 1: per-wave key counts (ids outside [-1, nkeys-2] are clamped into range by the host
    // check; the kernel trusts them)
    for (int i = lo + lane; i < hi; i += 64) atomicAdd(&cnt[wave * nkeys + ids[i] + 1], 1);
    __syncthreads();
    // each thread owns a contiguous key range [k0, k1)
    const int kper = (nkeys + kSortThreads - 1) / kSortThreads;
    const int k0 = min(nkeys, tid * kper), k1 = min(nkeys, k0 + kper);
    int run = 0;
    for (int k = k0; k < k1; ++k) {
        int s = 0;
        for (int w = 0; w < kSortWaves; ++w) s += cnt[w * nkeys + k];
        tot[k] = s;
        run += s;
    }
    int total = 0;
    int base = block_exscan(run, wsum, &total);
    // pass 2: per-(key, wave) start offsets
    for (int k = k0; k < k1; ++k) {
        for (int w = 0; w < kSortWaves; ++w) {
            const int c = cnt[w * nkeys + k];
            cnt[w * nkeys + k] = base;
            base += c;
        }
    }
    __syncthreads();
    // pass 3: stable scatter, each wave over its own range in order
    const unsigned long long lt = (1ull << lane) - 1ull;
    for (int c0 = lo; c0 < hi; c0 += 64) {
        const int i = c0 + lane;
        const bool valid = i < hi;
        const int key = valid ? ids[i] + 1 : 0;
        unsigned long long peers = __ballot(valid);
        for (int b = 0; b < 11; ++b) {
            const bool bit = (key >> b) & 1;
            const unsigned long long m = __ballot(bit);
            peers &= bit ? m : ~m;
        }
        const int rank = __popcll(peers & lt);
        int pos = 0;
        if (valid) pos = cnt[wave * nkeys + key] + rank;
        __builtin_amdgcn_wave_barrier();
        if (valid) {
            kpos[i] = pos;
            rowtok[pos] = i / nslot;
            if (rank == 0) cnt[wave * nkeys + key] += __popcll(peers);
        }
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    // tiles.  After pass 3 the running offset of the last wave for key k is the end of key k's run
    // in sorted order, so start(k) = cnt[last][k] - tot[k].
    int nt = 0;
    for (int k = max(k0, 1); k < k1; ++k) nt += (tot[k] + maxc - 1) / maxc;
    int nrouted = 0;
    int tb = block_exscan(nt, wsum, &nrouted);
    for (int k = max(k0, 1); k < k1; ++k) {
        const int start = cnt[(kSortWaves - 1) * nkeys + k] - tot[k];
        for (int r = 0; r < tot[k]; r += maxc) {
            qmm_moe_tile tl;
            tl.expert = k - 1; tl.k0 = start + r; tl.ncols = min(maxc, tot[k] - r);
            tiles[tb++] = tl;
        }
    }
    if (tid == 0) {
        const int start = cnt[(kSortWaves - 1) * nkeys + 0] - tot[0];
        int n = 0;
        for (int r = 0; r < tot[0]; r += maxc) {
            qmm_moe_tile tl;
            tl.expert = -1; tl.k0 = start + r; tl.ncols = min(maxc, tot[0] - r);
            tiles[nrouted + n++] = tl;
        }
        counts[0] = nrouted;
        counts[1] = n;
    }
}

// ------------------------------------------------------------------------------------------
// Grouped expert GEMM.  Work unit = (tile, 256-row block of the expert's weight): D[k0 + r][n] =
// sum_k A[row(r)][k] * W_e[n][k] for r < ncols, row(r) = rowtab[k0 + r] (or k0 + r), W_e the expert's
// Q4_K matrix (the shared matrix when expert < 0).  Tiles hold up to 64 sorted rows: the MFMA tile
// is 64 (rows) x 256 (weight rows), K step 64; 4 waves, wave w the weight rows 64w..64w+63, 2 x 2
// MFMA tiles of 32 x 32.  LDS: two A stages (64 x 64 bf16, DMA-gathered by row) and two W stages
// (256 x 64 bf16 dequantised from registers), 80 KiB, so two workgroups share a CU and their waves
// interleave on each SIMD.  Stage layout and swizzle as in gemm.hip (chunk c of row r in slot
// r*8 + (c ^ ((r >> 1) & 7))).
constexpr int MBM = 64, MBN = 256, MBK = 64;
constexpr int kAChunks = MBM * MBK / 8, kBChunks = MBN * MBK / 8;        // 512, 2048 chunks of 16 B
constexpr size_t kMoeGemmLds = 2 * (size_t)(kAChunks + kBChunks) * 16;   // 81,920 B

__device__ __forceinline__ int swz(int r, int c) { return r * 8 + (c ^ ((r >> 1) & 7)); }

struct MoeWRaw {
    uint4 hd, q0, q1;
    __device__ __forceinline__ void load(const uint8_t* __restrict__ We, int N, int K, int n0, int k0) {
        const int n = min(n0 + (int)threadIdx.x, N - 1);
        const uint8_t* bp = We + (size_t)n * ((size_t)(K >> 8) * 144) + (size_t)(k0 >> 8) * 144;
        const int j = (k0 >> 6) & 3;
        hd = ld16(bp);
        q0 = ld16(bp + 16 + 32 * j);
        q1 = ld16(bp + 32 + 32 * j);
    }
    __device__ __forceinline__ void store(uint4* Lb, int k0) const {
        const int j = (k0 >> 6) & 3, t = threadIdx.x;
        const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
        const Q4kScaleBytes sb = q4k_scale_bytes(hd.y, hd.z, hd.w);
        const float dA = d * (float)byte8(sb.sc_lo, sb.sc_hi, 2 * j), mA = dmin * (float)byte8(sb.m_lo, sb.m_hi, 2 * j);
        const float dB = d * (float)byte8(sb.sc_lo, sb.sc_hi, 2 * j + 1), mB = dmin * (float)byte8(sb.m_lo, sb.m_hi, 2 * j + 1);
        const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const float dl = hh ? dB : dA, ml = hh ? mB : mA;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                __bf16 v[8];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const uint32_t u = (hh ? (qw[2 * c + e] >> 4) : qw[2 * c + e]) & 0x0f0f0f0fu;
#pragma unroll
                    for (int b = 0; b < 4; ++b) v[4 * e + b] = (__bf16)(dl * (float)((u >> (8 * b)) & 0xffu) - ml);
                }
                Lb[swz(t, 4 * hh + c)] = *(const uint4*)v;
            }
        }
    }
};

// A tile (64 gathered rows, k0..k0+63) -> stage La: wave w issues chunk slots (2w + i) * 64 + lane
__device__ __forceinline__ void dma_a_rows(const uint16_t* __restrict__ A, const int* rows, int K, int k0, uint4* La) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = 16 * wave + 8 * i + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
        const uint32_t off = (uint32_t)rows[r] * (uint32_t)K + (uint32_t)(k0 + 8 * c);
        __builtin_amdgcn_global_load_lds(A + off, La + (2 * wave + i) * 64, 16, 0, 0);
    }
}

__global__ void __launch_bounds__(256) k_moe_gemm_bf16(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Wsh,
                                                       size_t ebytes, const qmm_moe_tile* __restrict__ tiles,
                                                       const int* __restrict__ counts, const int* __restrict__ rowtab,
                                                       const uint16_t* __restrict__ A, float* __restrict__ D, int N, int K) {
    extern __shared__ __align__(16) uint8_t smem_raw[];
    __shared__ int rows[MBM];
    const int ntl = counts[0] + counts[1];
    const int tix = blockIdx.x;
    if (tix >= ntl) return;
    const qmm_moe_tile tl = tiles[tix];
    const int n0 = blockIdx.y * MBN;
    uint4* const As = (uint4*)smem_raw;                  // 2 stages of kAChunks
    uint4* const Bs = As + 2 * kAChunks;                 // 2 stages of kBChunks
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (threadIdx.x < MBM) {
        const int k = tl.k0 + min((int)threadIdx.x, tl.ncols - 1);
        rows[threadIdx.x] = rowtab ? rowtab[k] : k;
    }
    __syncthreads();
    const uint8_t* We = tl.expert >= 0 ? W + (size_t)tl.expert * ebytes : Wsh;
    const int nk = K / MBK, lastk = (nk - 1) * MBK;
    MoeWRaw wr;
    wr.load(We, N, K, n0, 0);
    dma_a_rows(A, rows, K, 0, As);
    wr.store(Bs, 0);
    wr.load(We, N, K, n0, min(MBK, lastk));
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jn = 0; jn < 2; ++jn)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][jn][e] = 0.f;
    const int fr = lane & 31, fc = lane >> 5, fx = (fr >> 1) & 7;
    int foa[4], fob[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        foa[ks] = fr * 8 + ((2 * ks + fc) ^ fx);
        fob[ks] = (64 * wave + fr) * 8 + ((2 * ks + fc) ^ fx);
    }
    for (int s = 0; s < nk; ++s) {
        // A tile s+1 -> the other A stage by DMA; MFMAs of tile s; W tile s+1 (registers) -> the
        // other W stage; W tile s+2 -> registers
        const uint4* La = As + (s & 1) * kAChunks;
        const uint4* Lb = Bs + (s & 1) * kBChunks;
        dma_a_rows(A, rows, K, min((s + 1) * MBK, lastk), As + ((s + 1) & 1) * kAChunks);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8 af[2], bf[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) { const uint4 v = La[foa[ks] + 256 * t]; af[t] = *(const bf16x8*)&v; }
#pragma unroll
            for (int t = 0; t < 2; ++t) { const uint4 v = Lb[fob[ks] + 256 * t]; bf[t] = *(const bf16x8*)&v; }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int jn = 0; jn < 2; ++jn) acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[jn], acc[i][jn], 0, 0, 0);
        }
        wr.store(Bs + ((s + 1) & 1) * kBChunks, min((s + 1) * MBK, lastk));
        wr.load(We, N, K, n0, min((s + 2) * MBK, lastk));
        __builtin_amdgcn_s_waitcnt(0x0F73);   // vmcnt <= 3: this step's A DMA has landed
        lds_barrier();
    }
    __builtin_amdgcn_s_waitcnt(0);
    // acc[i][jn][e] = D[k0 + 32i + 8*(e/4) + 4*(lane/32) + e%4][n0 + 64w + 32jn + lane%32]
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int r = 32 * i + 8 * (e >> 2) + 4 * fc + (e & 3);
            if (r >= tl.ncols) continue;
#pragma unroll
            for (int jn = 0; jn < 2; ++jn) {
                const int n = n0 + 64 * wave + 32 * jn + fr;
                if (n < N) D[(size_t)(tl.k0 + r) * N + n] = acc[i][jn][e];
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// h = bf16(silu(g) * u), RNE; silu(x) = x / (1 + exp(-x)) (fn.hip:8)
__global__ void __launch_bounds__(256) k_moe_silu_bf16(const float* __restrict__ g, const float* __restrict__ u,
                                                       uint16_t* __restrict__ h, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float x = g[i];
    h[i] = (uint16_t)f2bf_bits(x / (1.f + expf(-x)) * u[i]);
}

}  // namespace
}  // namespace qmm

using namespace qmm;

extern "C" {

int qmm_moe_sort(const int* ids, int T, int nslot, int nexperts, int maxc, int* kpos, int* rowtok, qmm_moe_tile* tiles,
                 int* counts, void* stream) {
    if (!ids || !kpos || !rowtok || !tiles || !counts) return QMM_ERR_NULL;
    if (T < 0 || nslot < 1 || nexperts < 1 || nexperts + 1 > kMaxKeys || maxc < 1) return QMM_ERR_SHAPE;
    const int nkeys = nexperts + 1;
    const size_t lds = (size_t)(kSortWaves + 1) * nkeys * 4;
    hipLaunchKernelGGL(k_moe_sort, dim3(1), dim3(kSortThreads), lds, (hipStream_t)stream, ids, T * nslot, nslot, nkeys, maxc, kpos,
                       rowtok, tiles, counts);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_moe_gemm_bf16(int fmt, int shared_fmt, const void* W, const void* Wsh, size_t ebytes, const qmm_moe_tile* tiles,
                      const int* counts, int max_tiles, const int* rowtab, const uint16_t* A, float* D, int N, int K,
                      void* stream) {
    if (fmt != QMM_Q4_K || shared_fmt != QMM_Q4_K) return QMM_ERR_FORMAT;
    if (!W || !Wsh || !tiles || !counts || !A || !D) return QMM_ERR_NULL;
    if (N <= 0 || K <= 0 || K % 256 != 0 || max_tiles < 0) return QMM_ERR_SHAPE;
    if (max_tiles == 0) return QMM_OK;
    const dim3 grid(max_tiles, (N + MBN - 1) / MBN);
    hipLaunchKernelGGL(k_moe_gemm_bf16, grid, dim3(256), kMoeGemmLds, (hipStream_t)stream, (const uint8_t*)W, (const uint8_t*)Wsh,
                       ebytes, tiles, counts, rowtab, A, D, N, K);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_moe_silu_bf16(const float* gate, const float* up, uint16_t* h, size_t n, void* stream) {
    if (!gate || !up || !h) return QMM_ERR_NULL;
    if (n == 0) return QMM_OK;
    hipLaunchKernelGGL(k_moe_silu_bf16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, gate, up, h, n);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

}  // extern "C"
