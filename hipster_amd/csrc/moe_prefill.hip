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
//   qmm_moe_gemm_gate_up_bf16  the gate and up moe_gemm calls plus moe_silu_quant of
//                       qwen4exp.cpp:646-648 in one launch, writing h = bf16(silu(g) * u)
//   qmm_moe_silu_bf16   moe_silu_quant (fn.hip:206-211) for the bf16 path: h = bf16(silu(g) * u)
#include "qmm_common.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>

namespace qmm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------------------------------------
// Expert sort.  Slots te = t*nslot + e are ordered by key = id + 1 (0 = shared expert, id -1, then
// the experts ascending), stable in te: the reference's std::sort by (expert id, te)
// (qwen4exp.cpp:631-632).  A workgroup of 16 waves; wave w owns a contiguous slot range.  Pass 1
// counts keys per wave; pass 2 turns the counts into per-(key, wave) start offsets, key-major then
// wave order; pass 3 scatters each wave's range in order, a lane's rank among equal keys of its
// 64-slot chunk coming from ballot peer masks over the key bits -- deterministic and stable.  Large
// slot counts spread the same passes over several workgroups (k_moe_sort_count / _offsets /
// _scatter); small ones run in one (k_moe_sort).
// Tiles: per key, ceil(count / maxc) tiles of consecutive sorted positions (the reference cuts a
// tile at each expert change and every maxc positions, qwen4exp.cpp:636-641); routed-expert tiles
// first in expert order, then the shared-expert tiles.  counts = {routed tiles, shared tiles}.
constexpr int kSortThreads = 1024, kSortWaves = kSortThreads / 64, kMaxKeys = 1025, kSortBatch = 16, kSortMaxGroups = 64;

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

// Slots [lo, hi) of one workgroup are split over its 16 waves in contiguous runs of `per` (a
// multiple of 64); the same split is used by every kernel that counts or scatters them.
__device__ __forceinline__ void wave_range(int lo, int hi, int wave, int& wlo, int& whi) {
    const int per = ((hi - lo + kSortWaves - 1) / kSortWaves + 63) & ~63;
    wlo = min(hi, lo + wave * per);
    whi = min(hi, wlo + per);
}

// the sort key of an id: id + 1 (0 = the shared expert), ids outside [-1, nkeys - 2] clamped into
// that range, so a bad router output sorts wrongly but never indexes outside the count tables
__device__ __forceinline__ int sort_key(int id, int nkeys) { return min(max(id + 1, 0), nkeys - 1); }

// pass 1: key counts of the wave's slots into cnt[wave * nkeys + key] (LDS, zeroed by the caller).
// The ids are
// loaded kSortBatch per lane at a time, so the loads overlap instead of each waiting behind the
// previous LDS atomic.
__device__ __forceinline__ void sort_count(const int* __restrict__ ids, int lo, int hi, int nkeys, int* cnt) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int c0 = lo; c0 < hi; c0 += 64 * kSortBatch) {
        int kk[kSortBatch];
#pragma unroll
        for (int u = 0; u < kSortBatch; ++u) {      // unconditional (clamped) loads: no wait per load
            const int i = c0 + 64 * u + lane;
            const int v = sort_key(ids[min(i, hi - 1)], nkeys);
            kk[u] = i < hi ? v : -1;
        }
#pragma unroll
        for (int u = 0; u < kSortBatch; ++u)
            if (kk[u] >= 0) atomicAdd(&cnt[wave * nkeys + kk[u]], 1);
    }
}

// pass 3: stable scatter of the wave's slots in order; cnt[wave * nkeys + key] holds the wave's
// running offset of each key.  A lane's rank among the equal keys of its 64-slot chunk comes from
// ballot peer masks over the 11 key bits.
__device__ __forceinline__ void sort_scatter(const int* __restrict__ ids, int lo, int hi, int nkeys, int* cnt,
                                             int* __restrict__ kpos) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const unsigned long long lt = (1ull << lane) - 1ull;
    for (int b0 = lo; b0 < hi; b0 += 64 * kSortBatch) {
        int kk[kSortBatch];
#pragma unroll
        for (int u = 0; u < kSortBatch; ++u) {
            const int i = b0 + 64 * u + lane;
            const int v = sort_key(ids[min(i, hi - 1)], nkeys);
            kk[u] = i < hi ? v : 0;
        }
#pragma unroll
        for (int u = 0; u < kSortBatch; ++u) {
            const int c0 = b0 + 64 * u;
            if (c0 >= hi) break;
            const int i = c0 + lane;
            const bool valid = i < hi;
            const int key = kk[u];
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
                if (rank == 0) cnt[wave * nkeys + key] += __popcll(peers);
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
}

// tiles of the keys [k0, k1) owned by this thread, given each key's start and count (routed
// experts, keys >= 1, first in key order; then thread 0 writes the shared expert's, key 0)
__device__ __forceinline__ void sort_tiles(const int* start, const int* tot, int k0, int k1, int maxc, int* wsum,
                                           qmm_moe_tile* __restrict__ tiles, int* __restrict__ counts) {
    int nt = 0;
    for (int k = max(k0, 1); k < k1; ++k) nt += (tot[k] + maxc - 1) / maxc;
    int nrouted = 0;
    int tb = block_exscan(nt, wsum, &nrouted);
    for (int k = max(k0, 1); k < k1; ++k) {
        for (int r = 0; r < tot[k]; r += maxc) {
            qmm_moe_tile tl;
            tl.expert = k - 1; tl.k0 = start[k] + r; tl.ncols = min(maxc, tot[k] - r);
            tiles[tb++] = tl;
        }
    }
    if (threadIdx.x == 0) {
        int n = 0;
        for (int r = 0; r < tot[0]; r += maxc) {
            qmm_moe_tile tl;
            tl.expert = -1; tl.k0 = start[0] + r; tl.ncols = min(maxc, tot[0] - r);
            tiles[nrouted + n++] = tl;
        }
        counts[0] = nrouted;
        counts[1] = n;
    }
}

// Whole sort in one workgroup (small slot counts)
__global__ void __launch_bounds__(kSortThreads) k_moe_sort(const int* __restrict__ ids, int ns, int nslot, int nkeys, int maxc,
                                                           int* __restrict__ kpos, qmm_moe_tile* __restrict__ tiles,
                                                           int* __restrict__ counts) {
    extern __shared__ int sm[];
    int* cnt = sm;                                   // [kSortWaves][nkeys]: per-wave counts, then running offsets
    int* tot = cnt + kSortWaves * nkeys;             // [nkeys]
    int* start = tot + nkeys;                        // [nkeys]
    __shared__ int wsum[kSortWaves];
    const int tid = threadIdx.x, wave = tid >> 6;
    for (int i = tid; i < kSortWaves * nkeys; i += kSortThreads) cnt[i] = 0;
    __syncthreads();
    int lo, hi;
    wave_range(0, ns, wave, lo, hi);
    sort_count(ids, lo, hi, nkeys, cnt);
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
        start[k] = base;
        for (int w = 0; w < kSortWaves; ++w) {
            const int c = cnt[w * nkeys + k];
            cnt[w * nkeys + k] = base;
            base += c;
        }
    }
    __syncthreads();
    sort_scatter(ids, lo, hi, nkeys, cnt, kpos);
    sort_tiles(start, tot, k0, k1, maxc, wsum, tiles, counts);
}

// The same sort over G workgroups (large slot counts), in two launches: each workgroup counts the
// keys of its contiguous slot range into hist[g][key] (global scratch); then each workgroup counts
// its range again per wave, derives its start per (key, wave) from the whole table (keys before,
// then the same key in earlier workgroups and waves) and scatters; workgroup 0 also writes the
// tiles.  The order is the one-workgroup order: key, then workgroup, then wave, then slot -- i.e.
// key, then slot.
__global__ void __launch_bounds__(kSortThreads) k_moe_sort_count(const int* __restrict__ ids, int ns, int nkeys, int per,
                                                                 int* __restrict__ hist) {
    extern __shared__ int sm[];
    const int tid = threadIdx.x, wave = tid >> 6;
    for (int i = tid; i < kSortWaves * nkeys; i += kSortThreads) sm[i] = 0;
    __syncthreads();
    const int glo = min(ns, (int)blockIdx.x * per), ghi = min(ns, glo + per);
    int lo, hi;
    wave_range(glo, ghi, wave, lo, hi);
    sort_count(ids, lo, hi, nkeys, sm);
    __syncthreads();
    for (int k = tid; k < nkeys; k += kSortThreads) {
        int s = 0;
        for (int w = 0; w < kSortWaves; ++w) s += sm[w * nkeys + k];
        hist[(size_t)blockIdx.x * nkeys + k] = s;
    }
}

__global__ void __launch_bounds__(kSortThreads) k_moe_sort_scatter(const int* __restrict__ ids, int ns, int nkeys, int per, int G,
                                                                   int maxc, const int* __restrict__ hist, int* __restrict__ kpos,
                                                                   qmm_moe_tile* __restrict__ tiles, int* __restrict__ counts) {
    extern __shared__ int sm[];
    int* cnt = sm;                                   // [kSortWaves][nkeys]
    int* tot = cnt + kSortWaves * nkeys;             // [nkeys]
    int* start = tot + nkeys;                        // [nkeys]
    __shared__ int wsum[kSortWaves];
    const int tid = threadIdx.x, wave = tid >> 6, g = blockIdx.x;
    for (int i = tid; i < kSortWaves * nkeys; i += kSortThreads) cnt[i] = 0;
    __syncthreads();
    const int glo = min(ns, g * per), ghi = min(ns, glo + per);
    int lo, hi;
    wave_range(glo, ghi, wave, lo, hi);
    sort_count(ids, lo, hi, nkeys, cnt);
    // this workgroup's start per key: the keys before it, then the same key in earlier workgroups
    const int kper = (nkeys + kSortThreads - 1) / kSortThreads;
    const int k0 = min(nkeys, tid * kper), k1 = min(nkeys, k0 + kper);
    int run = 0;
    for (int k = k0; k < k1; ++k) {
        int s = 0, before = 0;
        for (int gg = 0; gg < G; ++gg) {
            const int c = hist[(size_t)gg * nkeys + k];
            before += gg < g ? c : 0;
            s += c;
        }
        tot[k] = s;
        start[k] = before;                           // offset within the key for now
        run += s;
    }
    int total = 0;
    int base = block_exscan(run, wsum, &total);      // also orders the count pass before the reads below
    for (int k = k0; k < k1; ++k) {
        int r = base + start[k];
        start[k] = base;
        base += tot[k];
        for (int w = 0; w < kSortWaves; ++w) {
            const int c = cnt[w * nkeys + k];
            cnt[w * nkeys + k] = r;
            r += c;
        }
    }
    __syncthreads();
    sort_scatter(ids, lo, hi, nkeys, cnt, kpos);
    if (g == 0) sort_tiles(start, tot, k0, k1, maxc, wsum, tiles, counts);
}

// rowtok[kpos[i]] = token of slot i: the inverse permutation, written by the whole grid (scattered
// 4-byte stores issued from the one sorting workgroup would all queue on a single CU)
__global__ void __launch_bounds__(256) k_moe_rowtok(const int* __restrict__ kpos, int* __restrict__ rowtok, int ns, int nslot) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < ns && (unsigned)kpos[i] < (unsigned)ns) rowtok[kpos[i]] = i / nslot;
}

// ------------------------------------------------------------------------------------------
// Grouped expert GEMM.  Work unit = (tile, block of the expert's weight rows).  A tile holds up to
// 128 sorted rows: D[k0 + r][n] = sum_k A[row(r)][k] * W_e[n][k] for r < ncols, row(r) =
// rowtab[k0 + r] (or k0 + r), W_e the expert's Q4_K matrix (the shared matrix when expert < 0).
//
// 512 threads = 8 waves, two per SIMD, side by side along the weight rows: wave w owns one 32-wide
// MFMA column block (256 weight rows per workgroup) and all NRB = ceil(ncols / 32) row blocks of
// the tile, so every weight is dequantised once per workgroup, by the wave that multiplies it,
// straight into MFMA operand registers; the two waves of a SIMD hide each other's waits.
// v_mfma_f32_32x32x16_bf16 takes from lane l weight row l%32 and k = 8(l/32)..+7 of a 16-wide K
// slice; for a 64-wide K step (one qs pair j of a block) these are the low nibbles of qs bytes
// 8h..8h+7 (slice 0) and 16+8h..16+8h+7 (slice 1) and the high nibbles of the same bytes (slices
// 2, 3), h = l/32.  A (gathered bf16 rows, DMA issued by waves 0-3) streams global -> LDS with
// global_load_lds_dwordx4 through a ring of XST = 5 stages issued four steps ahead; the weight rows'
// Q4_K blocks (144 contiguous bytes per row, so one DMA instruction covers about 7 rows: coalesced)
// stream through a ring of block stages, DMA issued by waves 4-7: two stages (one block of 4 K steps
// ahead) for tiles of 65-128 rows, three (two blocks ahead) for tiles of at most 64 rows, whose
// smaller A stages leave the room.  A tile of few rows spends little time per step, so one block in
// flight per CU would bound its weight stream at about 37 KB per memory latency.
// The raw bytes of step t+1 are dequantised while the MFMAs of step t run.  A stage: 32 NRB rows x 8
// chunks of 16 B, chunk c of row r in slot r*8 + (c ^ ((r >> 1) & 7)) (conflict-free fragment
// reads); block stage: 256 rows x 144 B, row-major.  The A ring comes first in LDS, then the weight
// ring.
// Gate/up mode: the 256 weight rows of a workgroup are 128 gate rows (waves 0-3) and the same 128
// up rows (waves 4-7); the up waves hand their results over through LDS and the gate waves write
// h = bf16(silu(g) * u).
constexpr int XBM = 128, XBW = 256, XBK = 64, XST = 5, XTHREADS = 512;
constexpr int kXA = XBM * XBK / 8;                          // 16-byte chunks per A stage (1024)
constexpr int kXW = 9 * XBW;                                // chunks per weight block stage (2304)
constexpr size_t kXLds = ((size_t)XST * kXA + 2 * (size_t)kXW) * 16;   // 155,648 B
// ring geometry for tiles of NRB row blocks: chunks per A stage, weight block stages
template <int NRB>
struct XRing {
    static constexpr int kA = 256 * NRB;
    static constexpr int WST = NRB <= 2 ? 3 : 2;
    static_assert(((size_t)XST * kA + (size_t)WST * kXW) * 16 <= kXLds, "ring exceeds the launch's LDS");
};

// s_waitcnt immediate for "vmcnt <= v" (expcnt, lgkmcnt unconstrained)
constexpr int vmcnt_imm(int v) { return (v & 15) | (7 << 4) | (15 << 8) | ((v >> 4) << 14); }

// wait until at most `rem` steps of L loads each are outstanding (rem = 0, 1 or 2)
template <int L>
__device__ __forceinline__ void wait_steps(int rem) {
    if (rem >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * L));
    else if (rem == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(L));
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
}

struct XArgs {
    const uint8_t* w0;     // expert matrices (gate in gate/up mode), expert e at w0 + e * ebytes
    const uint8_t* w0sh;   // shared-expert matrix
    const uint8_t* w1;     // up experts (gate/up mode only)
    const uint8_t* w1sh;
    size_t ebytes;
    const qmm_moe_tile* tiles;
    const int* counts;
    const int* rowtab;
    const uint16_t* A;
    void* D;               // f32 [k][ldd], or bf16 h [k][ldd] in gate/up mode
    int N, K, nb;          // nb = weight-row blocks per tile
    int ldd;               // row stride of D (elements)
    int trows, nimp, M;    // tiles == nullptr: implicit tiles of trows rows of expert 0, nimp of them, M rows;
                           // otherwise nimp = capacity of tiles (the device count is clamped to it)
    int bpu;               // k_moe_gemm_as: 256-row weight blocks per work unit
};

// scales of K step j (qs pair j: sub-blocks 2j, 2j+1) of a Q4_K block header, pre-scaled for
// q4_bf16x8_mix: {d*sc[2j] * 2^24, dmin*m[2j], d*sc[2j+1] * 2^20, dmin*m[2j+1]}
struct StepScl { float sa, ma, sb, mb; };
__device__ __forceinline__ StepScl q4k_step_scales(const uint4 hd, int j) {
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    const Q4kScaleBytes sb = q4k_scale_bytes(hd.y, hd.z, hd.w);
    StepScl c;
    c.sa = d * (float)byte8(sb.sc_lo, sb.sc_hi, 2 * j) * 16777216.f;
    c.ma = dmin * (float)byte8(sb.m_lo, sb.m_hi, 2 * j);
    c.sb = d * (float)byte8(sb.sc_lo, sb.sc_hi, 2 * j + 1) * 1048576.f;
    c.mb = dmin * (float)byte8(sb.m_lo, sb.m_hi, 2 * j + 1);
    return c;
}

template <bool GU, int NRB>
__device__ __forceinline__ void moe_gemm_tile(const XArgs& a, const qmm_moe_tile tl, int n0, uint4* As, const int* rows) {
    constexpr int kA = XRing<NRB>::kA, WST = XRing<NRB>::WST;
    uint4* const Ws = As + XST * kA;
    const int lane = threadIdx.x & 63, fr = lane & 31, h = lane >> 5, fx = (fr >> 1) & 7;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), team = wave >> 2, wq = wave & 3;
    const int K = a.K, N = a.N, nk = K / XBK, nblk = K >> 8;
    const uint32_t rowbytes = (uint32_t)(K >> 8) * 144u;
    const uint8_t* w0 = tl.expert >= 0 ? a.w0 + (size_t)tl.expert * a.ebytes : a.w0sh;
    const uint8_t* w1 = GU ? (tl.expert >= 0 ? a.w1 + (size_t)tl.expert * a.ebytes : a.w1sh) : w0;
    const uint32_t lA = lds_addr(As), lW = lds_addr(Ws);
    // A DMA (waves 0-3): instruction q of wave wq fills slots (wq + 4q) * 64 + lane = row block q
    uint32_t aoff[NRB];
#pragma unroll
    for (int q = 0; q < NRB; ++q) {
        const int r = 8 * (wq + 4 * q) + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
        aoff[q] = ((uint32_t)rows[r] * (uint32_t)K + (uint32_t)(8 * c)) * 2u;
    }
    // weight DMA (waves 4-7), one Q4_K block (144 B) of each of the 256 weight rows per 4 K steps:
    // instruction k = 9 wq + q (0..35) fills chunks 64k + lane = row (64k + lane) / 9, 16-byte part
    // (64k + lane) % 9.  In gate/up mode instructions 0-17 are exactly the 128 gate rows.
    uint32_t woff[9];
#pragma unroll
    for (int q = 0; q < 9; ++q) {
        const int k = 9 * wq + q, p = 64 * k + lane, row = p / 9, part = p - 9 * row;
        woff[q] = (uint32_t)min(n0 + (GU ? (row & 127) : row), N - 1) * rowbytes + (uint32_t)(16 * part);
    }
    auto issue = [&](int p, int st) {       // A of step p (waves 0-3)
        if (team == 0) {
            const uint8_t* abase = (const uint8_t*)a.A + (size_t)p * (XBK * 2);
            const uint32_t la = lA + (uint32_t)(st * kA * 16);
#pragma unroll
            for (int q = 0; q < NRB; ++q) dma16s(abase, aoff[q], la + (uint32_t)((wq + 4 * q) * 1024));
        }
    };
    auto issue_w = [&](int b) {             // weight block b into block stage b % WST (waves 4-7)
        if (team == 1) {
            const uint32_t lw = lW + (uint32_t)((b % WST) * kXW * 16);
#pragma unroll
            for (int q = 0; q < 9; ++q) {
                const int k = 9 * wq + q;
                dma16s((GU && k >= 18 ? w1 : w0) + b * 144, woff[q], lw + (uint32_t)(k * 1024));
            }
        }
    };
    // the lane's weight row (column slot of the stage) for its MFMA column block
    const int c0 = GU ? 128 * team + 32 * wq + fr : 32 * wave + fr;
    f32x16 acc[NRB];
#pragma unroll
    for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
    // A fragments of K slice s (16 wide) of the stage at la, row blocks 0..NRB-1
    auto afrag = [&](const uint4* la, int s, bf16x8 (&af)[NRB]) {
#pragma unroll
        for (int i = 0; i < NRB; ++i) {
            const uint4 v = la[(32 * i + fr) * 8 + ((2 * s + h) ^ fx)];
            af[i] = *(const bf16x8*)&v;
        }
    };
    // raw weight bytes of one step for the lane's weight row, and their decode
    struct Raw { uint4 hd; uint2 q0, q1; };
    auto rawread = [&](int p, Raw& r) {     // step p: block p / 4, qs pair p % 4
        const uint8_t* rp = (const uint8_t*)(Ws + ((p >> 2) % WST) * kXW) + c0 * 144;
        const int j = p & 3;
        r.hd = *(const uint4*)rp;
        r.q0 = *(const uint2*)(rp + 16 + 32 * j + 8 * h);
        r.q1 = *(const uint2*)(rp + 32 + 32 * j + 8 * h);
    };
    // K slice s (16 wide) of the step: s 0, 1 = low nibbles of the two qs halves (sub-block 2j),
    // s 2, 3 = their high nibbles (sub-block 2j+1)
    auto deq = [&](const Raw& r, const StepScl& c, int s) {
        const uint2 q = (s & 1) ? r.q1 : r.q0;
        return s < 2 ? q4_bf16x8_mix(q.x, q.y, 0x000f000fu, c.sa, -c.ma) : q4_bf16x8_mix(q.x, q.y, 0x00f000f0u, c.sb, -c.mb);
    };
    // before dequantising step p (waves 4-7 hold at most WST - 1 blocks in flight: block b + WST - 1
    // is issued at the first step of block b, after this wait, into the stage block b - 1 used)
    auto wait_rem = [&](int rem, int p) {
        if (team == 0) wait_steps<NRB>(rem);
        else if ((p & 3) == 0) {
            if (WST == 3 && (p >> 2) + 1 < nblk) __builtin_amdgcn_s_waitcnt(vmcnt_imm(9));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
    };
    // prologue (K % 256 == 0, so nk >= 4): A steps 0..3 and weight blocks 0 (and 1) in flight, wait
    // for A steps 0, 1 and block 0
    issue(0, 0);
    issue(1, 1);
    issue(2, 2);
    issue(3, 3);
    issue_w(0);
    if (WST == 3 && nblk > 1) issue_w(1);
    wait_rem(2, 0);
    lds_barrier();
    bf16x8 wa[4], wb[4], af0[NRB];
    {
        Raw r;
        rawread(0, r);
        const StepScl c = q4k_step_scales(r.hd, 0);
#pragma unroll
        for (int s = 0; s < 4; ++s) wa[s] = deq(r, c, s);
        afrag(As, 0, af0);
    }
    // Step t (t < nk-1): wait for step t+1's loads and barrier (t > 0); issue step t+4 into the
    // stage step t-1 used; then 4 chunks (K slice s), each the NRB MFMAs of step t for slice s and
    // the dequantisation of slice s of step t+1, fenced so that the MFMAs have VALU work of the same
    // wave to overlap with.  A fragments are read one slice ahead, slice 0 of step t+1 during step t.
    auto step = [&](int t, int st, int st1, int st4, const bf16x8 (&cur)[4], bf16x8 (&nxt)[4]) {
        if (t > 0) {
            wait_rem(min(nk - 1, t + 3) - (t + 1), t + 1);
            lds_barrier();
        }
        __builtin_amdgcn_sched_barrier(0);
        const uint4* la = As + st * kA;
        Raw r;
        rawread(t + 1, r);
        StepScl c;
        bf16x8 af[NRB], afn[NRB];
#pragma unroll
        for (int i = 0; i < NRB; ++i) af[i] = af0[i];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s == 1) {       // DMA for step t+4 (its stage was last read in step t-1) after chunk 0's MFMAs
                if (t + 4 < nk) issue(t + 4, st4);
                if ((t & 3) == 0 && (t >> 2) + WST - 1 < nblk) issue_w((t >> 2) + WST - 1);
                __builtin_amdgcn_sched_barrier(0);
            }
            afrag(s < 3 ? la : As + st1 * kA, s < 3 ? s + 1 : 0, afn);
            if (s == 0) c = q4k_step_scales(r.hd, (t + 1) & 3);
            nxt[s] = deq(r, c, s);
            asm volatile("" : : "v"(nxt[s]));   // keeps the dequantisation inside this chunk
#pragma unroll
            for (int i = 0; i < NRB; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], cur[s], acc[i], 0, 0, 0);
            if (s == 0) {
#pragma unroll
                for (int k = 0; k < NRB; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 44 / NRB + 1, 0);
                }
            } else {
#pragma unroll
                for (int k = 0; k < NRB; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 24 / NRB + 1, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < NRB; ++i) af[i] = afn[i];
        }
#pragma unroll
        for (int i = 0; i < NRB; ++i) af0[i] = af[i];
    };
    int st = 0;
    for (int t = 0; t < nk - 2; t += 2) {     // nk is a multiple of 4
        const int s1 = st == XST - 1 ? 0 : st + 1, s2 = s1 == XST - 1 ? 0 : s1 + 1;
        const int s3 = s2 == XST - 1 ? 0 : s2 + 1, s4 = s3 == XST - 1 ? 0 : s3 + 1, s5 = s4 == XST - 1 ? 0 : s4 + 1;
        step(t, st, s1, s4, wa, wb);
        step(t + 1, s1, s2, s5, wb, wa);
        st = s2;
    }
    {   // steps nk-2 and nk-1
        const int s1 = st == XST - 1 ? 0 : st + 1;
        step(nk - 2, st, s1, 0, wa, wb);
        const uint4* la = As + s1 * kA;
        bf16x8 af[NRB];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s == 0) {
#pragma unroll
                for (int i = 0; i < NRB; ++i) af[i] = af0[i];
            } else {
                afrag(la, s, af);
            }
#pragma unroll
            for (int i = 0; i < NRB; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], wb[s], acc[i], 0, 0, 0);
        }
    }
    // acc[i][e] = output row 32i + 8(e/4) + 4h + e%4 of the tile, weight row n0 + (column block) + fr
    if constexpr (GU) {
        // up waves (4-7) hand their accumulators to the gate waves of the same SIMD through LDS
        float* xch = (float*)As;                        // ring no longer needed: 4 x NRB x 16 x 64 floats
        lds_barrier();
        if (team == 1) {
#pragma unroll
            for (int i = 0; i < NRB; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) xch[((wq * NRB + i) * 16 + e) * 64 + lane] = acc[i][e];
        }
        lds_barrier();
        if (team == 0) {
            uint16_t* H = (uint16_t*)a.D;
            const int n = n0 + 32 * wq + fr;
#pragma unroll
            for (int i = 0; i < NRB; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int r = 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
                    if (r >= tl.ncols || n >= N) continue;
                    const float g = acc[i][e], u = xch[((wq * NRB + i) * 16 + e) * 64 + lane];
                    H[(size_t)(tl.k0 + r) * a.ldd + n] = (uint16_t)f2bf_bits(g / (1.f + __expf(-g)) * u);
                }
        }
    } else {
        float* D = (float*)a.D;
        const int n = n0 + 32 * wave + fr;
#pragma unroll
        for (int i = 0; i < NRB; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int r = 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
                if (r < tl.ncols && n < N) D[(size_t)(tl.k0 + r) * a.ldd + n] = acc[i][e];
            }
    }
}

// One workgroup per (tile, weight-row block).  Workgroup id i runs on XCD i % 8; XCD x takes tiles
// x, x+8, x+16, ... with all their row blocks, so the blocks of one tile share its A rows in one L2.
template <bool GU>
__global__ void __launch_bounds__(XTHREADS) k_moe_gemm_x(XArgs a) {
    extern __shared__ __align__(16) uint8_t smem_raw[];
    __shared__ int rows[XBM];
    const int id = blockIdx.x, sid = id >> 3;
    const int tix = 8 * (sid / a.nb) + (id & 7), nbi = sid % a.nb;
    if (tix >= (a.tiles ? min(a.counts[0] + a.counts[1], a.nimp) : a.nimp)) return;
    qmm_moe_tile tl;
    if (a.tiles) tl = a.tiles[tix];
    else tl = qmm_moe_tile{0, tix * a.trows, min(a.trows, a.M - tix * a.trows)};
    tl.ncols = max(1, min(tl.ncols, XBM));
    if (threadIdx.x < XBM) {
        const int k = tl.k0 + min((int)threadIdx.x, tl.ncols - 1);
        rows[threadIdx.x] = a.rowtab ? a.rowtab[k] : k;
    }
    __syncthreads();
    uint4* const As = (uint4*)smem_raw;
    const int n0 = nbi * (GU ? XBW / 2 : XBW);
    switch ((tl.ncols + 31) >> 5) {
        case 1: moe_gemm_tile<GU, 1>(a, tl, n0, As, rows); break;
        case 2: moe_gemm_tile<GU, 2>(a, tl, n0, As, rows); break;
        case 3: moe_gemm_tile<GU, 3>(a, tl, n0, As, rows); break;
        default: moe_gemm_tile<GU, 4>(a, tl, n0, As, rows); break;
    }
}

int launch_moe_gemm_x(bool gu, const XArgs& a, int max_tiles, hipStream_t s) {
    const int grid = 8 * ((max_tiles + 7) / 8) * a.nb;
    if (gu) hipLaunchKernelGGL(k_moe_gemm_x<true>, dim3(grid), dim3(XTHREADS), kXLds, s, a);
    else hipLaunchKernelGGL(k_moe_gemm_x<false>, dim3(grid), dim3(XTHREADS), kXLds, s, a);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

// ------------------------------------------------------------------------------------------
// Grouped expert GEMM with the tile's activations resident in LDS, for K = 512 (the MoE down
// projection).  Work unit = (tile, run of bpu consecutive 256-row weight blocks).  The tile's A rows
// (at most 128 x 512 bf16 = 128 KiB) are copied global -> LDS once per unit; after that every wave
// works alone: it streams its own 32 weight rows of each block straight into registers, dequantises
// them and multiplies them against A fragments read from LDS, block after block, and stores each
// block's f32 results.  The main loop has no workgroup barrier and no LDS writes, and A is read from
// global memory once per unit instead of once per weight block.
// The K order is k_moe_gemm_x's (same MFMA sequence, so the same results bit for bit): per 64-wide
// K step lane l (weight row l%32, h = l/32) takes qs bytes 8h..8h+7 and 16+8h..16+8h+7 of the step's
// pair, slices 0 and 1 their low nibbles, slices 2 and 3 their high nibbles, and the A fragment of
// slice s is chunk 2s + h of the step.  A in LDS: row r at r * 1040 bytes
// (64 chunks of 16 B and 16 B of padding), so the 16 rows a quarter-wave reads fall in 16 distinct
// bank groups and every fragment address is one lane base plus a constant; one DMA instruction
// copies one row.
constexpr int kAsK = 512, kAsThreads = 512, kAsBlocksPerUnit = 4, kAsRowBytes = 1040;
constexpr bool kAsDeferStores = false;

// f32 store the compiler does not see (address = wave-uniform base in SGPRs + per-lane 32-bit byte
// offset): its waits for the weight loads issued before it are then computed over loads only (loads
// complete in order, so such a wait can only last longer), instead of the full vmcnt(0) it places
// once loads and stores are both outstanding.  Unlike the DMA helpers it carries no s_nop guard (64
// stores per weight block): its base is only ever advanced by scalar adds, never reloaded by a VALU
// instruction, which tests/test_asm_hazards.py checks on the compiled code.
__device__ __forceinline__ void st_f32_nc(const uint8_t* base, uint32_t voff, float v) {
    asm volatile("global_store_dword %0, %1, %2" : : "v"(voff), "v"(v), "s"(base) : "memory");
}

// one Q4_K block (4 K steps) of the lane's weight row: header and the lane's two 8-byte qs pieces
// per step j (bytes 8h.. and 16+8h.. of pair j)
struct AsRaw { uint4 hd; uint2 a0, b0, a1, b1, a2, b2, a3, b3; };

template <int NRB>
__device__ __forceinline__ void moe_as_unit(const XArgs& a, const qmm_moe_tile tl, int b0, int b1, const int* rows,
                                            uint8_t* As) {
    const int lane = threadIdx.x & 63, fr = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr uint32_t rowbytes = 2 * 144u;          // two Q4_K blocks per weight row
    const int N = a.N;
    const uint8_t* w = tl.expert >= 0 ? a.w0 + (size_t)tl.expert * a.ebytes : a.w0sh;
    {   // A rows 0 .. 32 NRB - 1 -> LDS, one DMA instruction (64 lanes x 16 B) per row
        const uint32_t la = lds_addr(As);
        for (int r = wave; r < NRB * 32; r += 8)
            dma16((const uint8_t*)a.A + ((size_t)rows[r] * kAsK + (size_t)(8 * lane)) * 2, la + (uint32_t)(r * kAsRowBytes));
    }
    // group g = Q4_K block g % 2 of weight block b0 + g / 2; the lane's row in it (clamped: rows past
    // N load row N-1 and are not stored)
    const int nblk = b1 - b0, ng = 2 * nblk;
    auto load = [&](int g, AsRaw& r) {
        const int b = b0 + (g >> 1);
        const uint8_t* p = w + (size_t)min(b * 256 + 32 * wave + fr, N - 1) * rowbytes + (size_t)(g & 1) * 144;
        const uint8_t* pq = p + 16 + 8 * h;
        r.hd = ld16(p);
        r.a0 = *(const uint2*)(pq);
        r.b0 = *(const uint2*)(pq + 16);
        r.a1 = *(const uint2*)(pq + 32);
        r.b1 = *(const uint2*)(pq + 48);
        r.a2 = *(const uint2*)(pq + 64);
        r.b2 = *(const uint2*)(pq + 80);
        r.a3 = *(const uint2*)(pq + 96);
        r.b3 = *(const uint2*)(pq + 112);
    };
    f32x16 acc0[NRB], acc1[NRB];
#pragma unroll
    for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc0[i][e] = acc1[i][e] = 0.f;
    AsRaw ra, rb;
    load(0, ra);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));      // the A copy has landed (and group 0)
    __syncthreads();
    // lane bases: row fr (row blocks 0, 1) and row 64 + fr (row blocks 2, 3), chunk h
    typedef __attribute__((address_space(3))) const uint8_t lds_u8;
    const lds_u8* alo = (const lds_u8*)As + fr * kAsRowBytes + 16 * h;
    const lds_u8* ahi = alo + 64 * kAsRowBytes;
    asm volatile("" : "+v"(ahi));     // a base of its own: otherwise folded into alo + offsets past 64 KiB

    // K step t (0..7) of the row; the four slices' NRB MFMAs each
    auto step = [&](const uint2 qa, const uint2 qb, const StepScl& c, int t, f32x16 (&acc)[NRB]) {
        bf16x8 wv[4];
        wv[0] = q4_bf16x8_mix(qa.x, qa.y, 0x000f000fu, c.sa, -c.ma);
        wv[1] = q4_bf16x8_mix(qb.x, qb.y, 0x000f000fu, c.sa, -c.ma);
        wv[2] = q4_bf16x8_mix(qa.x, qa.y, 0x00f000f0u, c.sb, -c.mb);
        wv[3] = q4_bf16x8_mix(qb.x, qb.y, 0x00f000f0u, c.sb, -c.mb);
        // A fragments one slice ahead, each slice fenced: two slices' fragments live at most
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        u32x4 af[NRB], an[NRB];
        auto rd = [&](u32x4 (&v)[NRB], int s) {
            const int off = (8 * t + 2 * s) * 16;
#pragma unroll
            for (int i = 0; i < NRB; ++i)
                v[i] = *(const __attribute__((address_space(3))) u32x4*)((i < 2 ? alo : ahi) + (i & 1) * 32 * kAsRowBytes + off);
        };
        rd(af, 0);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s < 3) rd(an, s + 1);
#pragma unroll
            for (int i = 0; i < NRB; ++i)
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[i]), wv[s], acc[i], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < NRB; ++i) af[i] = an[i];
        }
    };
    // results of weight block b (tile row 32i + 8(e/4) + e%4 + 4h): the uniform row part walks a
    // scalar pointer (kept opaque, so its 64 values are formed one at a time instead of hoisted out of
    // the loop), the lane part (4h rows, column n) is a fixed byte offset; then the set restarts at 0
    auto store = [&](f32x16 (&acc)[NRB], int b) {
        const int n = b * 256 + 32 * wave + fr;
        const uint32_t voff = (uint32_t)(4 * h * a.ldd + n) * 4u;
        int rem = n < N ? tl.ncols - 4 * h : 0;     // the lane stores uniform row offsets below rem
        asm volatile("" : "+v"(rem));               // (compared here, not as 64 hoisted masks)
        const size_t rs = (size_t)a.ldd * 4;
        const uint8_t* p = (const uint8_t*)a.D + (size_t)tl.k0 * rs;
#pragma unroll
        for (int i = 0; i < NRB; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                asm volatile("" : "+s"(p));
                if (32 * i + 8 * (e >> 2) + (e & 3) < rem) st_f32_nc(p, voff, acc[i][e]);
                acc[i][e] = 0.f;
                p += (e & 3) == 3 ? 5 * rs : rs;     // next row: +1, or +5 after the 4th of a group of 8
            }
    };
    // group g (Q4_K block kb = g % 2 of its weight block): the K steps of raw r into acc; the next
    // group's loads go out after the first step.  Deferred stores: the previous block's set accp is
    // stored after the first step of a block's first group (the wait for the next weights, three
    // steps later, then finds those stores drained); otherwise a block's set is stored at its end.
    // Fenced steps: hoisting a step's A fragments and dequantisation over the previous step's MFMAs
    // runs out of registers.
    auto group = [&](int g, int kb, const AsRaw& r, AsRaw& fill, f32x16 (&acc)[NRB], f32x16 (&accp)[NRB]) {
        const int t0 = 4 * kb;
        step(r.a0, r.b0, q4k_step_scales(r.hd, 0), t0, acc);
        __builtin_amdgcn_sched_barrier(0);
        load(min(g + 1, ng - 1), fill);
        if (kAsDeferStores && kb == 0 && g > 0) store(accp, b0 + (g >> 1) - 1);
        __builtin_amdgcn_sched_barrier(0);
        step(r.a1, r.b1, q4k_step_scales(r.hd, 1), t0 + 1, acc);
        __builtin_amdgcn_sched_barrier(0);
        step(r.a2, r.b2, q4k_step_scales(r.hd, 2), t0 + 2, acc);
        __builtin_amdgcn_sched_barrier(0);
        step(r.a3, r.b3, q4k_step_scales(r.hd, 3), t0 + 3, acc);
        __builtin_amdgcn_sched_barrier(0);
        if (!kAsDeferStores && kb == 1) store(acc, b0 + (g >> 1));
    };
    if constexpr (kAsDeferStores) {
        // blocks in pairs: acc0 for even blocks, acc1 for odd ones
        for (int bi = 0; bi < nblk; bi += 2) {
            group(2 * bi, 0, ra, rb, acc0, acc1);
            group(2 * bi + 1, 1, rb, ra, acc0, acc1);
            if (bi + 1 < nblk) {
                group(2 * bi + 2, 0, ra, rb, acc1, acc0);
                group(2 * bi + 3, 1, rb, ra, acc1, acc0);
            }
        }
        if ((nblk - 1) & 1) store(acc1, b1 - 1);
        else store(acc0, b1 - 1);
    } else {
        for (int bi = 0; bi < nblk; ++bi) {
            group(2 * bi, 0, ra, rb, acc0, acc1);
            group(2 * bi + 1, 1, rb, ra, acc0, acc1);
        }
    }
}

// One workgroup per (tile, run of bpu weight blocks); workgroup id i runs on XCD i % 8 and XCD x
// takes tiles x, x+8, ... with all their runs (the runs of a tile share its A rows in one L2).
__global__ void __launch_bounds__(kAsThreads) k_moe_gemm_as(XArgs a) {
    extern __shared__ __align__(16) uint8_t smem_raw[];
    __shared__ int rows[XBM];
    const int nu = (a.nb + a.bpu - 1) / a.bpu;
    const int id = blockIdx.x, sid = id >> 3;
    const int tix = 8 * (sid / nu) + (id & 7), ui = sid % nu;
    if (tix >= min(a.counts[0] + a.counts[1], a.nimp)) return;
    qmm_moe_tile tl = a.tiles[tix];
    tl.ncols = max(1, min(tl.ncols, XBM));
    if (threadIdx.x < XBM) {
        const int k = tl.k0 + min((int)threadIdx.x, tl.ncols - 1);
        rows[threadIdx.x] = a.rowtab ? a.rowtab[k] : k;
    }
    __syncthreads();
    const int b0 = ui * a.bpu, b1 = min(a.nb, b0 + a.bpu);
    switch ((tl.ncols + 31) >> 5) {
        case 1: moe_as_unit<1>(a, tl, b0, b1, rows, smem_raw); break;
        case 2: moe_as_unit<2>(a, tl, b0, b1, rows, smem_raw); break;
        case 3: moe_as_unit<3>(a, tl, b0, b1, rows, smem_raw); break;
        default: moe_as_unit<4>(a, tl, b0, b1, rows, smem_raw); break;
    }
}

int launch_moe_gemm_as(XArgs a, int max_tiles, hipStream_t s) {
    const int nu = (a.nb + a.bpu - 1) / a.bpu;
    const int grid = 8 * ((max_tiles + 7) / 8) * nu;
    hipLaunchKernelGGL(k_moe_gemm_as, dim3(grid), dim3(kAsThreads), (size_t)XBM * kAsRowBytes, s, a);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

}  // namespace

int launch_q4k_rows_gemm(const void* W, const uint16_t* A, float* D, int M, int N, int K, int ldd, int trows, hipStream_t s) {
    const int nimp = (M + trows - 1) / trows;
    XArgs a{(const uint8_t*)W, (const uint8_t*)W, nullptr, nullptr, 0, nullptr, nullptr, nullptr, A, D, N, K,
            (N + XBW - 1) / XBW, ldd, trows, nimp, M};
    return launch_moe_gemm_x(false, a, nimp, s);
}

namespace {

// ------------------------------------------------------------------------------------------
// h = bf16(silu(g) * u), RNE; silu(x) = x / (1 + __expf(-x)) as the reference (fn.hip:8)
__global__ void __launch_bounds__(256) k_moe_silu_bf16(const float* __restrict__ g, const float* __restrict__ u,
                                                       uint16_t* __restrict__ h, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float x = g[i];
    h[i] = (uint16_t)f2bf_bits(x / (1.f + __expf(-x)) * u[i]);
}

}  // namespace
}  // namespace qmm

using namespace qmm;

extern "C" {

int qmm_moe_sort(const int* ids, int T, int nslot, int nexperts, int maxc, int* kpos, int* rowtok, qmm_moe_tile* tiles,
                 int* counts, void* stream) {
    if (!ids || !kpos || !rowtok || !tiles || !counts) return QMM_ERR_NULL;
    if (T < 0 || nslot < 1 || nexperts < 1 || nexperts + 1 > kMaxKeys || maxc < 1 || maxc > QMM_MOE_MAX_TILE_ROWS) return QMM_ERR_SHAPE;
    const int nkeys = nexperts + 1, ns = T * nslot;
    hipStream_t st = (hipStream_t)stream;
    // G workgroups of at least 1024 slots each, their counts (G x nkeys) held in rowtok until the
    // rowtok kernel overwrites it; one workgroup when that does not give at least 4
    const int G = std::min(std::min(ns / 1024, ns / nkeys), kSortMaxGroups);
    if (G >= 4) {
        const int per = (ns + G - 1) / G;
        const size_t lds_w = (size_t)kSortWaves * nkeys * 4;
        hipLaunchKernelGGL(k_moe_sort_count, dim3(G), dim3(kSortThreads), lds_w, st, ids, ns, nkeys, per, rowtok);
        QMM_LAUNCH_CHECK();
        hipLaunchKernelGGL(k_moe_sort_scatter, dim3(G), dim3(kSortThreads), lds_w + (size_t)2 * nkeys * 4, st, ids, ns, nkeys, per, G,
                           maxc, rowtok, kpos, tiles, counts);
        QMM_LAUNCH_CHECK();
    } else {
        const size_t lds = (size_t)(kSortWaves + 2) * nkeys * 4;
        hipLaunchKernelGGL(k_moe_sort, dim3(1), dim3(kSortThreads), lds, st, ids, ns, nslot, nkeys, maxc, kpos, tiles, counts);
        QMM_LAUNCH_CHECK();
    }
    if (ns > 0) {
        hipLaunchKernelGGL(k_moe_rowtok, dim3((ns + 255) / 256), dim3(256), 0, st, kpos, rowtok, ns, nslot);
        QMM_LAUNCH_CHECK();
    }
    return QMM_OK;
}

int qmm_moe_gemm_bf16(int fmt, int shared_fmt, const void* W, const void* Wsh, size_t ebytes, const qmm_moe_tile* tiles,
                      const int* counts, int max_tiles, const int* rowtab, const uint16_t* A, float* D, int N, int K,
                      void* stream) {
    // the reference's moe_gemm formats (gemv.hip:962-968), routed and shared independent, and IQ4_XS;
    // K granule per format as qmm_gemv_q8 (256; 64 for Q8_0_SOA, 32 for Q5_1_SOA)
    auto fmt_ok = [](int f) { return f == QMM_Q4_K || f == QMM_Q5_K || f == QMM_IQ4_XS || f == QMM_Q8_0_SOA || f == QMM_Q5_1_SOA; };
    auto kgran = [](int f) { return f == QMM_Q5_1_SOA ? 32 : f == QMM_Q8_0_SOA ? 64 : 256; };
    if (!fmt_ok(fmt) || !fmt_ok(shared_fmt)) return QMM_ERR_FORMAT;
    if (!W || !Wsh || !tiles || !counts || !A || !D) return QMM_ERR_NULL;
    if (N <= 0 || K <= 0 || K % kgran(fmt) != 0 || K % kgran(shared_fmt) != 0 || max_tiles < 0) return QMM_ERR_SHAPE;
    if (max_tiles == 0) return QMM_OK;
    if (fmt != QMM_Q4_K || shared_fmt != QMM_Q4_K)
        return launch_moe_gemm_fmt(fmt, shared_fmt, W, Wsh, ebytes, tiles, counts, max_tiles, rowtab, A, D, N, K,
                                   (hipStream_t)stream);
    XArgs a{(const uint8_t*)W, (const uint8_t*)Wsh, nullptr, nullptr, ebytes, tiles, counts, rowtab, A, D, N, K,
            (N + XBW - 1) / XBW, N, 0, max_tiles, 0, kAsBlocksPerUnit};
    if (K == kAsK) return launch_moe_gemm_as(a, max_tiles, (hipStream_t)stream);
    return launch_moe_gemm_x(false, a, max_tiles, (hipStream_t)stream);
}

int qmm_moe_gemm_gate_up_bf16(int fmt, int shared_fmt, const void* Wg, const void* Wgsh, const void* Wu, const void* Wush,
                              size_t ebytes, const qmm_moe_tile* tiles, const int* counts, int max_tiles, const int* rowtab,
                              const uint16_t* A, uint16_t* H, int N, int K, void* stream) {
    if (fmt != QMM_Q4_K || shared_fmt != QMM_Q4_K) return QMM_ERR_FORMAT;
    if (!Wg || !Wgsh || !Wu || !Wush || !tiles || !counts || !A || !H) return QMM_ERR_NULL;
    if (N <= 0 || K <= 0 || K % 256 != 0 || max_tiles < 0) return QMM_ERR_SHAPE;
    if (max_tiles == 0) return QMM_OK;
    XArgs a{(const uint8_t*)Wg, (const uint8_t*)Wgsh, (const uint8_t*)Wu, (const uint8_t*)Wush, ebytes, tiles, counts,
            rowtab, A, H, N, K, (N + XBW / 2 - 1) / (XBW / 2), N, 0, max_tiles, 0};
    return launch_moe_gemm_x(true, a, max_tiles, (hipStream_t)stream);
}

int qmm_moe_silu_bf16(const float* gate, const float* up, uint16_t* h, size_t n, void* stream) {
    if (!gate || !up || !h) return QMM_ERR_NULL;
    if (n == 0) return QMM_OK;
    hipLaunchKernelGGL(k_moe_silu_bf16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, gate, up, h, n);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

}  // extern "C"
