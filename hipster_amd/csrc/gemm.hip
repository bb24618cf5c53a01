// gemm.hip -- prefill-sized matrix products on gfx950: dequantisation to bf16, a Q4_K-weight GEMM
// with the dequantisation fused into the LDS staging of the weight tile, a plain bf16 GEMM and the
// bf16 <-> f32 helpers of the reference's engine/kernels/gemm.h.
//
// Entry points (C ABI, include/hipster_qmm.h) and the reference functions they replace:
//   qmm_dequant_bf16        hip::dequant_bf16     engine/kernels/gemm.hip:16-76,96-107
//   qmm_gemm_wq             (new) dequant_bf16 + BlasLt::gemm fused; engine/src/qwen35.cpp:204-239,
//                           engine/src/qwen4exp.cpp:513-527 are the callers it serves
//   qmm_gemm_bf16           hip::BlasLt::gemm     engine/kernels/gemm.hip:125-160 (own MFMA kernel, no hipBLASLt)
//   qmm_f32_to_bf16, qmm_bf16_to_f32, qmm_bf16_to_f32_seg, qmm_bf16_to_f32_seg2   gemm.hip:77-95
//
// Q4_K GEMM (qmm_gemm_wq): 256 x 256 output tiles, K step 64, 512 threads (two waves per SIMD, so
// one wave's MFMAs hide the other's dequantisation), v_mfma_f32_32x32x16_bf16.  A streams
// global -> LDS by DMA three stages ahead; a K step of 64 is exactly one 32-byte qs "pair" of each
// weight row's block, dequantised from registers into a two-stage bf16 W ring.  bf16 GEMM
// (qmm_gemm_bf16): 256 x 256 tiles, 4 waves, v_mfma_f32_16x16x32_bf16, register-staged two-stage
// LDS ring.  Both map workgroups XCD-aware: consecutive workgroup ids go to different XCDs, so tile
// ids are assigned so that the M tiles of one weight tile run on the same XCD and share its L2.
#include "fmt_dequant.hpp"
#include "qmm_common.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

namespace qmm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------
// Bit-exact dequantisation to bf16 (engine/src/quant.h:43-53,65-80 arithmetic, then RNE to bf16 as
// engine/kernels/gemm.hip:12).  Contraction is off: (d*sc)*q and dmin*m are rounded on their own,
// exactly as the host reference computes them.
#pragma clang fp contract(off)

// Q4_K: one thread per 32-weight sub-block (8 per block); writes 32 bf16 (64 B)
__global__ void __launch_bounds__(256) k_dequant_q4k_bf16(const uint8_t* __restrict__ W, uint16_t* __restrict__ out,
                                                          size_t nsub, int K) {
    const size_t g = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= nsub) return;
    const size_t blk = g >> 3;
    const int s = (int)(g & 7), j = s >> 1, h = s & 1;
    const uint8_t* bp = W + blk * 144;
    const uint4 hd = ld16(bp);
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    const Q4kScaleBytes sb = q4k_scale_bytes(hd.y, hd.z, hd.w);
    const float dl = d * (float)byte8(sb.sc_lo, sb.sc_hi, s), ml = dmin * (float)byte8(sb.m_lo, sb.m_hi, s);
    const uint4 q0 = ld16(bp + 16 + 32 * j), q1 = ld16(bp + 32 + 32 * j);
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    uint32_t o[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t v = h ? (qw[i] >> 4) : qw[i];
        uint32_t bf[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) bf[b] = f2bf_bits(dl * (float)((v >> (8 * b)) & 15u) - ml);
        o[2 * i] = bf[0] | (bf[1] << 16);
        o[2 * i + 1] = bf[2] | (bf[3] << 16);
    }
    // element index of this sub-block: row-major [N][K] with K = nb * 256 -> block blk holds elements blk*256..
    uint4* dst = (uint4*)(out + blk * 256 + 32 * s);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
}

// Q6_K (GGUF 210-byte blocks, or the row-SoA repack): one thread per 16 weights sharing one scale
template <int F>
__global__ void __launch_bounds__(256) k_dequant_q6k_bf16(const uint8_t* __restrict__ W, uint16_t* __restrict__ out,
                                                          size_t ngrp, int K) {
    const size_t gi = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (gi >= ngrp) return;
    const int nb = K >> 8;
    const size_t blkg = gi >> 4;                       // global block index (row * nb + b)
    const int grp = (int)(gi & 15);                    // 16-weight group within the block
    const size_t row = blkg / nb;
    const int b = (int)(blkg - row * nb);
    const uint8_t *ql, *qh, *sc, *dp;
    if constexpr (F == QMM_Q6_K) {
        const uint8_t* bp = W + blkg * 210;
        ql = bp; qh = bp + 128; sc = bp + 192; dp = bp + 208;
    } else {
        const uint8_t* rp = W + row * ((size_t)nb * 210);
        ql = rp + (size_t)b * 128; qh = rp + (size_t)nb * 128 + (size_t)b * 64;
        sc = rp + (size_t)nb * 192 + (size_t)b * 16; dp = rp + (size_t)nb * 208 + (size_t)b * 2;
    }
    const float d = h2f((uint32_t)dp[0] | ((uint32_t)dp[1] << 8));
    // element e = 16 * grp + i: half n = e / 128, r = e % 128, quarter g = r / 32, l = r % 32
    const int e0 = 16 * grp, n = e0 >> 7, r0 = e0 & 127, g = r0 >> 5, l0 = r0 & 31;
    const float ds = d * (float)(int8_t)sc[8 * n + (l0 >> 4) + 2 * g];
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
        uint32_t bf[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int l = l0 + i + k;
            const uint32_t lo = ql[64 * n + l + 32 * (g & 1)], hi = qh[32 * n + l];
            const int q = (int)((g < 2 ? (lo & 15u) : (lo >> 4)) | (((hi >> (2 * g)) & 3u) << 4)) - 32;
            bf[k] = f2bf_bits(ds * (float)q);
        }
        o[i >> 1] = bf[0] | (bf[1] << 16);
    }
    uint4* dst = (uint4*)(out + row * (size_t)K + (size_t)b * 256 + e0);
    dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
    dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
}

#pragma clang fp contract(on)

// ------------------------------------------------------------------------------------------
// bf16 <-> f32 helpers (gemm.hip:77-95 semantics; bf16 from f32 by RNE without a NaN case)
__global__ void k_f32_to_bf16(const float* __restrict__ x, uint16_t* __restrict__ o, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) o[i] = (uint16_t)f2bf_bits(x[i]);
}
__global__ void k_bf16_to_f32(const uint16_t* __restrict__ x, float* __restrict__ o, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) o[i] = bf2f(x[i]);
}
// rows m < M of a [M][Nt] bf16 matrix, columns off..off+N (plus a second matrix when x2) -> f32 [M][N]
__global__ void k_bf16_to_f32_seg2(const uint16_t* __restrict__ x, const uint16_t* __restrict__ x2, int Nt, int off, int N,
                                   float* __restrict__ o, int M) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)M * N) return;
    const int m = (int)(i / N), c = (int)(i % N);
    const size_t idx = (size_t)m * Nt + off + c;
    float v = bf2f(x[idx]);
    if (x2) v += bf2f(x2[idx]);
    o[i] = v;
}

// ------------------------------------------------------------------------------------------
// bf16 x bf16 MFMA GEMM (the BlasLt::gemm twin).  Macro tile GBM x GBN = 256 x 256, K step 64, 4 waves as 2 x 2, each wave a
// 128 x 128 tile = 8 x 8 MFMA tiles of 16 x 16 (256 f32 accumulators per lane, held in AGPRs).
// LDS holds two stages of {A 256 x 64, W 256 x 64} bf16 with rows padded to 72 elements (144 B):
// the 16-byte fragment reads of 16 consecutive rows then fall on 16 distinct 4-bank groups.
// Step s: issue the global loads of step s+1 into registers, run the 128 MFMAs of step s from
// stage s&1, write step s+1's registers into the other stage, barrier.
constexpr int GBM = 256, GBN = 256, GBK = 64, GLD = GBK + 8;
constexpr int kStageElems = (GBM + GBN) * GLD;                 // bf16 elements per stage
constexpr size_t kGemmLds = 2 * (size_t)kStageElems * 2;     // bytes (147,456)

// A tile loader: bf16 [M][K] row-major; thread t owns 16-byte column t%8 of rows t/8 + 32p
struct ALoad {
    uint4 r[8];
    __device__ __forceinline__ void load(const uint16_t* __restrict__ A, int M, int lda, int m0, int k0) {
        const int t = threadIdx.x;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const int m = min(m0 + 32 * p + (t >> 3), M - 1);
            r[p] = ld16(A + (size_t)m * lda + k0 + 8 * (t & 7));
        }
    }
    __device__ __forceinline__ void store(__bf16* La) const {
        const int t = threadIdx.x;
#pragma unroll
        for (int p = 0; p < 8; ++p) *(uint4*)&La[(32 * p + (t >> 3)) * GLD + 8 * (t & 7)] = r[p];
    }
};

// W tile loader, bf16 [N][K]: thread t copies the 64 elements of row n0+t
struct BLoadBf16 {
    uint4 r[8];
    __device__ __forceinline__ void load(const uint16_t* __restrict__ W, int N, int ldw, int n0, int k0) {
        const int n = min(n0 + (int)threadIdx.x, N - 1);
        const uint16_t* p = W + (size_t)n * ldw + k0;
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = ld16(p + 8 * i);
    }
    __device__ __forceinline__ void store(__bf16* Lb, int) const {
        uint4* dst = (uint4*)&Lb[threadIdx.x * GLD];
#pragma unroll
        for (int i = 0; i < 8; ++i) dst[i] = r[i];
    }
};

// tile id -> (m tile, n tile), XCD-aware: workgroup id i runs on XCD i % 8; give XCD x the
// contiguous tile range [x * ntiles/8, (x+1) * ntiles/8) with M tiles fastest, so the M tiles that
// share a weight tile share one L2.  Falls back to the plain order when the count is not a multiple of 8.
__device__ __forceinline__ void tile_of(int bid, int mt, int nt, int& tm, int& tn) {
    const int ntiles = mt * nt;
    int id = bid;
    if ((ntiles & 7) == 0) id = (bid & 7) * (ntiles >> 3) + (bid >> 3);
    tm = id % mt;
    tn = id / mt;
}

// 128 MFMAs of one K step from one LDS stage
__device__ __forceinline__ void mfma_step(const __bf16* La, const __bf16* Lb, int wm, int wn, int fr, int fk, f32x4 (&acc)[8][8]) {
#pragma unroll
    for (int ks = 0; ks < GBK / 32; ++ks) {
        bf16x8 af[8], bf[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) af[i] = *(const bf16x8*)&La[(128 * wm + 16 * i + fr) * GLD + 32 * ks + fk];
#pragma unroll
        for (int jn = 0; jn < 8; ++jn) bf[jn] = *(const bf16x8*)&Lb[(128 * wn + 16 * jn + fr) * GLD + 32 * ks + fk];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int jn = 0; jn < 8; ++jn) acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[jn], acc[i][jn], 0, 0, 0);
    }
}

// Step s: the global loads of step s+1 go out first, then the MFMAs of step s from LDS stage s&1,
// then step s+1's registers are written (A copied, W dequantised) into the other stage.
template <class BL, class WT, bool OUT_BF16>
__global__ void __launch_bounds__(256) k_gemm(const uint16_t* __restrict__ A, const WT* __restrict__ W, void* __restrict__ D,
                                              int M, int N, int K, int lda, int ldw) {
    extern __shared__ __align__(16) uint8_t smem_raw[];
    __bf16* const lds = (__bf16*)smem_raw;
    const int mt = (M + GBM - 1) / GBM, nt = (N + GBN - 1) / GBN;
    int tm, tn;
    tile_of(blockIdx.x, mt, nt, tm, tn);
    const int m0 = tm * GBM, n0 = tn * GBN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wm = wave & 1, wn = wave >> 1;
    const int nk = K / GBK;
    ALoad al;
    BL bl;
    al.load(A, M, lda, m0, 0);
    bl.load(W, N, ldw, n0, 0);
    al.store(lds);
    bl.store(lds + GBM * GLD, 0);
    lds_barrier();
    f32x4 acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int jn = 0; jn < 8; ++jn) acc[i][jn] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int fr = lane & 15, fk = 8 * (lane >> 4);
    for (int s = 0; s < nk; ++s) {
        const __bf16* La = lds + (size_t)(s & 1) * kStageElems;
        const bool more = s + 1 < nk;
        if (more) {
            al.load(A, M, lda, m0, (s + 1) * GBK);
            bl.load(W, N, ldw, n0, (s + 1) * GBK);
        }
        mfma_step(La, La + GBM * GLD, wm, wn, fr, fk, acc);
        if (more) {
            __bf16* Sa = lds + (size_t)((s + 1) & 1) * kStageElems;
            al.store(Sa);
            bl.store(Sa + GBM * GLD, (s + 1) * GBK);
        }
        lds_barrier();
    }
    // epilogue: acc[i][jn][r] = D[m0 + 128wm + 16i + 4*(lane/16) + r][n0 + 128wn + 16jn + lane%16]
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + 128 * wm + 16 * i + 4 * (lane >> 4) + r;
            if (m >= M) continue;
#pragma unroll
            for (int jn = 0; jn < 8; ++jn) {
                const int n = n0 + 128 * wn + 16 * jn + fr;
                if (n >= N) continue;
                if constexpr (OUT_BF16) ((uint16_t*)D)[(size_t)m * N + n] = (uint16_t)f2bf_bits(acc[i][jn][r]);
                else ((float*)D)[(size_t)m * N + n] = acc[i][jn][r];
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// Fused Q4_K GEMM with DMA-staged A.  The A tile goes global -> LDS with global_load_lds_dwordx4 (no
// registers), three stages deep; the bf16 W tile, dequantised from Q4_K registers, two stages.
// Stage layout: 256 rows x 8 chunks of 16 B, unpadded, chunk c of row r stored in slot
// r*8 + (c ^ ((r >> 1) & 7)): a DMA instruction writes 1 KiB of consecutive slots (lane i -> slot
// base + i, so the swizzle is applied to the global address each lane fetches), and the 16
// consecutive rows of an MFMA fragment read land on 16 distinct 4-bank groups.
// Step s: DMA A tile s+2 -> A stage (s+2)%3; MFMAs of tile s (A stage s%3, W stage s%2); tile s+1's
// W registers -> W stage (s+1)%2; W tile s+2 -> registers; wait; barrier.  The A tile thus has two
// steps of MFMA time to land.
constexpr int kChunks = GBM * GBK / 8;                         // 16-byte chunks per stage (2048)

// The five stages are separate LDS variables and every access names its stage at compile time (the
// K loop is unrolled by 6 = 3 A stages x 2 W stages).  The compiler then knows which stage each DMA
// writes, so an LDS read waits only for DMA into its own stage, and its count of the W register
// loads stays exact (with one LDS array it would wait for every DMA in flight before each read).
__shared__ uint4 gA0[kChunks], gA1[kChunks], gA2[kChunks], gB0[kChunks], gB1[kChunks];
template <int S>
__device__ __forceinline__ uint4* ga() {
    if constexpr (S == 0) return gA0;
    else if constexpr (S == 1) return gA1;
    else return gA2;
}
template <int S>
__device__ __forceinline__ uint4* gb() {
    if constexpr (S == 0) return gB0;
    else return gB1;
}
template <int V>
using IC = std::integral_constant<int, V>;

// Workgroup barrier for a kernel whose DMA into LDS is still in flight on purpose.  A workgroup
// release fence on LDS would wait for every outstanding DMA (vmcnt(0)); here the release is at wave
// scope (it only keeps the compiler from moving LDS accesses across it), this wave's own LDS stores
// are retired with lgkmcnt(0), and the DMA a reader depends on has been waited for explicitly with
// vmcnt(n) before the barrier.
__device__ __forceinline__ void lds_barrier_dma() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_s_waitcnt(0xC07F);       // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ int swz(int r, int c) { return r * 8 + (c ^ ((r >> 1) & 7)); }

// 32 x 32 x 16 MFMA tiles.  Operand layout (v_mfma_f32_32x32x16_bf16): lane l supplies row (or
// column) l%32 and the 8 consecutive k values 8*(l/32)..+7 of the 16-wide K slice; output element i
// of lane l is row 8*(i/4) + 4*(l/32) + i%4, column l%32.  Fragment row R = base + 32*t + l%32 keeps
// (R >> 1) & 7 == ((l%32) >> 1) & 7, so fragment t of slice ks sits at lane base + 256*t chunks.
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------------------------------------
// Two waves per SIMD ("ping-pong"): 512 threads, 8 waves as 2 (M) x 4 (N), wave tile 128 x 64 =
// 4 x 2 MFMA tiles of 32 x 32 (128 accumulators per lane).  The two waves of a SIMD interleave in
// hardware: while one issues MFMAs the other runs its W dequantisation, DMA issue and fragment
// reads, so the non-MFMA work of a step hides under the other wave's MFMAs.  Each W row is
// dequantised by two threads, one sub-block (32 weights) each.
constexpr int kPPThreads = 512;

__device__ __forceinline__ void dma_a_pp(const uint16_t* __restrict__ A, int M, int lda, int m0, int k0, uint4* La) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // chunk slot p = (4w + i) * 64 + lane: row r = 32w + 8i + lane/8, slot column lane%8
        const int r = 32 * wave + 8 * i + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
        const uint32_t off = (uint32_t)min(m0 + r, M - 1) * (uint32_t)lda + (uint32_t)(k0 + 8 * c);
        __builtin_amdgcn_global_load_lds(A + off, La + (4 * wave + i) * 64, 16, 0, 0);
    }
}

struct WRawQ4KHalf {
    uint4 hd, q0, q1;
    __device__ __forceinline__ void load(const uint8_t* __restrict__ W, int N, int K, int, int n0, int k0) {
        const int n = min(n0 + (int)(threadIdx.x >> 1), N - 1);
        const uint8_t* bp = W + (size_t)n * ((size_t)(K >> 8) * 144) + (size_t)(k0 >> 8) * 144;
        const int j = (k0 >> 6) & 3;
        hd = ld16(bp);
        q0 = ld16(bp + 16 + 32 * j);
        q1 = ld16(bp + 32 + 32 * j);
    }
    // thread t: row t/2, sub-block 2j + (t&1): 32 bf16 -> chunks 4*(t&1)..+3 of the row, each weight
    // bf16(fmaf(dl, q, -ml)) through v_fma_mix_f32 (q4_bf16x8_mix: the low nibbles with dl * 2^24, the
    // high ones in place with dl * 2^20)
    __device__ __forceinline__ void store(uint4* Lb, int k0) const {
        const int t = threadIdx.x, h = t & 1, row = t >> 1;
        const int sbi = 2 * ((k0 >> 6) & 3) + h;
        const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
        const Q4kScaleBytes sb = q4k_scale_bytes(hd.y, hd.z, hd.w);
        const float dl = d * (float)byte8(sb.sc_lo, sb.sc_hi, sbi), ml = dmin * (float)byte8(sb.m_lo, sb.m_hi, sbi);
        const float s24 = dl * (h ? 1048576.f : 16777216.f);
        const uint32_t m = h ? 0x00f000f0u : 0x000f000fu;
        const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const qmm_bf16x8 v = q4_bf16x8_mix(qw[2 * c], qw[2 * c + 1], m, s24, -ml);
            Lb[swz(row, 4 * h + c)] = __builtin_bit_cast(uint4, v);
        }
    }
};

// W from bf16 rows [N][K] (the BlasLt::gemm twin): thread t copies the 32 weights of row t/2, half t&1
// of the step, a step ahead
struct WRawBf16Half {
    SubRaw r;                               // r.v[0..3]: the 64 bytes
    __device__ __forceinline__ void load(const uint8_t* __restrict__ W, int N, int, int ldw, int n0, int k0) {
        const int n = min(n0 + (int)(threadIdx.x >> 1), N - 1);
        const uint16_t* p = (const uint16_t*)W + (size_t)n * ldw + k0 + 32 * (threadIdx.x & 1);
#pragma unroll
        for (int c = 0; c < 4; ++c) r.v[c] = ld16(p + 8 * c);
    }
    __device__ __forceinline__ void store(uint4* Lb, int) const {
        const int t = threadIdx.x, h = t & 1, row = t >> 1;
#pragma unroll
        for (int c = 0; c < 4; ++c) Lb[swz(row, 4 * h + c)] = r.v[c];
    }
};

// W in one of the other quantised formats: thread t loads the raw bytes of row t/2's sub-block
// (k0/32 + (t&1)) a step ahead and dequantises them exactly (as qmm_dequant_bf16), RNE to bf16
template <int F>
struct WRawFmtHalf {
    SubRaw r;
    __device__ __forceinline__ void load(const uint8_t* __restrict__ W, int N, int K, int, int n0, int k0) {
        const int n = min(n0 + (int)(threadIdx.x >> 1), N - 1);
        sub_load<F>(W + (size_t)n * fmt_row_bytes_rt(F, K), K, (k0 >> 5) + (int)(threadIdx.x & 1), r);
    }
    __device__ __forceinline__ void store(uint4* Lb, int k0) const {
        const int t = threadIdx.x, h = t & 1, row = t >> 1;
        float w[32];
        sub_decode<F>(r, (k0 >> 5) + h, w);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = f2bf_bits(w[8 * c + 2 * k]) | (f2bf_bits(w[8 * c + 2 * k + 1]) << 16);
            Lb[swz(row, 4 * h + c)] = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
};

// D = A . W^T with W from the source WR (Q4_K blocks, bf16 rows or another format), f32 or bf16 (RNE)
// out.  K % 128 == 0 (an even step count for the 3 x 2 stage unroll).
template <class WR, bool OUT_BF16>
__global__ void __launch_bounds__(kPPThreads) k_gemm_pp(const uint16_t* __restrict__ A, const uint8_t* __restrict__ W,
                                                       void* __restrict__ Dv, int M, int N, int K, int ldd, int lda,
                                                       int ldw) {
    const int mt = (M + GBM - 1) / GBM, nt = (N + GBN - 1) / GBN;
    int tm, tn;
    tile_of(blockIdx.x, mt, nt, tm, tn);
    const int m0 = tm * GBM, n0 = tn * GBN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wm = wave & 1, wn = wave >> 1;
    const int nk = K / GBK, lastk = (nk - 1) * GBK;
    WR wr;
    wr.load(W, N, K, ldw, n0, 0);
    dma_a_pp(A, M, lda, m0, 0, ga<0>());
    dma_a_pp(A, M, lda, m0, min(GBK, lastk), ga<1>());
    wr.store(gb<0>(), 0);
    wr.load(W, N, K, ldw, n0, min(GBK, lastk));
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jn = 0; jn < 2; ++jn)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][jn][e] = 0.f;
    const int fr = lane & 31, fc = lane >> 5, fx = (fr >> 1) & 7;
    int foa[4], fob[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        foa[ks] = (128 * wm + fr) * 8 + ((2 * ks + fc) ^ fx);
        fob[ks] = (64 * wn + fr) * 8 + ((2 * ks + fc) ^ fx);
    }
    // step s with A stage SA = s % 3 and W stage SB = s % 2
    auto body = [&](auto sa_c, auto sb_c, int s) {
        constexpr int SA = decltype(sa_c)::value, SB = decltype(sb_c)::value;
        const uint4* La = ga<SA>();
        const uint4* Lb = gb<SB>();
        dma_a_pp(A, M, lda, m0, min((s + 2) * GBK, lastk), ga<(SA + 2) % 3>());
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8 af[4], bf[2];
#pragma unroll
            for (int t = 0; t < 4; ++t) { const uint4 v = La[foa[ks] + 256 * t]; af[t] = *(const bf16x8*)&v; }
#pragma unroll
            for (int t = 0; t < 2; ++t) { const uint4 v = Lb[fob[ks] + 256 * t]; bf[t] = *(const bf16x8*)&v; }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jn = 0; jn < 2; ++jn) acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[jn], acc[i][jn], 0, 0, 0);
        }
        wr.store(gb<1 - SB>(), min((s + 1) * GBK, lastk));
        wr.load(W, N, K, ldw, n0, min((s + 2) * GBK, lastk));
        // A tile s+1 (DMA'd a step ago, before W tile s+1's loads) has landed once at most this
        // step's 4 DMAs and 3 W loads are outstanding
        __builtin_amdgcn_s_waitcnt(0x0F77);   // vmcnt <= 7
        lds_barrier_dma();
    };
    int s = 0;
    for (; s + 6 <= nk; s += 6) {
        body(IC<0>(), IC<0>(), s);
        body(IC<1>(), IC<1>(), s + 1);
        body(IC<2>(), IC<0>(), s + 2);
        body(IC<0>(), IC<1>(), s + 3);
        body(IC<1>(), IC<0>(), s + 4);
        body(IC<2>(), IC<1>(), s + 5);
    }
    if (s < nk) {                              // nk is even, so 2 or 4 steps remain
        body(IC<0>(), IC<0>(), s);
        body(IC<1>(), IC<1>(), s + 1);
        if (s + 2 < nk) {
            body(IC<2>(), IC<0>(), s + 2);
            body(IC<0>(), IC<1>(), s + 3);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);            // drain the clamped trailing DMAs
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int m = m0 + 128 * wm + 32 * i + 8 * (e >> 2) + 4 * fc + (e & 3);
            if (m >= M) continue;
#pragma unroll
            for (int jn = 0; jn < 2; ++jn) {
                const int n = n0 + 64 * wn + 32 * jn + fr;
                if (n < N) {
                    if constexpr (OUT_BF16) ((uint16_t*)Dv)[(size_t)m * ldd + n] = (uint16_t)f2bf_bits(acc[i][jn][e]);
                    else ((float*)Dv)[(size_t)m * ldd + n] = acc[i][jn][e];
                }
            }
        }
    }
}

// One workgroup of k_gemm_pp fills a CU (160 KiB of LDS), so its tiles run in rounds of one per
// CU.  When the last round would keep at most a quarter of the CUs busy for a whole tile time, the
// 256 x 256 kernel takes only whole rounds (whole columns of M tiles) and the remaining columns go
// to the grouped-GEMM kernel as (32 rows x 256 columns) work units, enough of them to spread over
// every CU.  Every output element is one bf16 MFMA dot product over K in the same order either way.
int launch_gemm_q4k(const void* W, const uint16_t* A, float* D, int M, int N, int K, hipStream_t s) {
    const int mt = (M + GBM - 1) / GBM, nt = (N + GBN - 1) / GBN, cus = device_cu_count();
    int nbig = nt;                                   // column tiles for the 256 x 256 kernel
    const int total = mt * nt, rem = total % cus;
    if (total > cus && rem != 0 && 4 * rem <= cus && mt <= cus) nbig = (total - rem) / mt;
    const int nb_cols = std::min(N, nbig * GBN);
    if (nbig > 0) {
        hipLaunchKernelGGL((k_gemm_pp<WRawQ4KHalf, false>), dim3(mt * nbig), dim3(kPPThreads), 0, s, A, (const uint8_t*)W, D, M,
                           nb_cols, K, N, K, K);
        QMM_LAUNCH_CHECK();
    }
    if (nb_cols < N) {
        const size_t rowbytes = (size_t)(K / 256) * 144;
        return launch_q4k_rows_gemm((const uint8_t*)W + (size_t)nb_cols * rowbytes, A, D + nb_cols, M, N - nb_cols, K, N, 32, s);
    }
    return QMM_OK;
}


// ---- bf16 dequantisation of the other formats (gemm.hip:16-50,83-92 of the reference): one thread
// per 32-weight sub-block (dq_sub32: exact f32), 64 bytes of bf16 out, round-to-nearest-even
// (gemm.hip:12).
template <int F>
__global__ void __launch_bounds__(256) k_dequant_fmt_bf16(const uint8_t* __restrict__ W, uint16_t* __restrict__ out,
                                                         size_t nsub, int K) {
    const size_t g = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= nsub) return;
    const int n32 = K >> 5;
    const size_t row = g / n32;
    const int sb = (int)(g - row * n32);
    float w[32];
    dq_sub32<F>(W + row * fmt_row_bytes_rt(F, K), K, sb, w);
    uint4* dst = (uint4*)(out + row * (size_t)K + 32 * (size_t)sb);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = f2bf_bits(w[8 * v + 2 * k]) | (f2bf_bits(w[8 * v + 2 * k + 1]) << 16);
        dst[v] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

}  // namespace
}  // namespace qmm

using namespace qmm;

extern "C" {

int qmm_dequant_bf16(int fmt, const void* W, uint16_t* out, int N, int K, void* stream) {
    if (!W || !out) return QMM_ERR_NULL;
    // K % 256, or K % 64 (Q8_0_SOA) / K % 32 (Q5_1_SOA) for the row-SoA repacks of 32-weight blocks
    const int kg = fmt == QMM_Q5_1_SOA ? 32 : fmt == QMM_Q8_0_SOA ? 64 : 256;
    if (N <= 0 || K <= 0 || K % kg != 0) return QMM_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    const size_t nb = (size_t)N * (K / 256);
    const size_t nsub = (size_t)N * (K / 32);      // 32-weight sub-blocks
    switch (fmt) {
        case QMM_Q4_K:
            hipLaunchKernelGGL(k_dequant_q4k_bf16, dim3((unsigned)((nb * 8 + 255) / 256)), dim3(256), 0, s, (const uint8_t*)W, out,
                               nb * 8, K);
            break;
        case QMM_Q6_K:
            hipLaunchKernelGGL(k_dequant_q6k_bf16<QMM_Q6_K>, dim3((unsigned)((nb * 16 + 255) / 256)), dim3(256), 0, s,
                               (const uint8_t*)W, out, nb * 16, K);
            break;
        case QMM_Q6_K_SOA:
            hipLaunchKernelGGL(k_dequant_q6k_bf16<QMM_Q6_K_SOA>, dim3((unsigned)((nb * 16 + 255) / 256)), dim3(256), 0, s,
                               (const uint8_t*)W, out, nb * 16, K);
            break;
#define QMM_DQF(F) case F: hipLaunchKernelGGL(k_dequant_fmt_bf16<F>, dim3((unsigned)((nsub + 255) / 256)), dim3(256), 0, s, \
                                              (const uint8_t*)W, out, nsub, K); break;
        QMM_DQF(QMM_Q5_K) QMM_DQF(QMM_IQ4_XS) QMM_DQF(QMM_Q8_0_SOA) QMM_DQF(QMM_Q5_1_SOA)
#undef QMM_DQF
        default: return QMM_ERR_FORMAT;
    }
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_gemm_wq(int fmt, const void* W, const uint16_t* A, float* D, int M, int N, int K, void* stream) {
    if (!(fmt == QMM_Q4_K || fmt == QMM_Q5_K || fmt == QMM_IQ4_XS || fmt == QMM_Q6_K_SOA || fmt == QMM_Q8_0_SOA ||
          fmt == QMM_Q5_1_SOA))
        return QMM_ERR_FORMAT;
    if (!W || !A || !D) return QMM_ERR_NULL;
    // K % 256 for the block formats (K % 512 for Q6_K_SOA: an even block count keeps its streams dword
    // aligned); the 32-weight SoA formats need K % 128 (the kernel's even step count)
    const int kg = (fmt == QMM_Q8_0_SOA || fmt == QMM_Q5_1_SOA) ? 2 * GBK : fmt == QMM_Q6_K_SOA ? 512 : 256;
    if (M <= 0 || N <= 0 || K <= 0 || K % kg != 0) return QMM_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    if (fmt == QMM_Q4_K) return launch_gemm_q4k(W, A, D, M, N, K, s);
    const dim3 grid((unsigned)(((M + GBM - 1) / GBM) * ((N + GBN - 1) / GBN)));
#define QMM_GWQ(F) case F: hipLaunchKernelGGL((k_gemm_pp<WRawFmtHalf<F>, false>), grid, dim3(kPPThreads), 0, s, A, (const uint8_t*)W, \
                                              (void*)D, M, N, K, N, K, K); break;
    switch (fmt) {
        QMM_GWQ(QMM_Q5_K) QMM_GWQ(QMM_IQ4_XS) QMM_GWQ(QMM_Q6_K_SOA) QMM_GWQ(QMM_Q8_0_SOA) QMM_GWQ(QMM_Q5_1_SOA)
    }
#undef QMM_GWQ
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_gemm_bf16_ld(const uint16_t* A, int lda, const uint16_t* W, int ldw, uint16_t* D, int M, int N, int K, void* stream) {
    if (!A || !W || !D) return QMM_ERR_NULL;
    if (M <= 0 || N <= 0 || K <= 0 || K % GBK != 0 || lda < K || ldw < K) return QMM_ERR_SHAPE;
    // 16-byte row pieces: both operands' rows start 16-byte aligned
    if (((uintptr_t)A | (uintptr_t)W) % 16 != 0 || lda % 8 != 0 || ldw % 8 != 0) return QMM_ERR_ARG;
    // the DMA of A addresses rows with 32-bit element offsets
    if ((uint64_t)(M - 1) * (uint64_t)lda + (uint64_t)K > 0xffffffffull) return QMM_ERR_SHAPE;
    const int grid = ((M + GBM - 1) / GBM) * ((N + GBN - 1) / GBN);
    if (K % (2 * GBK) == 0)     // the two-waves-per-SIMD kernel of the fused GEMM, bf16 rows as its W source
        hipLaunchKernelGGL((k_gemm_pp<WRawBf16Half, true>), dim3(grid), dim3(kPPThreads), 0, (hipStream_t)stream, A,
                           (const uint8_t*)W, (void*)D, M, N, K, N, lda, ldw);
    else
        hipLaunchKernelGGL((k_gemm<BLoadBf16, uint16_t, true>), dim3(grid), dim3(256), kGemmLds, (hipStream_t)stream, A, W,
                           (void*)D, M, N, K, lda, ldw);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_gemm_bf16(const uint16_t* A, const uint16_t* W, uint16_t* D, int M, int N, int K, void* stream) {
    return qmm_gemm_bf16_ld(A, K, W, K, D, M, N, K, stream);
}

int qmm_f32_to_bf16(const float* x, uint16_t* out, size_t n, void* stream) {
    if (!x || !out) return QMM_ERR_NULL;
    if (n == 0) return QMM_OK;
    hipLaunchKernelGGL(k_f32_to_bf16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x, out, n);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_bf16_to_f32(const uint16_t* x, float* out, size_t n, void* stream) {
    if (!x || !out) return QMM_ERR_NULL;
    if (n == 0) return QMM_OK;
    hipLaunchKernelGGL(k_bf16_to_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x, out, n);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_bf16_to_f32_seg2(const uint16_t* x, const uint16_t* x2, int Nt, int off, int N, float* out, int M, void* stream) {
    if (!x || !out) return QMM_ERR_NULL;
    if (M < 0 || N < 0 || off < 0 || off + N > Nt) return QMM_ERR_SHAPE;
    const size_t n = (size_t)M * N;
    if (n == 0) return QMM_OK;
    hipLaunchKernelGGL(k_bf16_to_f32_seg2, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x, x2, Nt, off,
                       N, out, M);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_bf16_to_f32_seg(const uint16_t* x, int Nt, int off, int N, float* out, int M, void* stream) {
    return qmm_bf16_to_f32_seg2(x, nullptr, Nt, off, N, out, M, stream);
}

}  // extern "C"
