// router.hip -- the MoE router matmul on gfx950 (wave64), and the router matmul + routing in one call:
//
//   this library        reference
//   qmm_f32_gemv        fn::f32_gemv            engine/kernels/fn.h:37, fn.hip:251-277
//   qmm_moe_router      fn::f32_gemv + fn::moe_route (engine/src/qwen4exp.cpp:346-347)
//   qmm_gemm_f32        hip::BlasLt::gemm_f32   engine/kernels/gemm.h:31, gemm.hip:162-186 (the prefill
//                                               router, qwen4exp.cpp:626; hipBLASLt there)
//
// y[t][n] = W[n] . x[t] in f32, computed the reference's way so that the logits are its bits: a row is
// one group of 32 lanes (here half a wave64), lane l accumulates the float4 steps i = 4l + 128k in
// order, each step t = fma(a.w, b.w, fma(a.z, b.z, fma(a.x, b.x, a.y * b.y))) and acc += t (the
// contraction the reference's hipcc build makes of `acc += a.x*b.x + a.y*b.y + a.z*b.z + a.w*b.w`),
// and the 32 partial sums are folded by the xor butterfly (lane l with l^16, then l^8, ..., l^1).
// A column's arithmetic does not depend on how many columns share the pass (T-invariant).
//
// The reference launches one kernel per 8 tokens; here one launch covers every pass of 1, 2 or 8 tokens
// (grid y).
// A workgroup is one wave (two rows), so the 513-row router spreads over every CU; per pass the lanes
// issue the W and x loads of up to 10 steps before the arithmetic; W (N x K f32, 5.25 MB for the
// 513 x 2560 router) is read once per pass.
#include "qmm_common.hpp"

namespace qmm {
namespace {

constexpr int kGemvRowsPerBlock = 2;    // one wave = 2 rows of 32 lanes: N/2 workgroups spread over the CUs

// U float4 steps per lane are loaded before their arithmetic (U*(1+NT) float4 registers), so a lane
// makes ceil(K / (128 U)) memory round trips
template <int NT, int U>
__global__ void __launch_bounds__(64) k_f32_gemv(const float* __restrict__ W, const float* __restrict__ x,
                                                 float* __restrict__ y, int N, int K, int T) {
    const int n = blockIdx.x * kGemvRowsPerBlock + (threadIdx.x >> 5), l = threadIdx.x & 31;
    const int t0 = blockIdx.y * NT;     // NT columns per pass
    const int nt = min(NT, T - t0);
    if (n >= N) return;                 // uniform over the 32 lanes of a row
    const float* w = W + (size_t)n * K;
    const float* xr = x + (size_t)t0 * K;
    float acc[NT];
#pragma unroll
    for (int c = 0; c < NT; ++c) acc[c] = 0.f;
    for (int i0 = 4 * l; i0 < K; i0 += 128 * U) {
        float4 a[U], b[U][NT];
#pragma unroll
        for (int u = 0; u < U; ++u) {                // clamped addresses: every load is in bounds
            const int i = min(i0 + 128 * u, K - 4);
            a[u] = *(const float4*)(w + i);
#pragma unroll
            for (int c = 0; c < NT; ++c) b[u][c] = *(const float4*)(xr + (size_t)min(c, nt - 1) * K + i);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (i0 + 128 * u < K) {
#pragma unroll
                for (int c = 0; c < NT; ++c) {
                    const float4 bb = b[u][c];
                    const float t = fmaf(a[u].w, bb.w, fmaf(a[u].z, bb.z, fmaf(a[u].x, bb.x, a[u].y * bb.y)));
                    acc[c] = acc[c] + t;
                }
            }
        }
    }
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        const float v = hw32_sum(acc[c]);
        if (l == 0 && c < nt) y[(size_t)(t0 + c) * N + n] = v;
    }
}

// D[m][n] = A[m] . W[n] over K in f32 on the matrix cores (v_mfma_f32_32x32x2_f32): the prefill router
// GEMM for any K % 4 == 0 (K % 32 == 0 takes k_gemm_f32d below), 2048 x 513 x 2560 for a 2048-token chunk -- about one 32 x 32 output block per SIMD of the
// chip, so the work is cut finer than the output: a workgroup owns one 32 x 32 block and its 4 waves
// take a quarter of K each (steps of 16), added in a fixed order ((w0 + w1) + (w2 + w3)) through LDS
// at the end.  There is no reuse inside a
// workgroup to stage, so each lane loads its A and W pieces straight into registers, three steps
// ahead of their MFMAs.  Tiles run W-block-fastest and each XCD takes a contiguous range of them
// (workgroup i runs on XCD i % 8): an XCD holds a few A strips (2 MB for 8 strips of 2048-float rows)
// and sweeps W with them, so the re-reads of A and W are L2 hits.  Lane (r, h) feeds row r at k = kb + 8h + i to MFMA i of a step (any pairing of
// k across the MFMAs gives the same sum over k); one accumulator chain (back-to-back MFMAs of one
// shape forward it), which keeps the kernel under 96 registers: 5 workgroups per CU, so the 1088
// workgroups of a 2048-token chunk run in one round.  f32 accumulation in the matrix unit's order: the result agrees
// with a double-precision dot to f32 rounding (the reference's hipBLASLt order is unspecified too).
typedef float f32x16_t __attribute__((ext_vector_type(16)));
constexpr int kFTile = 32, kFStep = 16, kFRing = 3;

// p[k .. k + 3] if k < lim, else zeros (the address is clamped so that the load stays in the row)
__device__ __forceinline__ float4 ld_f4z(const float* p, int k, int lim) {
    const float4 v = *(const float4*)(p + min(k, lim - 4));
    const bool in = k < lim;
    return make_float4(in ? v.x : 0.f, in ? v.y : 0.f, in ? v.z : 0.f, in ? v.w : 0.f);
}

struct F32Piece { float4 a0, a1, w0, w1; };

__global__ void __launch_bounds__(256) k_gemm_f32(const float* __restrict__ A, const float* __restrict__ W,
                                                  float* __restrict__ D, int M, int N, int K, int nnt, int xcd_ord) {
    __shared__ float red[4 * 16 * 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int fr = lane & 31, h = lane >> 5;
    const int id = blockIdx.x, total = gridDim.x;
    const int t = xcd_ord ? (id & 7) * (total >> 3) + (id >> 3) : id;
    const int m0 = (t / nnt) * kFTile, n0 = (t % nnt) * kFTile;
    const float* ar = A + (size_t)min(m0 + fr, M - 1) * K;
    const float* wr = W + (size_t)min(n0 + fr, N - 1) * K;
    // steps of 16: the full ones [0, nfull) split over the 4 waves; a partial last step (K % 16 != 0)
    // is done by wave 3 after its loop, with the lanes past K loading zeros
    const int nfull = K / kFStep, nst = (K + kFStep - 1) / kFStep;
    const int s0 = wave * nst / 4, s1 = min((wave + 1) * nst / 4, nfull);
    F32Piece ring[kFRing];
    // plain loads (every step of [s0, s1) is in the rows), consumed by the MFMAs as they are, so that
    // the waits for one ring slot leave the next slots' loads in flight
    auto load = [&](int s, F32Piece& p) {
        const float* pa = ar + (size_t)s * kFStep + 8 * h;
        const float* pw = wr + (size_t)s * kFStep + 8 * h;
        p.a0 = *(const float4*)pa; p.a1 = *(const float4*)(pa + 4);
        p.w0 = *(const float4*)pw; p.w1 = *(const float4*)(pw + 4);
    };
    f32x16_t acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    auto mma = [&](const F32Piece& p) {
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(p.a0.x, p.w0.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(p.a0.y, p.w0.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(p.a0.z, p.w0.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(p.a0.w, p.w0.w, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(p.a1.x, p.w1.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(p.a1.y, p.w1.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(p.a1.z, p.w1.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(p.a1.w, p.w1.w, acc, 0, 0, 0);
    };
    if (s0 < s1) {
#pragma unroll
        for (int i = 0; i < kFRing - 1; ++i) load(min(s0 + i, s1 - 1), ring[i]);
        for (int s = s0; s < s1; s += kFRing) {         // ring slot i holds step s + i
#pragma unroll
            for (int i = 0; i < kFRing; ++i) {
                // steps past the wave's share re-load its last step (in bounds) and are not used
                load(min(s + i + kFRing - 1, s1 - 1), ring[(i + kFRing - 1) % kFRing]);
                if (s + i < s1) mma(ring[i]);
            }
        }
    }
    if (wave == 3 && nfull < nst) {
        F32Piece p;
        const int k = nfull * kFStep + 8 * h;
        p.a0 = ld_f4z(ar, k, K); p.a1 = ld_f4z(ar, k + 4, K);
        p.w0 = ld_f4z(wr, k, K); p.w1 = ld_f4z(wr, k + 4, K);
        mma(p);
    }
    // the four quarter sums, added in a fixed order; red[(w * 16 + e) * 64 + lane]
#pragma unroll
    for (int e = 0; e < 16; ++e) red[(wave * 16 + e) * 64 + lane] = acc[e];
    __syncthreads();
    const int q = wave;                                  // this thread: elements 4q .. 4q + 3 of lane `lane`
    const int n = n0 + fr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = 4 * q + i, o = e * 64 + lane;
        const float v = (red[o] + red[16 * 64 + o]) + (red[2 * 16 * 64 + o] + red[3 * 16 * 64 + o]);
        const int m = m0 + 8 * (e >> 2) + 4 * h + (e & 3);   // acc[e]: row 8 (e / 4) + 4 h + e % 4, column fr
        if (m < M && n < N) D[(size_t)m * N + n] = v;
    }
}

// The same product with the A and W pieces staged by DMA (global_load_lds_dwordx4) into a ring of NS
// stages private to each wave (stage = 32 k: 4 KB of A rows, 4 KB of W rows), for K % 32 == 0.  One
// DMA instruction moves 8 rows x 128 contiguous bytes (whole cache lines), where the register kernel's
// loads touch 32 rows per instruction; the ring needs no registers.  With NS = 2 (64 KB per workgroup,
// two workgroups per CU) a wave computes one stage while the next lands and the other workgroup's
// wave on the same SIMD covers the rest of the latency: 59 us at 2048 x 513 x 2048 against 86 us for
// the register kernel.  Slot (row, chunk q) of a stage
// sits at row * 8 + (q ^ swz(row)): the DMA lanes of one instruction write 8 whole rows, and the
// MFMA fragment reads (16 consecutive rows, one chunk) fall in distinct banks.
__device__ __forceinline__ int f32_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

#define QMM_VMWAIT(n) asm volatile("s_waitcnt vmcnt(" #n ")" ::: "memory")

template <int NS>
__global__ void __launch_bounds__(256) k_gemm_f32d(const float* __restrict__ A, const float* __restrict__ W,
                                                   float* __restrict__ D, int M, int N, int K, int nnt, int xcd_ord) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int fr = lane & 31, h = lane >> 5;
    const int id = blockIdx.x, total = gridDim.x;
    const int t = xcd_ord ? (id & 7) * (total >> 3) + (id >> 3) : id;
    const int m0 = (t / nnt) * kFTile, n0 = (t % nnt) * kFTile;
    const int nstg = K / 32, s0 = wave * nstg / 4, n = (wave + 1) * nstg / 4 - s0;
    uint8_t* wring = smem + (size_t)wave * NS * 8192;
    const uint32_t lring = lds_addr(wring);
    uint32_t aoff[4], woff[4];                      // byte offsets of this lane's DMA pieces at k = 0
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = 8 * j + (lane >> 3), q = (lane & 7) ^ f32_swz(row);
        aoff[j] = ((uint32_t)min(m0 + row, M - 1) * (uint32_t)K + 4u * q) * 4u;
        woff[j] = ((uint32_t)min(n0 + row, N - 1) * (uint32_t)K + 4u * q) * 4u;
    }
    auto issue = [&](int i) {                       // stage i of this wave into slot i % NS
        const uint32_t st = lring + (uint32_t)(i % NS) * 8192u, kb = (uint32_t)(s0 + i) * 128u;
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16s(A, aoff[j] + kb, st + 1024u * j);
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16s(W, woff[j] + kb, st + 4096u + 1024u * j);
    };
    f32x16_t acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
    for (int i = 0; i < NS - 1; ++i)
        if (i < n) issue(i);
    for (int i = 0; i < n; ++i) {
        if (i + NS - 1 < n) issue(i + NS - 1);     // into the slot of stage i - 1, read in the last iteration
        const int after = min(NS - 1, n - 1 - i);  // stages issued after stage i (8 DMA instructions each)
        if (after >= 3) QMM_VMWAIT(24);
        else if (after == 2) QMM_VMWAIT(16);
        else if (after == 1) QMM_VMWAIT(8);
        else QMM_VMWAIT(0);
        const uint8_t* st = wring + (size_t)(i % NS) * 8192;
        const int sw = f32_swz(fr);
        float4 av[4], wv[4];                        // the stage's fragments first, then its 16 MFMAs
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int slot = fr * 8 + ((4 * h + c) ^ sw);
            av[c] = *(const float4*)(st + 16 * slot);
            wv[c] = *(const float4*)(st + 4096 + 16 * slot);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[c].x, wv[c].x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[c].y, wv[c].y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[c].z, wv[c].z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[c].w, wv[c].w, acc, 0, 0, 0);
        }
    }
    __syncthreads();                                // every wave done with its ring: reuse it for the sums
    float* red = (float*)smem;
#pragma unroll
    for (int e = 0; e < 16; ++e) red[(wave * 16 + e) * 64 + lane] = acc[e];
    __syncthreads();
    const int nn = n0 + fr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = 4 * wave + i, o = e * 64 + lane;
        const float v = (red[o] + red[16 * 64 + o]) + (red[2 * 16 * 64 + o] + red[3 * 16 * 64 + o]);
        const int m = m0 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (m < M && nn < N) D[(size_t)m * N + nn] = v;
    }
}

constexpr int kF32dStages = 2;   // 64 KB of LDS per workgroup: two workgroups per CU (measured against 3 and 4)

}  // namespace
}  // namespace qmm

using namespace qmm;

extern "C" {

int qmm_f32_gemv(const float* W, const float* x, float* y, int N, int K, int T, void* stream) {
    if (!W || !x || !y) return QMM_ERR_NULL;
    if (N < 0 || T < 0 || K <= 0 || K % 4 != 0) return QMM_ERR_SHAPE;
    if (((reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(x)) & 15) != 0) return QMM_ERR_ARG;
    if (N == 0 || T == 0) return QMM_OK;
    // columns per pass: 1 for one token; 2 up to 8 tokens (8 steps in flight per lane; W is re-read
    // per pass, mostly from cache); 8 beyond (fewer W passes, 3 steps in flight)
    const int np = T == 1 ? 1 : (T <= 8 ? 2 : 8);
    const unsigned gx = (unsigned)((N + kGemvRowsPerBlock - 1) / kGemvRowsPerBlock);
    const unsigned gy = (unsigned)((T + np - 1) / np);
    if (gy > 65535u) return QMM_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    if (np == 1) hipLaunchKernelGGL((k_f32_gemv<1, 10>), dim3(gx, gy), dim3(64), 0, s, W, x, y, N, K, T);
    else if (np == 2) hipLaunchKernelGGL((k_f32_gemv<2, 8>), dim3(gx, gy), dim3(64), 0, s, W, x, y, N, K, T);
    else hipLaunchKernelGGL((k_f32_gemv<8, 3>), dim3(gx, gy), dim3(64), 0, s, W, x, y, N, K, T);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_gemm_f32(const float* A, const float* W, float* D, int M, int N, int K, void* stream) {
    if (!A || !W || !D) return QMM_ERR_NULL;
    if (M < 0 || N < 0 || K <= 0 || K % 4 != 0) return QMM_ERR_SHAPE;
    if (((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(W)) & 15) != 0) return QMM_ERR_ARG;
    if (M == 0 || N == 0) return QMM_OK;
    const long long nmt = (M + kFTile - 1) / kFTile, nnt = (N + kFTile - 1) / kFTile, total = nmt * nnt;
    if (total > 0x7fffffffLL) return QMM_ERR_SHAPE;
    const bool dma = K % 32 == 0 && (size_t)M * K * 4 <= 0xffffffffu && (size_t)N * K * 4 <= 0xffffffffu;
    if (dma)
        hipLaunchKernelGGL(k_gemm_f32d<kF32dStages>, dim3((unsigned)total), dim3(256), (size_t)kF32dStages * 4 * 8192,
                           (hipStream_t)stream, A, W, D, M, N, K, (int)nnt, (int)(total % 8 == 0));
    else
        hipLaunchKernelGGL(k_gemm_f32, dim3((unsigned)total), dim3(256), 0, (hipStream_t)stream, A, W, D, M, N, K, (int)nnt,
                           (int)(total % 8 == 0));
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_moe_router(const float* Wr, const float* x, float* logits, int* ids, float* w, int T, int nexp, int K, int topk,
                   void* stream) {
    if (!Wr || !x || !logits || !ids || !w) return QMM_ERR_NULL;
    // every check of both steps before the first launch (the routing's limits: 1024 experts, top-16)
    if (nexp < 1 || nexp > 1024 || topk < 1 || topk > 16 || topk > nexp || T < 0) return QMM_ERR_SHAPE;
    const int st = qmm_f32_gemv(Wr, x, logits, nexp + 1, K, T, stream);
    if (st != QMM_OK) return st;
    return qmm_moe_route_n(logits, ids, w, T, nexp, nexp + 1, topk, stream);
}

}  // extern "C"
