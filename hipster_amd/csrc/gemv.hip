// gemv.hip -- decode GEMV for GGUF Q4_K / Q6_K weights on gfx950 (wave64).
//
// Entry points (C ABI, include/hipster_qmm.h): qmm_quantize_x_q8, qmm_gemv_q8, qmm_gemv_multi,
// qmm_gemv_q4_K_f32.  Reference counterparts: engine/kernels/gemv.hip:36-51 (x quantiser),
// :291-321 + :1225-1242 + :1466-1485 (gemv_q8), :1042-1067 + :1355-1369 (gemv_multi),
// :1177-1216 + :1486-1489 (gemv_q4_K_f32).
//
// Q4_K kernel layout ("chunk-coalesced"): a row of nb superblocks is 9*nb 16-byte chunks
// (chunk 0 of a block = {d, dmin, scales[12]}, chunks 1..8 = qs).  One wave streams a row with
// lane l owning chunks l, l+64, l+128, ... so every weight load instruction reads 1 KiB of
// contiguous HBM.  A qs chunk (p = 1..8) holds 16 low nibbles of sub-block 2j and 16 high
// nibbles of sub-block 2j+1 (j = (p-1)/2, positions 16h..16h+15, h = (p-1)&1); its lane re-reads
// the block header from L1 (the same lines the wave just fetched) instead of shuffling it over.
// Activations are int8 (x quantised per 32), staged once per workgroup in LDS when they fit.
// The per-lane partial sums are reduced across the wave in a fixed butterfly order, so a
// column's result does not depend on how many columns the call carries (T-invariance).
#include "q4k_pair.hpp"
#include "qmm_common.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <string.h>

namespace qmm {
namespace {

constexpr int kBlock = 256;        // threads per workgroup (4 waves)
constexpr int kWavesPerBlock = kBlock / kWave;
#ifndef QMM_XLDS_BUDGET
#define QMM_XLDS_BUDGET (64 * 1024)
#endif
constexpr size_t kXLdsBudget = QMM_XLDS_BUDGET;   // bytes of LDS a workgroup may use for staged x
// x is loaded ahead of the weights (see k_gemv_q4k_q8) for ncol up to this value
#ifndef QMM_Q4K_XFIRST_NCOL
#define QMM_Q4K_XFIRST_NCOL 4
#endif

int g_cu_count = 0;
int device_cu_count() {
    if (g_cu_count == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_cu_count = n;
        else
            g_cu_count = 256;
    }
    return g_cu_count;
}

// ------------------------------------------------------------------------------------------
// x -> q8 per 32 (gemv.hip:36-51 semantics).  One 32-lane half-wave per 32-block.
__global__ void __launch_bounds__(256) k_quantize_x_q8(const float* __restrict__ x, int8_t* __restrict__ q,
                                                       float* __restrict__ d, float* __restrict__ s,
                                                       float2* __restrict__ ds, int K) {
    const int col = blockIdx.y;
    const int sb = blockIdx.x * 8 + (threadIdx.x >> 5), l = threadIdx.x & 31;
    if (sb * 32 >= K) return;
    const float v = x[(size_t)col * K + sb * 32 + l];
    float amax = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    const float dd = amax / 127.f, id = amax > 0.f ? 127.f / amax : 0.f;
    const int qi = __float2int_rn(v * id);
    int sum = qi;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 32);
    q[(size_t)col * K + sb * 32 + l] = (int8_t)qi;
    if (l == 0) {
        const size_t o = (size_t)col * (K / 32) + sb;
        d[o] = dd;
        s[o] = dd * (float)sum;
        if (ds) ds[o] = make_float2(dd, dd * (float)sum);
    }
}


// Q4_K weights sharing x and K in one launch (the reference's k_gemv_multi, gemv.hip:1042-1067):
// workgroup (16-row tile) i belongs to segment s when t0[s] <= i < t0[s + 1]
constexpr int kQSegMax = 4;
struct QSegs {
    const uint8_t* w[kQSegMax];
    float* y[kQSegMax];
    int N[kQSegMax];
    int t0[kQSegMax + 1];
    int nseg;
};

// ILOAD pair iterations per load batch; NITER > 0: the row is exactly NITER iterations and is
// loaded in one batch, with x staged from registers loaded ahead of the weights (XU units per
// thread); NITER == 0: any length, streamed in double-buffered batches of ILOAD.  The rows of every
// segment get the same arithmetic as alone.
template <int NCOL, int ILOAD, int NITER, bool XLDS>
__global__ void __launch_bounds__(kBlock) k_gemv_q4k_q8(QSegs sg, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                        const float* __restrict__ xs, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int XU = (NITER > 0 && XLDS && NCOL <= QMM_Q4K_XFIRST_NCOL) ? 2 * NCOL : 0;
    int si = 0;
#pragma unroll
    for (int i = 1; i < kQSegMax; ++i)
        if (i < sg.nseg && (int)blockIdx.x >= sg.t0[i]) si = i;
    const uint8_t* __restrict__ W = sg.w[si];
    float* __restrict__ y = sg.y[si];
    const int N = sg.N[si];
    const int nb = K >> 8, ntask = 4 * nb, nsb = K >> 5;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = lane & 15, j = t & 3;
    const int row = (((int)blockIdx.x - sg.t0[si]) * kWavesPerBlock + wave) * 4 + (lane >> 4);
    const uint8_t* rp = W + (size_t)min(row, N - 1) * ((size_t)nb * 144);
    Q4kPairs<ILOAD> A, B;
    XPairSrc<XLDS> xsrc[NCOL];
    if constexpr (XU > 0) {
        XStage<NCOL, (XU > 0 ? XU : 1)> S;
        stage_pairs_load<NCOL>(xq, xd, xs, K, S);         // x first (older loads) ...
        q4k_load_pairs<ILOAD>(rp, t, j, ntask, 0, A);     // ... then the weights
        stage_pairs_store<NCOL>(smem, K, S);              // waits for x only
        lds_barrier();                                    // not __syncthreads(): keeps the weight loads in flight
    } else {
        q4k_load_pairs<ILOAD>(rp, t, j, ntask, 0, A);
        if constexpr (XLDS) stage_xq8_pairs<NCOL>(smem, xq, xd, xs, K);
    }
    if constexpr (XLDS) {
#pragma unroll
        for (int c = 0; c < NCOL; ++c) xsrc[c] = XPairSrc<XLDS>{smem + (size_t)c * (K + (K >> 2)), nullptr, nullptr, K};
    } else {
#pragma unroll
        for (int c = 0; c < NCOL; ++c)
            xsrc[c] = XPairSrc<XLDS>{(const uint8_t*)(xq + (size_t)c * K), xd + (size_t)c * nsb, xs + (size_t)c * nsb, K};
    }
    const Q4kPairDecode dc(j);
    const bool exact = (nb & 3) == 0;
    float acc[NCOL];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = 0.f;
    if constexpr (NITER > 0) {
        if (exact) q4k_pairs_compute<NCOL, ILOAD, XLDS, true>(A, dc, t, ntask, 0, xsrc, acc);
        else q4k_pairs_compute<NCOL, ILOAD, XLDS, false>(A, dc, t, ntask, 0, xsrc, acc);
    } else {
        const int niter = (ntask + 15) >> 4, nbatch = (niter + ILOAD - 1) / ILOAD;
        const int lastb = (nbatch - 1) * ILOAD;
        for (int bi = 0; bi < nbatch; bi += 2) {
            q4k_load_pairs<ILOAD>(rp, t, j, ntask, min((bi + 1) * ILOAD, lastb), B);
            q4k_pairs_compute<NCOL, ILOAD, XLDS, false>(A, dc, t, ntask, bi * ILOAD, xsrc, acc);
            q4k_load_pairs<ILOAD>(rp, t, j, ntask, min((bi + 2) * ILOAD, lastb), A);
            if (bi + 1 < nbatch) q4k_pairs_compute<NCOL, ILOAD, XLDS, false>(B, dc, t, ntask, (bi + 1) * ILOAD, xsrc, acc);
        }
    }
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = group_sum(acc[c], 16);
    if (t == 0 && row < N) {
#pragma unroll
        for (int c = 0; c < NCOL; ++c) y[(size_t)c * N + row] = acc[c];
    }
}

// f32 x in, q8 arithmetic: the q8 quantisation of x fused into the staging of k_gemv_q4k_q8 (x
// loaded ahead of the weights and quantised while they stream in), so quantize_x_q8 + gemv_q8 is
// one launch with bit-identical results.  Rows of NITER pair iterations (K <= 1024 * NITER).
// BS threads (BS/64 waves of 4 rows): the per-lane work is the same for any BS; a larger workgroup
// stages (and quantises) x once for more rows.
template <int NCOL, int NITER, int BS>
__global__ void __launch_bounds__(BS) k_gemv_q4k_fx(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                    float* __restrict__ y, int N, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int nb = K >> 8, ntask = 4 * nb;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = lane & 15, j = t & 3;
    const int row = (blockIdx.x * (BS / 64) + wave) * 4 + (lane >> 4);
    const uint8_t* rp = W + (size_t)min(row, N - 1) * ((size_t)nb * 144);
    Q4kPairs<NITER> A;
    {
        XStageF<NCOL, (128 * NCOL * NITER + BS - 1) / BS> S;   // NCOL * K/8 <= 128 * NCOL * NITER slots
        stagef_load<NCOL, (128 * NCOL * NITER + BS - 1) / BS, BS>(x, K, S);   // x first (older loads) ...
        q4k_load_pairs<NITER>(rp, t, j, ntask, 0, A);     // ... then the weights
        stagef_store<NCOL, (128 * NCOL * NITER + BS - 1) / BS, BS>(smem, K, S);   // quantise while the weights stream in
        lds_barrier();
    }
    XPairSrc<true> xsrc[NCOL];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) xsrc[c] = XPairSrc<true>{smem + (size_t)c * (K + (K >> 2)), nullptr, nullptr, K};
    const Q4kPairDecode dc(j);
    float acc[NCOL];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = 0.f;
    if ((nb & 3) == 0) q4k_pairs_compute<NCOL, NITER, true, true>(A, dc, t, ntask, 0, xsrc, acc);
    else q4k_pairs_compute<NCOL, NITER, true, false>(A, dc, t, ntask, 0, xsrc, acc);
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = group_sum(acc[c], 16);
    if (t == 0 && row < N) {
#pragma unroll
        for (int c = 0; c < NCOL; ++c) y[(size_t)c * N + row] = acc[c];
    }
}

// ------------------------------------------------------------------------------------------
// Q6_K x int8 GEMV, one superblock per lane, TPR lanes per row (TPR fixed per tensor shape).
// F = QMM_Q6_K (GGUF 210-byte blocks, 2-byte aligned) or QMM_Q6_K_SOA (row streams).
// The 208 bytes {ql, qh, scales} of a GGUF block are read as 13 dword-aligned 16-byte loads
// starting at the dword below the block and realigned by 0 or 2 bytes; d is read on its own.
struct Q6Parts { uint32_t ql[32], qh[16], sc[4]; float d; };

template <int F>
__device__ __forceinline__ void q6k_load(const uint8_t* __restrict__ rp, int b, int nb, Q6Parts& o) {
    if constexpr (F == QMM_Q6_K) {
        const uint8_t* blk = rp + (size_t)b * 210;
        const uintptr_t addr = (uintptr_t)blk;
        const uint32_t sh = (uint32_t)(addr & 3u);
        const uint8_t* base = (const uint8_t*)(addr & ~(uintptr_t)3);
        uint32_t raw[53];
#pragma unroll
        for (int i = 0; i < 13; ++i) {
            const uint4 v = ld16_a4(base + 16 * i);
            raw[4 * i] = v.x; raw[4 * i + 1] = v.y; raw[4 * i + 2] = v.z; raw[4 * i + 3] = v.w;
        }
        // bytes 206..209 of the block when it starts 2 bytes into a dword; else only d at 208
        raw[52] = sh ? *(const uint32_t*)(base + 208) : (uint32_t)(*(const uint16_t*)(blk + 208)) << 16;
        uint32_t al[52];
#pragma unroll
        for (int i = 0; i < 52; ++i) al[i] = alignbyte(raw[i + 1], raw[i], sh);
#pragma unroll
        for (int i = 0; i < 32; ++i) o.ql[i] = al[i];
#pragma unroll
        for (int i = 0; i < 16; ++i) o.qh[i] = al[32 + i];
#pragma unroll
        for (int i = 0; i < 4; ++i) o.sc[i] = al[48 + i];
        // d = bytes 208..209 of the block: the top half of raw[52] in both cases
        o.d = h2f(raw[52] >> 16);
    } else {
        const uint8_t* ql = rp + (size_t)b * 128;
        const uint8_t* qh = rp + (size_t)nb * 128 + (size_t)b * 64;
        const uint8_t* sc = rp + (size_t)nb * 192 + (size_t)b * 16;
        const uint16_t* dp = (const uint16_t*)(rp + (size_t)nb * 208) + b;
#pragma unroll
        for (int i = 0; i < 8; ++i) { const uint4 v = ld16_a4(ql + 16 * i); o.ql[4 * i] = v.x; o.ql[4 * i + 1] = v.y; o.ql[4 * i + 2] = v.z; o.ql[4 * i + 3] = v.w; }
#pragma unroll
        for (int i = 0; i < 4; ++i) { const uint4 v = ld16_a4(qh + 16 * i); o.qh[4 * i] = v.x; o.qh[4 * i + 1] = v.y; o.qh[4 * i + 2] = v.z; o.qh[4 * i + 3] = v.w; }
        const uint4 v = ld16_a4(sc);
        o.sc[0] = v.x; o.sc[1] = v.y; o.sc[2] = v.z; o.sc[3] = v.w;
        o.d = h2f(*dp);
    }
}

// sum over the 256 weights of a Q6_K block against int8 x (x words xw[64], scales xd[8])
__device__ __forceinline__ float q6k_dot_q8(const Q6Parts& P, const uint32_t* xw, const float* xdv) {
    float acc = 0.f;
#pragma unroll
    for (int n = 0; n < 2; ++n) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            int isum[2] = {0, 0};
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                const uint32_t A = P.ql[16 * n + w], B = P.ql[16 * n + 8 + w], Hh = P.qh[8 * n + w];
                uint32_t q;
                if (g == 0) q = (A & 0x0f0f0f0fu) | ((Hh << 4) & 0x30303030u);
                else if (g == 1) q = (B & 0x0f0f0f0fu) | ((Hh << 2) & 0x30303030u);
                else if (g == 2) q = ((A >> 4) & 0x0f0f0f0fu) | (Hh & 0x30303030u);
                else q = ((B >> 4) & 0x0f0f0f0fu) | ((Hh >> 2) & 0x30303030u);
                isum[w >> 2] = sdot4(q6_signed(q), xw[32 * n + 8 * g + w], isum[w >> 2]);
            }
            const int s16 = 8 * n + 2 * g;   // scale index of the first 16 of this 32-run
            const int sa = (int)(int8_t)((P.sc[s16 >> 2] >> (8 * (s16 & 3))) & 0xffu);
            const int sbv = (int)(int8_t)((P.sc[(s16 + 1) >> 2] >> (8 * ((s16 + 1) & 3))) & 0xffu);
            acc += P.d * xdv[4 * n + g] * (float)(sa * isum[0] + sbv * isum[1]);
        }
    }
    return acc;
}

template <int F, int NCOL, int TPR, bool XLDS>
__global__ void __launch_bounds__(kBlock) k_gemv_q6k_q8(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                        const float* __restrict__ xd, const float* __restrict__ xs,
                                                        float* __restrict__ y, int N, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int ROWS = kBlock / TPR;
    const int nb = K >> 8, nsb = K >> 5;
    const size_t rb = (size_t)nb * 210;
    const int8_t* xq_s = xq; const float* xd_s = xd;
    if constexpr (XLDS) {
        stage_xq8<NCOL>(smem, xq, xd, xs, K);
        xq_s = (const int8_t*)smem;
        xd_s = (const float*)(smem + (size_t)NCOL * K);
    }
    const int lane = threadIdx.x % TPR, r = threadIdx.x / TPR;
    const int nrb = (N + ROWS - 1) / ROWS;
    for (int vb = blockIdx.x; vb < nrb; vb += gridDim.x) {
        const int row = vb * ROWS + r;
        float acc[NCOL];
#pragma unroll
        for (int c = 0; c < NCOL; ++c) acc[c] = 0.f;
        if (row < N) {
            const uint8_t* rp = W + (size_t)row * rb;
            for (int b = lane; b < nb; b += TPR) {
                Q6Parts P;
                q6k_load<F>(rp, b, nb, P);
#pragma unroll
                for (int c = 0; c < NCOL; ++c) {
                    uint32_t xw[64];
                    const uint4* xp = (const uint4*)(xq_s + (size_t)c * K + (size_t)b * 256);
#pragma unroll
                    for (int i = 0; i < 16; ++i) { const uint4 v = xp[i]; xw[4 * i] = v.x; xw[4 * i + 1] = v.y; xw[4 * i + 2] = v.z; xw[4 * i + 3] = v.w; }
                    float xdv[8];
                    const float4 d0 = *(const float4*)(xd_s + (size_t)c * nsb + 8 * b), d1 = *(const float4*)(xd_s + (size_t)c * nsb + 8 * b + 4);
                    xdv[0] = d0.x; xdv[1] = d0.y; xdv[2] = d0.z; xdv[3] = d0.w; xdv[4] = d1.x; xdv[5] = d1.y; xdv[6] = d1.z; xdv[7] = d1.w;
                    acc[c] += q6k_dot_q8(P, xw, xdv);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < NCOL; ++c) acc[c] = group_sum(acc[c], TPR);
        if (row < N && lane == 0) {
#pragma unroll
            for (int c = 0; c < NCOL; ++c) y[(size_t)c * N + row] = acc[c];
        }
    }
}

// ------------------------------------------------------------------------------------------
// Q6_K x int8 GEMV, "unit" mapping: one row per wave, a lane owns quarter blocks.  Quarter
// (n, lh) of a block (engine/src/quant.h:65-80: for half n, l < 32, the four weights 128n + l +
// {0, 32, 64, 96} come from ql[64n + l] (low / high nibble), ql[64n + 32 + l] and qh[32n + l] bits
// {0-1, 2-3, 4-5, 6-7}) takes l = 16lh .. 16lh+15: 16 bytes of ql run A, 16 of ql run B, 16 of qh,
// scales sc[8n + lh + {0, 2, 4, 6}] and d -- 64 weights, every byte of the block read once.  Unit
// u = 4b + 2n + lh; lane l takes units l, l + 64, ... (all of them loaded before any compute).
// x (q8) is staged per workgroup in LDS transposed for this order: the 16 x of group g of unit u
// (x[256b + 128n + 32g + 16lh ..]) at (g * K/64 + u) * 16, and the four q8 scales the unit needs
// (d of q8 blocks 8b + 4n + g) as a float4 at K + 16u.  Per group: isum = sum (q - 32) * xq over 16
// (v_dot4), acc += (d * xd) * (float)(sc * isum).
struct Q6Unit { uint4 a, b, h; uint32_t sc0, sc1; float d; };

template <int F>
__device__ __forceinline__ void q6k_load_unit(const uint8_t* __restrict__ rp, int nb, int u, Q6Unit& o) {
    const int b = u >> 2, n = (u >> 1) & 1, lh = u & 1;
    if constexpr (F == QMM_Q6_K_SOA) {
        const uint8_t* ql = rp + (size_t)b * 128 + 64 * n + 16 * lh;
        o.a = ld16_a4(ql);
        o.b = ld16_a4(ql + 32);
        o.h = ld16_a4(rp + (size_t)nb * 128 + (size_t)b * 64 + 32 * n + 16 * lh);
        const u32x2_a4 sc = *(const u32x2_a4*)(rp + (size_t)nb * 192 + (size_t)b * 16 + 8 * n);
        o.sc0 = sc.x; o.sc1 = sc.y;
        o.d = h2f(*(const uint16_t*)(rp + (size_t)nb * 208 + 2 * b));
    } else {
        // 210-byte blocks start 0 or 2 bytes into a dword: dword-aligned loads, realigned by sh
        const uintptr_t addr = (uintptr_t)(rp + (size_t)b * 210);
        const uint32_t sh = (uint32_t)(addr & 3u);
        const uint8_t* base = (const uint8_t*)(addr & ~(uintptr_t)3);
        auto piece = [&](int off) {
            const uint4 v = ld16_a4(base + off);
            const uint32_t e = *(const uint32_t*)(base + off + 16);
            return make_uint4(alignbyte(v.y, v.x, sh), alignbyte(v.z, v.y, sh), alignbyte(v.w, v.z, sh), alignbyte(e, v.w, sh));
        };
        o.a = piece(64 * n + 16 * lh);
        o.b = piece(64 * n + 32 + 16 * lh);
        o.h = piece(128 + 32 * n + 16 * lh);
        const uint4 sc = ld16_a4(base + 192 + 8 * n);             // bytes 192+8n .. +15 (+sh)
        o.sc0 = alignbyte(sc.y, sc.x, sh);
        o.sc1 = alignbyte(sc.z, sc.y, sh);
        // d = bytes 208..209: the top half of the dword at 208 when sh = 2, else the bottom of 208
        const uint32_t dw = *(const uint32_t*)(base + 208);
        o.d = h2f(sh ? dw >> 16 : dw);
    }
}

// stage q8 x of nc columns in the unit-transposed layout (column c at c * 5K/4)
__device__ __forceinline__ void stage_xq8_q6units(uint8_t* lds, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                  int K, int nc) {
    const int U = K >> 6, nx = U * 4, nsb = K >> 5;
    for (int v = threadIdx.x; v < nc * nx; v += blockDim.x) {
        const int c = v / nx, r = v - c * nx, g = r / U, u = r - g * U;
        const int b = u >> 2, n = (u >> 1) & 1, lh = u & 1;
        *(uint4*)(lds + (size_t)c * (K + (K >> 2)) + (size_t)(g * U + u) * 16) =
            ld16(xq + (size_t)c * K + (size_t)b * 256 + 128 * n + 32 * g + 16 * lh);
    }
    for (int v = threadIdx.x; v < nc * U; v += blockDim.x) {
        const int c = v / U, u = v - c * U;
        const int b = u >> 2, n = (u >> 1) & 1;
        *(float4*)(lds + (size_t)c * (K + (K >> 2)) + (size_t)K + (size_t)u * 16) =
            *(const float4*)(xd + (size_t)c * nsb + 8 * b + 4 * n);
    }
    __syncthreads();
}

// x-first staging of the first pass (nc <= 2 columns): the x units are loaded into registers before
// the weight loads are issued and written to LDS after, so waiting for x does not wait for the
// weights (vmcnt retires in issue order).  Unit v < nc*4U: 16 x bytes of (column, group g, unit u);
// above: the q8 scale float4 of (column, unit).
template <int UX>
struct XQ6Stage { uint4 v[UX]; };

template <int UX>
__device__ __forceinline__ void q6x_load(const int8_t* __restrict__ xq, const float* __restrict__ xd, int K, int nc,
                                         XQ6Stage<UX>& S) {
    const int U = K >> 6, nx = 4 * U, nq = nc * nx, nt = nq + nc * U, nsb = K >> 5;
#pragma unroll
    for (int k = 0; k < UX; ++k) {
        const int v = min((int)threadIdx.x + kBlock * k, nt - 1);
        if (v < nq) {
            const int c = v / nx, r = v - c * nx, g = r / U, u = r - g * U;
            S.v[k] = ld16(xq + (size_t)c * K + (size_t)(u >> 2) * 256 + 128 * ((u >> 1) & 1) + 32 * g + 16 * (u & 1));
        } else {
            const int w = v - nq, c = w / U, u = w - c * U;
            const float4 f = *(const float4*)(xd + (size_t)c * nsb + 8 * (u >> 2) + 4 * ((u >> 1) & 1));
            S.v[k] = make_uint4(__float_as_uint(f.x), __float_as_uint(f.y), __float_as_uint(f.z), __float_as_uint(f.w));
        }
    }
}
template <int UX>
__device__ __forceinline__ void q6x_store(uint8_t* lds, int K, int nc, const XQ6Stage<UX>& S) {
    const int U = K >> 6, nx = 4 * U, nq = nc * nx, nt = nq + nc * U;
#pragma unroll
    for (int k = 0; k < UX; ++k) {
        const int v = (int)threadIdx.x + kBlock * k;
        if (v >= nt) continue;
        size_t off;
        if (v < nq) {
            const int c = v / nx, r = v - c * nx, g = r / U, u = r - g * U;
            off = (size_t)c * (K + (K >> 2)) + (size_t)(g * U + u) * 16;
        } else {
            const int w = v - nq, c = w / U, u = w - c * U;
            off = (size_t)c * (K + (K >> 2)) + (size_t)K + (size_t)u * 16;
        }
        *(uint4*)(lds + off) = S.v[k];
    }
}

// Columns are staged and computed in passes of cpp (what the LDS budget holds); the weights are
// loaded once, and every column gets the same arithmetic whatever NCOL and cpp are.
template <int F, int NCOL, int NIT>
__global__ void __launch_bounds__(kBlock) k_gemv_q6k_u(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                       const float* __restrict__ xd, float* __restrict__ y, int N, int K, int cpp) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int nb = K >> 8, U = K >> 6, nsb = K >> 5;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = blockIdx.x * kWavesPerBlock + wave;
    const uint8_t* rp = W + (size_t)min(row, N - 1) * ((size_t)nb * 210);
    Q6Unit P[NIT];
    if constexpr (NCOL <= 2) {
        // K <= 4096 NIT: (4U + U) * NCOL / 256 <= 1.25 NIT NCOL units per thread
        XQ6Stage<(5 * NIT * NCOL + 3) / 4> S;
        q6x_load(xq, xd, K, min(cpp, NCOL), S);              // x first (older loads) ...
#pragma unroll
        for (int i = 0; i < NIT; ++i) q6k_load_unit<F>(rp, nb, min(lane + 64 * i, U - 1), P[i]);   // ... then the weights
        q6x_store(smem, K, min(cpp, NCOL), S);               // waits for x only
        lds_barrier();
    } else {
        stage_xq8_q6units(smem, xq, xd, K, min(cpp, NCOL));
#pragma unroll
        for (int i = 0; i < NIT; ++i) q6k_load_unit<F>(rp, nb, min(lane + 64 * i, U - 1), P[i]);
    }
    float acc[NCOL];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = 0.f;
    for (int c0 = 0; c0 < NCOL; c0 += cpp) {
        if (c0 > 0) {
            __syncthreads();                                   // the previous pass's x reads are done
            stage_xq8_q6units(smem, xq + (size_t)c0 * K, xd + (size_t)c0 * nsb, K, min(cpp, NCOL - c0));
        }
#pragma unroll
        for (int i = 0; i < NIT; ++i) {
            const int u = lane + 64 * i, uc = min(u, U - 1), lh = uc & 1;
            const Q6Unit& q = P[i];
            const uint32_t A[4] = {q.a.x, q.a.y, q.a.z, q.a.w}, B[4] = {q.b.x, q.b.y, q.b.z, q.b.w}, H[4] = {q.h.x, q.h.y, q.h.z, q.h.w};
            // scales sc[lh + 2g], g = 0..3, of the unit's 8-byte scale run {sc0, sc1}: bytes lh, lh+2,
            // lh+4, lh+6 gathered with one byte permute
            const uint32_t scr = __builtin_amdgcn_perm(q.sc1, q.sc0, lh ? 0x07050301u : 0x06040200u);
            uint32_t qw[4][4];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                qw[0][w] = q6_signed((A[w] & 0x0f0f0f0fu) | ((H[w] << 4) & 0x30303030u));
                qw[1][w] = q6_signed((B[w] & 0x0f0f0f0fu) | ((H[w] << 2) & 0x30303030u));
                qw[2][w] = q6_signed(((A[w] >> 4) & 0x0f0f0f0fu) | (H[w] & 0x30303030u));
                qw[3][w] = q6_signed(((B[w] >> 4) & 0x0f0f0f0fu) | ((H[w] >> 2) & 0x30303030u));
            }
#pragma unroll
            for (int c = 0; c < NCOL; ++c) {
                if (c < c0 || c >= c0 + cpp) continue;
                const uint8_t* xc = smem + (size_t)(c - c0) * (K + (K >> 2));
                const float4 xs4 = *(const float4*)(xc + (size_t)K + (size_t)uc * 16);
                const float xsg[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
                float v = 0.f;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const uint4 xv = *(const uint4*)(xc + (size_t)(g * U + uc) * 16);
                    int is = sdot4(qw[g][0], xv.x, 0);
                    is = sdot4(qw[g][1], xv.y, is);
                    is = sdot4(qw[g][2], xv.z, is);
                    is = sdot4(qw[g][3], xv.w, is);
                    const int scg = (int)(int8_t)((scr >> (8 * g)) & 0xffu);
                    v = __builtin_fmaf(q.d * xsg[g], (float)(scg * is), v);
                }
                acc[c] += u < U ? v : 0.f;
            }
        }
    }
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = wave_sum(acc[c]);
    if (lane == 0 && row < N) {
#pragma unroll
        for (int c = 0; c < NCOL; ++c) y[(size_t)c * N + row] = acc[c];
    }
}

// Several columns at once (NCOL >= 5): x of all NCOL columns staged once per workgroup of 16 rows
// (1024 threads, one row per wave, so the x copy is paid once per 16 rows instead of once per 4 rows
// and per pass of k_gemv_q6k_u's 64 KiB budget).  Column c at c * 9K/8: the x units as k_gemv_q6k_u
// lays them out, then its q8 scales d as they are in memory (the float4 of unit u is the one of unit
// pair u / 2, at K + 16 (u / 2)).  Same per-lane arithmetic and reduction as k_gemv_q6k_u, so every
// column is bitwise the one-column kernel's.  Needs NCOL * 9K/8 bytes of LDS.
constexpr int kQ6WideWaves = 16;
inline size_t q6w_lds_bytes(int ncol, int K) { return (size_t)ncol * ((size_t)K + K / 8); }

template <int F, int NCOL, int NIT>
__global__ void __launch_bounds__(64 * kQ6WideWaves) k_gemv_q6k_w(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                                  const float* __restrict__ xd, float* __restrict__ y, int N, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int nb = K >> 8, U = K >> 6, nsb = K >> 5, ccol = K + (K >> 3);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = blockIdx.x * kQ6WideWaves + wave;
    const uint8_t* rp = W + (size_t)min(row, N - 1) * ((size_t)nb * 210);
    Q6Unit P[NIT];
#pragma unroll
    for (int i = 0; i < NIT; ++i) q6k_load_unit<F>(rp, nb, min(lane + 64 * i, U - 1), P[i]);   // weights first
    {
        const int nx = 4 * U;
        for (int v = threadIdx.x; v < NCOL * nx; v += 64 * kQ6WideWaves) {
            const int c = v / nx, r = v - c * nx, g = r / U, u = r - g * U;
            const int b = u >> 2, n = (u >> 1) & 1, lh = u & 1;
            *(uint4*)(smem + (size_t)c * ccol + (size_t)(g * U + u) * 16) =
                ld16(xq + (size_t)c * K + (size_t)b * 256 + 128 * n + 32 * g + 16 * lh);
        }
        const int nd = nsb >> 2;                                    // float4 of d per column
        for (int v = threadIdx.x; v < NCOL * nd; v += 64 * kQ6WideWaves) {
            const int c = v / nd, w = v - c * nd;
            *(float4*)(smem + (size_t)c * ccol + (size_t)K + (size_t)w * 16) = *(const float4*)(xd + (size_t)c * nsb + 4 * w);
        }
    }
    lds_barrier();
    float acc[NCOL];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = 0.f;
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
        const int u = lane + 64 * i, uc = min(u, U - 1), lh = uc & 1;
        const Q6Unit& q = P[i];
        const uint32_t A[4] = {q.a.x, q.a.y, q.a.z, q.a.w}, B[4] = {q.b.x, q.b.y, q.b.z, q.b.w}, H[4] = {q.h.x, q.h.y, q.h.z, q.h.w};
        const uint32_t scr = __builtin_amdgcn_perm(q.sc1, q.sc0, lh ? 0x07050301u : 0x06040200u);
        uint32_t qw[4][4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            qw[0][w] = q6_signed((A[w] & 0x0f0f0f0fu) | ((H[w] << 4) & 0x30303030u));
            qw[1][w] = q6_signed((B[w] & 0x0f0f0f0fu) | ((H[w] << 2) & 0x30303030u));
            qw[2][w] = q6_signed(((A[w] >> 4) & 0x0f0f0f0fu) | (H[w] & 0x30303030u));
            qw[3][w] = q6_signed(((B[w] >> 4) & 0x0f0f0f0fu) | ((H[w] >> 2) & 0x30303030u));
        }
#pragma unroll
        for (int c = 0; c < NCOL; ++c) {
            const uint8_t* xc = smem + (size_t)c * ccol;
            const float4 xs4 = *(const float4*)(xc + (size_t)K + (size_t)(uc >> 1) * 16);
            const float xsg[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
            float v = 0.f;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint4 xv = *(const uint4*)(xc + (size_t)(g * U + uc) * 16);
                int is = sdot4(qw[g][0], xv.x, 0);
                is = sdot4(qw[g][1], xv.y, is);
                is = sdot4(qw[g][2], xv.z, is);
                is = sdot4(qw[g][3], xv.w, is);
                const int scg = (int)(int8_t)((scr >> (8 * g)) & 0xffu);
                v = __builtin_fmaf(q.d * xsg[g], (float)(scg * is), v);
            }
            acc[c] += u < U ? v : 0.f;
        }
    }
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = wave_sum(acc[c]);
    if (lane == 0 && row < N) {
#pragma unroll
        for (int c = 0; c < NCOL; ++c) y[(size_t)c * N + row] = acc[c];
    }
}

// ------------------------------------------------------------------------------------------
// Q4_K x f32 GEMV (gemv.hip:1177-1216 semantics): acc += dA*sum(x*qA) + dB*sum(x*qB) - the min
// terms once per sub-block, with f32 x and per-sub-block sums of x staged in LDS when they fit.
// Same chunk-coalesced weight stream as k_gemv_q4k_q8.
template <int NCOL, bool XLDS>
__global__ void __launch_bounds__(kBlock) k_gemv_q4k_f32(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                         float* __restrict__ y, int N, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int nb = K >> 8, C = 9 * nb, nsb = K >> 5;
    const size_t rb = (size_t)nb * 144;
    // xsum[c][sb] = sum of the 32 x of sub-block sb (sequential order); x itself from LDS or global
    float* xsum = (float*)smem;
    const float* xs_src = x;
    if constexpr (XLDS) {
        float* xl = xsum + NCOL * nsb;
        for (int i = threadIdx.x; i < NCOL * K / 4; i += blockDim.x) ((float4*)xl)[i] = ((const float4*)x)[i];
        xs_src = xl;
    }
    for (int i = threadIdx.x; i < NCOL * nsb; i += blockDim.x) {
        const float* p = x + (size_t)i * 32;
        float s = 0.f;
        for (int l = 0; l < 32; ++l) s += p[l];
        xsum[i] = s;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = (int)((long long)N * blockIdx.x / gridDim.x), r1 = (int)((long long)N * (blockIdx.x + 1) / gridDim.x);
    const int nci = (C + 63) >> 6;
    for (int row = r0 + wave; row < r1; row += kWavesPerBlock) {
        const uint8_t* rp = W + (size_t)row * rb;
        float acc[NCOL];
#pragma unroll
        for (int c = 0; c < NCOL; ++c) acc[c] = 0.f;
        for (int i = 0; i < nci; ++i) {
            const int cidx = lane + 64 * i;
            if (cidx >= C) break;
            const int b = cidx / 9, p = cidx - 9 * b;
            const uint4 w = ld16(rp + (size_t)cidx * 16);
            if (p == 0) continue;
            const uint4 hd = ld16(rp + (size_t)b * 144);
            const int j = (p - 1) >> 1, h = (p - 1) & 1;
            const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
            const Q4kScaleBytes sb = q4k_scale_bytes(hd.y, hd.z, hd.w);
            const float dA = d * (float)byte8(sb.sc_lo, sb.sc_hi, 2 * j), dB = d * (float)byte8(sb.sc_lo, sb.sc_hi, 2 * j + 1);
            const float mA = dmin * (float)byte8(sb.m_lo, sb.m_hi, 2 * j), mB = dmin * (float)byte8(sb.m_lo, sb.m_hi, 2 * j + 1);
            const uint32_t wq[4] = {w.x, w.y, w.z, w.w};
            const int kA = 256 * b + 64 * j + 16 * h, sA = 8 * b + 2 * j;
#pragma unroll
            for (int c = 0; c < NCOL; ++c) {
                const float* xa = xs_src + (size_t)c * K + kA;
                float sa = 0.f, sbv = 0.f;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 va = *(const float4*)(xa + 4 * q), vb = *(const float4*)(xa + 32 + 4 * q);
                    const uint32_t wv = wq[q];
                    sa += va.x * (float)(wv & 15u) + va.y * (float)((wv >> 8) & 15u) + va.z * (float)((wv >> 16) & 15u) + va.w * (float)((wv >> 24) & 15u);
                    sbv += vb.x * (float)((wv >> 4) & 15u) + vb.y * (float)((wv >> 12) & 15u) + vb.z * (float)((wv >> 20) & 15u) + vb.w * (float)((wv >> 28) & 15u);
                }
                float a = dA * sa + dB * sbv;
                if (h == 0) a -= mA * xsum[c * nsb + sA] + mB * xsum[c * nsb + sA + 1];
                acc[c] += a;
            }
        }
#pragma unroll
        for (int c = 0; c < NCOL; ++c) acc[c] = wave_sum(acc[c]);
        if (lane == 0) {
#pragma unroll
            for (int c = 0; c < NCOL; ++c) y[(size_t)c * N + row] = acc[c];
        }
    }
}

// ------------------------------------------------------------------------------------------
// host launchers
inline size_t xq8_lds_bytes(int ncol, int K) { return (size_t)ncol * K + 2 * (size_t)ncol * (K / 32) * 4; }

// workgroups for the persistent row-range kernels: enough to give every CU several waves, never
// more than one row per wave
inline int persistent_grid(int N) {
    const int want = device_cu_count() * 4;
    const int maxg = (N + kWavesPerBlock - 1) / kWavesPerBlock;
    return want < maxg ? want : maxg;
}

// Launch shape of the Q4_K kernel: 16 rows per workgroup, the row loaded in one batch when it is
// at most 6 pair iterations (K <= 6144), else streamed in double-buffered batches of 4.  It
// depends on (N, K) only, never on ncol (T-invariance).  x goes to LDS when NCOL columns fit in
// kXLdsBudget (5K/4 bytes per column).
template <int NCOL, int ILOAD, int NITER>
int launch_q4k_q8_i(const QSegs& sg, qmm_xq8 x, int K, hipStream_t s) {
    const size_t lds = (size_t)NCOL * (K + K / 4);
    const int grid = sg.t0[sg.nseg];
    if (lds <= kXLdsBudget)
        hipLaunchKernelGGL((k_gemv_q4k_q8<NCOL, ILOAD, NITER, true>), dim3(grid), dim3(kBlock), lds, s, sg, x.q, x.d, x.s, K);
    else
        hipLaunchKernelGGL((k_gemv_q4k_q8<NCOL, ILOAD, NITER, false>), dim3(grid), dim3(kBlock), 0, s, sg, x.q, x.d, x.s, K);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

template <int NCOL>
int launch_q4k_q8_segs(const QSegs& sg, qmm_xq8 x, int K, hipStream_t s) {
    switch ((K / 256 * 4 + 15) / 16) {   // pair iterations per lane
        case 1: return launch_q4k_q8_i<NCOL, 1, 1>(sg, x, K, s);
        case 2: return launch_q4k_q8_i<NCOL, 2, 2>(sg, x, K, s);
        case 3: return launch_q4k_q8_i<NCOL, 3, 3>(sg, x, K, s);
        case 4: return launch_q4k_q8_i<NCOL, 4, 4>(sg, x, K, s);
        case 5: return launch_q4k_q8_i<NCOL, 5, 5>(sg, x, K, s);
        case 6: return launch_q4k_q8_i<NCOL, 6, 6>(sg, x, K, s);
        default: return launch_q4k_q8_i<NCOL, 4, 0>(sg, x, K, s);
    }
}

// segments (Q4_K, one K) as a tile table
inline QSegs q4k_segs(const qmm_gemv_seg* segs, int nseg, int c0) {
    QSegs sg = {};
    sg.nseg = nseg;
    for (int i = 0; i < nseg; ++i) {
        sg.w[i] = (const uint8_t*)segs[i].w;
        sg.y[i] = segs[i].y + (size_t)c0 * segs[i].N;
        sg.N[i] = segs[i].N;
        sg.t0[i + 1] = sg.t0[i] + (segs[i].N + 4 * kWavesPerBlock - 1) / (4 * kWavesPerBlock);
    }
    return sg;
}

template <int NCOL>
int launch_q4k_q8(const void* W, qmm_xq8 x, float* y, int N, int K, hipStream_t s) {
    const qmm_gemv_seg seg = {QMM_Q4_K, W, y, N, K};
    return launch_q4k_q8_segs<NCOL>(q4k_segs(&seg, 1, 0), x, K, s);
}

// ncol (1..8) columns against nseg Q4_K segments sharing x and K on the dot4 kernel, one launch
int gemv_q4k_q8_multi(const qmm_gemv_seg* segs, int nseg, qmm_xq8 x, int K, int ncol, int c0, hipStream_t s) {
    const QSegs sg = q4k_segs(segs, nseg, c0);
    switch (ncol) {
        case 1: return launch_q4k_q8_segs<1>(sg, x, K, s);
        case 2: return launch_q4k_q8_segs<2>(sg, x, K, s);
        case 3: return launch_q4k_q8_segs<3>(sg, x, K, s);
        case 4: return launch_q4k_q8_segs<4>(sg, x, K, s);
        case 5: return launch_q4k_q8_segs<5>(sg, x, K, s);
        case 6: return launch_q4k_q8_segs<6>(sg, x, K, s);
        case 7: return launch_q4k_q8_segs<7>(sg, x, K, s);
        case 8: return launch_q4k_q8_segs<8>(sg, x, K, s);
        default: return QMM_ERR_SHAPE;
    }
}

// 256 threads: measured against 320, 384 and 512 (12.6 vs 15.5-16.8 us at 17408 x 5120, M=1)
template <int NCOL>
int launch_q4k_fx(const void* W, const float* x, float* y, int N, int K, hipStream_t s) {
    constexpr int BS = kBlock, ROWS = 4 * (BS / 64);
    const size_t lds = (size_t)NCOL * (K + K / 4);
    const int grid = (N + ROWS - 1) / ROWS;
#define QMM_FX(IV) case IV: hipLaunchKernelGGL((k_gemv_q4k_fx<NCOL, IV, BS>), dim3(grid), dim3(BS), lds, s, (const uint8_t*)W, x, y, N, K); break;
    switch ((K / 256 * 4 + 15) / 16) {
        QMM_FX(1) QMM_FX(2) QMM_FX(3) QMM_FX(4) QMM_FX(5) QMM_FX(6)
        default: return QMM_ERR_SHAPE;
    }
#undef QMM_FX
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

// lanes per row for the Q6_K kernel: a function of K only (never of ncol)
inline int q6k_tpr(int K) { const int nb = K / 256; return nb >= 32 ? 8 : nb >= 8 ? 4 : nb >= 2 ? 2 : 1; }

template <int F, int NCOL, int TPR>
int launch_q6k_q8_t(const void* W, qmm_xq8 x, float* y, int N, int K, hipStream_t s) {
    constexpr int ROWS = kBlock / TPR;
    const size_t lds = xq8_lds_bytes(NCOL, K);
    const int grid = (N + ROWS - 1) / ROWS;
    if (lds <= kXLdsBudget)
        hipLaunchKernelGGL((k_gemv_q6k_q8<F, NCOL, TPR, true>), dim3(grid), dim3(kBlock), lds, s, (const uint8_t*)W, x.q, x.d, x.s, y, N, K);
    else
        hipLaunchKernelGGL((k_gemv_q6k_q8<F, NCOL, TPR, false>), dim3(grid), dim3(kBlock), 0, s, (const uint8_t*)W, x.q, x.d, x.s, y, N, K);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}
template <int F, int NCOL>
int launch_q6k_q8(const void* W, qmm_xq8 x, float* y, int N, int K, hipStream_t s) {
    const size_t per_col = (size_t)K + K / 4;
    const int g = (int)std::min<size_t>(NCOL, kXLdsBudget / per_col);
    if constexpr (NCOL >= 5) {     // measured at 5120 x 17408: 3 columns faster, 4 equal in the unit kernel
      if (K <= 64 * 64 * 6 && q6w_lds_bytes(NCOL, K) <= 160 * 1024) {   // all columns in one pass
        const int grid = (N + kQ6WideWaves - 1) / kQ6WideWaves;
        const size_t lds_w = q6w_lds_bytes(NCOL, K);
#define QMM_Q6W(IV) case IV: hipLaunchKernelGGL((k_gemv_q6k_w<F, NCOL, IV>), dim3(grid), dim3(64 * kQ6WideWaves), lds_w, s, (const uint8_t*)W, x.q, x.d, y, N, K); break;
        switch ((K / 64 + 63) / 64) {
            QMM_Q6W(1) QMM_Q6W(2) QMM_Q6W(3) QMM_Q6W(4) QMM_Q6W(5) QMM_Q6W(6)
            default: return QMM_ERR_SHAPE;
        }
#undef QMM_Q6W
        QMM_LAUNCH_CHECK();
        return QMM_OK;
      }
    }
    if (g >= 1 && K <= 64 * 64 * 6) {                       // unit kernel: at most 6 units per lane
        const int grid = (N + kWavesPerBlock - 1) / kWavesPerBlock;
        const size_t lds_u = (size_t)g * per_col;
#define QMM_Q6U(IV) case IV: hipLaunchKernelGGL((k_gemv_q6k_u<F, NCOL, IV>), dim3(grid), dim3(kBlock), lds_u, s, (const uint8_t*)W, x.q, x.d, y, N, K, g); break;
        switch ((K / 64 + 63) / 64) {
            QMM_Q6U(1) QMM_Q6U(2) QMM_Q6U(3) QMM_Q6U(4) QMM_Q6U(5) QMM_Q6U(6)
            default: return QMM_ERR_SHAPE;
        }
#undef QMM_Q6U
        QMM_LAUNCH_CHECK();
        return QMM_OK;
    }
    switch (q6k_tpr(K)) {
        case 1: return launch_q6k_q8_t<F, NCOL, 1>(W, x, y, N, K, s);
        case 2: return launch_q6k_q8_t<F, NCOL, 2>(W, x, y, N, K, s);
        case 4: return launch_q6k_q8_t<F, NCOL, 4>(W, x, y, N, K, s);
        default: return launch_q6k_q8_t<F, NCOL, 8>(W, x, y, N, K, s);
    }
}

template <int NCOL>
int launch_gemv_q8_ncol(int fmt, const void* W, qmm_xq8 x, float* y, int N, int K, hipStream_t s) {
    switch (fmt) {
        case QMM_Q4_K: return launch_q4k_q8<NCOL>(W, x, y, N, K, s);
        case QMM_Q6_K: return launch_q6k_q8<QMM_Q6_K, NCOL>(W, x, y, N, K, s);
        case QMM_Q6_K_SOA: return launch_q6k_q8<QMM_Q6_K_SOA, NCOL>(W, x, y, N, K, s);
        default: return QMM_ERR_FORMAT;
    }
}

// ------------------------------------------------------------------------------------------
// Q4_K x f32 GEMV on the pair mapping of k_gemv_q4k_q8 (16 lanes per row, a lane owns one 32-byte
// qs pair = 64 weights per iteration, all of a row's loads in flight at once).  x is staged per
// workgroup in LDS as f32, transposed at 16-byte granularity (float4 unit u of pair p at
// (u * K/64 + p) * 16, so consecutive lanes read consecutive banks), followed by the 32-element
// sums of x per sub-block (pair p: {xs(2p), xs(2p+1)} at 4K + 8p).  Per pair and column:
// sA = sum x * qA, sB = sum x * qB (one cvt_f32_ubyte and one fma per weight; the high nibbles stay
// in place as 16 q and the exact 1/16 moves into dB) and acc += dA sA + dB sB - (mA xsA + mB xsB),
// the reference's arithmetic (gemv.hip:1177-1216) in another summation order.
template <int NCOL, int U>
__device__ __forceinline__ void stage_f32_pairs(uint8_t* lds, int K, const XStageF<NCOL, U>& S) {
    const int k8 = K >> 3, n8 = NCOL * k8, kp = K >> 6;
    const size_t cs = (size_t)K * 4 + (size_t)(K >> 3);      // bytes per column
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int e = (int)threadIdx.x + kPairBlock * u;      // floats 8e..8e+7 (quads share e < n8)
        const float4 a = S.v[u][0], b = S.v[u][1];
        float sum = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
        sum += __int_as_float(quad_xor<1>(__float_as_int(sum)));
        sum += __int_as_float(quad_xor<2>(__float_as_int(sum)));
        if (e < n8) {
            const int c = e / k8, f8 = e - c * k8, g = 2 * f8;   // float4 units g, g+1 of the column
            uint8_t* base = lds + (size_t)c * cs;
            const int p = g >> 4, uu = g & 15;
            *(float4*)(base + (size_t)(uu * kp + p) * 16) = a;
            *(float4*)(base + (size_t)((uu + 1) * kp + p) * 16) = b;
            if ((f8 & 3) == 0) *(float*)(base + (size_t)K * 4 + (size_t)(f8 >> 2) * 4) = sum;
        }
    }
}

template <int NCOL, int NITER>
__global__ void __launch_bounds__(kBlock) k_gemv_q4k_f32p(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                          float* __restrict__ y, int N, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int nb = K >> 8, ntask = 4 * nb, kp = K >> 6;
    const size_t cs = (size_t)K * 4 + (size_t)(K >> 3);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = lane & 15, j = t & 3;
    const int row = (blockIdx.x * kWavesPerBlock + wave) * 4 + (lane >> 4);
    const uint8_t* rp = W + (size_t)min(row, N - 1) * ((size_t)nb * 144);
    Q4kPairs<NITER> A;
    {
        XStageF<NCOL, (NCOL * NITER + 1) / 2> S;
        stagef_load<NCOL>(x, K, S);                       // x first (older loads) ...
        q4k_load_pairs<NITER>(rp, t, j, ntask, 0, A);     // ... then the weights
        stage_f32_pairs<NCOL>(smem, K, S);
        lds_barrier();
    }
    const Q4kPairDecode dc(j);
    float acc[NCOL];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = 0.f;
#pragma unroll
    for (int i = 0; i < NITER; ++i) {
        const int task = t + 16 * i, tk = min(task, ntask - 1);
        const uint4 hd = A.h[i], w0 = A.q0[i], w1 = A.q1[i];
        const uint32_t scw = (((hd.y >> dc.sh0) & dc.m0) | (hd.w & dc.m2)) >> dc.bsh;
        const uint32_t mw = (((hd.z >> dc.sh0) & dc.m0) | ((hd.w >> 4) & dc.m2)) >> dc.bsh;
        const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
        const float dA = d * (float)(scw & 0xffu), dB16 = d * (float)((scw >> 8) & 0xffu) * 0.0625f;
        const float mA = dmin * (float)(mw & 0xffu), mB = dmin * (float)((mw >> 8) & 0xffu);
        const uint32_t wq[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int c = 0; c < NCOL; ++c) {
            const uint8_t* xc = smem + (size_t)c * cs;
            float sa = 0.f, sb = 0.f;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t lo = opaque(wq[q] & 0x0f0f0f0fu), hi = opaque(wq[q] & 0xf0f0f0f0u);
                const float4 xa = *(const float4*)(xc + (size_t)(q * kp + tk) * 16);
                const float4 xb = *(const float4*)(xc + (size_t)((8 + q) * kp + tk) * 16);
                sa = __builtin_fmaf(xa.x, (float)(lo & 0xffu), sa);
                sa = __builtin_fmaf(xa.y, (float)((lo >> 8) & 0xffu), sa);
                sa = __builtin_fmaf(xa.z, (float)((lo >> 16) & 0xffu), sa);
                sa = __builtin_fmaf(xa.w, (float)(lo >> 24), sa);
                sb = __builtin_fmaf(xb.x, (float)(hi & 0xffu), sb);
                sb = __builtin_fmaf(xb.y, (float)((hi >> 8) & 0xffu), sb);
                sb = __builtin_fmaf(xb.z, (float)((hi >> 16) & 0xffu), sb);
                sb = __builtin_fmaf(xb.w, (float)(hi >> 24), sb);
            }
            const float2 xs = *(const float2*)(xc + (size_t)K * 4 + (size_t)tk * 8);
            const float v = dA * sa + dB16 * sb - (mA * xs.x + mB * xs.y);
            acc[c] += task < ntask ? v : 0.f;
        }
    }
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = group_sum(acc[c], 16);
    if (t == 0 && row < N) {
#pragma unroll
        for (int c = 0; c < NCOL; ++c) y[(size_t)c * N + row] = acc[c];
    }
}

template <int NCOL>
int launch_q4k_f32p(const void* W, const float* x, float* y, int N, int K, hipStream_t s) {
    const size_t lds = (size_t)NCOL * ((size_t)K * 4 + (size_t)(K >> 3));
    const int grid = (N + 4 * kWavesPerBlock - 1) / (4 * kWavesPerBlock);
#define QMM_FP(IV) case IV: hipLaunchKernelGGL((k_gemv_q4k_f32p<NCOL, IV>), dim3(grid), dim3(kBlock), lds, s, (const uint8_t*)W, x, y, N, K); break;
    switch ((K / 256 * 4 + 15) / 16) {
        QMM_FP(1) QMM_FP(2) QMM_FP(3) QMM_FP(4) QMM_FP(5) QMM_FP(6)
        default: return QMM_ERR_SHAPE;
    }
#undef QMM_FP
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

template <int NCOL>
int launch_q4k_f32(const void* W, const float* x, float* y, int N, int K, hipStream_t s) {
    const size_t xsum = (size_t)NCOL * (K / 32) * 4, xf = (size_t)NCOL * K * 4;
    const int grid = persistent_grid(N);
    if (xsum + xf <= kXLdsBudget)
        hipLaunchKernelGGL((k_gemv_q4k_f32<NCOL, true>), dim3(grid), dim3(kBlock), xsum + xf, s, (const uint8_t*)W, x, y, N, K);
    else
        hipLaunchKernelGGL((k_gemv_q4k_f32<NCOL, false>), dim3(grid), dim3(kBlock), xsum, s, (const uint8_t*)W, x, y, N, K);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

bool fmt_supported_q8(int fmt) {
    return fmt == QMM_Q4_K || fmt == QMM_Q6_K || fmt == QMM_Q6_K_SOA || fmt == QMM_Q5_K || fmt == QMM_IQ4_XS ||
           fmt == QMM_Q8_0_SOA || fmt == QMM_Q5_1_SOA;
}

// K granule per format: 256 for the block formats; the row-SoA repacks of 32-weight blocks take
// K % 32 (Q5_1_SOA: 24-byte units, rows 8-byte aligned) or K % 64 (Q8_0_SOA: 34 bytes per 32 weights,
// so K % 64 keeps every row dword aligned for the 16-byte loads)
int gemv_k_granule(int fmt) { return fmt == QMM_Q5_1_SOA ? 32 : fmt == QMM_Q8_0_SOA ? 64 : 256; }

int check_gemv_shape(int fmt, int N, int K) {
    if (N <= 0 || K <= 0 || K % gemv_k_granule(fmt) != 0) return QMM_ERR_SHAPE;
    if (fmt == QMM_Q6_K_SOA && ((K / 256) & 1)) return QMM_ERR_SHAPE;   // streams must stay dword aligned
    return QMM_OK;
}

}  // namespace

// Q4_K calls with at least this many columns run on the matrix cores (gemv_mfma.hip: the same bits;
// at 17408 x 5120 it is the faster kernel from 4 columns on)
int g_mfma_min_ncol = 4;
// Q6_K_SOA calls with at least this many columns (and at most 8) run on the matrix cores (measured at
// 5120 x 17408: 2 columns 26.5 us on the dot4 kernel against 33, 3 columns 35 against 33, 4 43 against 33)
int g_q6_mfma_min_ncol = 3;
// Q8_0_SOA calls with at least this many columns (and at most 8) run on the matrix cores (measured at
// 17408 x 5120: 25.0-25.3 us at any column count; the dot4 kernel 24.2-24.7 at 3 columns, 26.8 at 4,
// 35.0 at 8)
int g_q80_mfma_min_ncol = 4;

int gemv_q8_dispatch(int fmt, const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, hipStream_t s) {
    if (fmt == QMM_Q8_0_SOA && ncol >= g_q80_mfma_min_ncol && gemv_q80_mfma_fits(K, ncol) && ((uintptr_t)x.d & 7) == 0)
        return gemv_q80_mfma(W, x, y, N, K, ncol, s);
    if (fmt == QMM_Q5_K || fmt == QMM_IQ4_XS || fmt == QMM_Q8_0_SOA || fmt == QMM_Q5_1_SOA)
        return gemv_fmt_dispatch(fmt, W, x, y, N, K, ncol, s);
    if (fmt == QMM_Q4_K && ncol >= g_mfma_min_ncol && ncol <= 16 && gemv_q4k_mfma_lds(K, ncol) <= kMfmaLdsMax) {
        const qmm_gemv_seg seg = {QMM_Q4_K, W, y, N, K};
        return gemv_q4k_mfma(&seg, 1, x, K, ncol, s);
    }
    if (fmt == QMM_Q6_K_SOA && ncol >= g_q6_mfma_min_ncol && ncol <= 8 && K >= 512 && K % 512 == 0 &&
        gemv_q6k_mfma_fits(K, ncol) && ((uintptr_t)x.d & 15) == 0)
        return gemv_q6k_mfma(W, x, y, N, K, ncol, s);
    switch (ncol) {
        case 1: return launch_gemv_q8_ncol<1>(fmt, W, x, y, N, K, s);
        case 2: return launch_gemv_q8_ncol<2>(fmt, W, x, y, N, K, s);
        case 3: return launch_gemv_q8_ncol<3>(fmt, W, x, y, N, K, s);
        case 4: return launch_gemv_q8_ncol<4>(fmt, W, x, y, N, K, s);
        case 5: return launch_gemv_q8_ncol<5>(fmt, W, x, y, N, K, s);
        case 6: return launch_gemv_q8_ncol<6>(fmt, W, x, y, N, K, s);
        case 7: return launch_gemv_q8_ncol<7>(fmt, W, x, y, N, K, s);
        case 8: return launch_gemv_q8_ncol<8>(fmt, W, x, y, N, K, s);
        default: return QMM_ERR_SHAPE;
    }
}

// one run of nseg (<= 4) segments of format fmt sharing x: Q4_K on the matrix cores (16 columns per
// launch) from g_mfma_min_ncol columns on, else the dot4 kernel (8 per launch); Q5_K, IQ4_XS, Q8_0_SOA
// and Q5_1_SOA in one launch per 8 columns; Q6_K (both layouts) per segment
int gemv_multi_run(const qmm_gemv_seg* segs, int nseg, qmm_xq8 x, int K, int ncol, hipStream_t s) {
    const int fmt = segs[0].fmt;
    auto xcols = [&](int c0) {
        return qmm_xq8{x.q + (size_t)c0 * K, x.d + (size_t)c0 * (K / 32), x.s + (size_t)c0 * (K / 32), nullptr};
    };
    if (fmt == QMM_Q4_K) {
        int cpl = 16;                                         // columns per matrix-core launch
        while (cpl > 1 && gemv_q4k_mfma_lds(K, cpl) > kMfmaLdsMax) cpl /= 2;
        const bool mfma = ncol >= g_mfma_min_ncol && cpl >= 2;
        const int step = mfma ? cpl : 8;
        for (int c0 = 0; c0 < ncol; c0 += step) {
            const int nc = ncol - c0 < step ? ncol - c0 : step;
            const qmm_xq8 xc = xcols(c0);
            qmm_gemv_seg sc[4];
            for (int i = 0; i < nseg; ++i) {
                sc[i] = segs[i];
                sc[i].y = segs[i].y + (size_t)c0 * segs[i].N;
            }
            // a tail pass of fewer columns runs the dot4 kernel (the same bits)
            const int e = mfma && nc >= g_mfma_min_ncol ? gemv_q4k_mfma(sc, nseg, xc, K, nc, s) : gemv_q4k_q8_multi(segs, nseg, xc, K, nc, c0, s);
            if (e) return e;
        }
        return QMM_OK;
    }
    const bool fmt_multi = fmt == QMM_Q5_K || fmt == QMM_IQ4_XS || fmt == QMM_Q8_0_SOA || fmt == QMM_Q5_1_SOA;
    for (int c0 = 0; c0 < ncol; c0 += 8) {
        const int nc = ncol - c0 < 8 ? ncol - c0 : 8;
        const qmm_xq8 xc = xcols(c0);
        qmm_gemv_seg sc[4];
        for (int i = 0; i < nseg; ++i) {
            sc[i] = segs[i];
            sc[i].y = segs[i].y + (size_t)c0 * segs[i].N;
        }
        if (fmt_multi) {
            if (int e = gemv_fmt_dispatch_segs(fmt, sc, nseg, xc, K, nc, s)) return e;
        } else {
            for (int i = 0; i < nseg; ++i)
                if (int e = gemv_q8_dispatch(fmt, sc[i].w, xc, sc[i].y, sc[i].N, K, nc, s)) return e;
        }
    }
    return QMM_OK;
}

}  // namespace qmm

using namespace qmm;

extern "C" {

int qmm_set_gemv_mfma_min_ncol(int n) {
    const int prev = g_mfma_min_ncol;
    g_mfma_min_ncol = n < 1 ? 1 : n;
    return prev;
}

int qmm_set_gemv_q6k_mfma_min_ncol(int n) {
    const int prev = g_q6_mfma_min_ncol;
    g_q6_mfma_min_ncol = n < 1 ? 1 : n;
    return prev;
}

int qmm_set_gemv_q80_mfma_min_ncol(int n) {
    const int prev = g_q80_mfma_min_ncol;
    g_q80_mfma_min_ncol = n < 1 ? 1 : n;
    return prev;
}

int qmm_quantize_x_q8(const float* x, qmm_xq8 out, int ncol, int K, void* stream) {
    if (!x || !out.q || !out.d || !out.s) return QMM_ERR_NULL;
    if (ncol <= 0 || K <= 0 || K % 32 != 0) return QMM_ERR_SHAPE;
    dim3 grid((K / 32 + 7) / 8, ncol);
    hipLaunchKernelGGL(k_quantize_x_q8, grid, dim3(256), 0, (hipStream_t)stream, x, out.q, out.d, out.s, (float2*)out.ds, K);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_gemv_q8_f32x(int fmt, const void* W, const float* x, float* y, int N, int K, int ncol, void* stream) {
    if (fmt != QMM_Q4_K) return QMM_ERR_FORMAT;
    if (!W || !x || !y) return QMM_ERR_NULL;
    if (int e = check_gemv_shape(fmt, N, K)) return e;
    if (ncol < 1 || ncol > 4 || K > 6144) return QMM_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    switch (ncol) {
        case 1: return launch_q4k_fx<1>(W, x, y, N, K, s);
        case 2: return launch_q4k_fx<2>(W, x, y, N, K, s);
        case 3: return launch_q4k_fx<3>(W, x, y, N, K, s);
        default: return launch_q4k_fx<4>(W, x, y, N, K, s);
    }
}

int qmm_gemv_q8(int fmt, const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, int tpr, int rpt, void* stream) {
    if (!fmt_supported_q8(fmt)) return QMM_ERR_FORMAT;
    if (!W || !x.q || !x.d || !x.s || !y) return QMM_ERR_NULL;
    if (int e = check_gemv_shape(fmt, N, K)) return e;
    // rpt 5 and rpt 4 with tpr 3 read the reference's experimental interleaved weight layouts
    // (repack_interleave8, gemv.hip:1467-1472; repack_wmma_il, gemv_wmma mode 3)
    if (rpt == 5) {
        if (fmt != QMM_Q4_K && fmt != QMM_Q5_K && fmt != QMM_IQ4_XS) return QMM_ERR_FORMAT;
        if (N % 8 != 0 || ncol < 1 || ncol > 8) return QMM_ERR_SHAPE;
        return gemv_il_dispatch(8, fmt, W, x, y, N, K, ncol, (hipStream_t)stream);
    }
    if (rpt == 4 && tpr == 3) {
        if (fmt != QMM_Q4_K && fmt != QMM_Q5_K && fmt != QMM_IQ4_XS && fmt != QMM_Q6_K_SOA && fmt != QMM_Q8_0_SOA)
            return QMM_ERR_FORMAT;
        if (K % 256 != 0 || ncol < 1 || ncol > 16) return QMM_ERR_SHAPE;
        return gemv_il_dispatch(16, fmt, W, x, y, N, K, ncol, (hipStream_t)stream);
    }
    // rpt 4 is the reference's route to its T-invariant WMMA GEMV (gemv.hip:1472-1475, up to 16
    // columns), which every GEMV here already is
    if (rpt == 4) {
        if (ncol < 1 || ncol > 16) return QMM_ERR_SHAPE;
        const qmm_gemv_seg seg = {fmt, W, y, N, K};
        return qmm_gemv_multi(&seg, 1, x, ncol, stream);
    }
    // any other tpr / rpt: the reference's launch-shape knobs (its unlisted values fall to a default
    // kernel, gemv.hip:1236-1242); the launch shape here follows the tensor shape
    if (ncol < 1 || ncol > 8) return QMM_ERR_SHAPE;
    return gemv_q8_dispatch(fmt, W, x, y, N, K, ncol, (hipStream_t)stream);
}

int qmm_gemv_multi(const qmm_gemv_seg* segs, int nseg, qmm_xq8 x, int ncol, void* stream) {
    if (!segs || !x.q || !x.d || !x.s) return QMM_ERR_NULL;
    if (nseg < 1 || nseg > 4 || ncol < 1) return QMM_ERR_SHAPE;
    for (int i = 0; i < nseg; ++i) {
        if (!fmt_supported_q8(segs[i].fmt)) return QMM_ERR_FORMAT;
        if (!segs[i].w || !segs[i].y) return QMM_ERR_NULL;
        if (int e = check_gemv_shape(segs[i].fmt, segs[i].N, segs[i].K)) return e;
        if (segs[i].K != segs[0].K) return QMM_ERR_SHAPE;
    }
    const int K = segs[0].K;
    // runs of consecutive segments of one format (at most 4, the reference's gemv_wmma grouping), each
    // run in one launch per column pass; every row gets the arithmetic of its format's plain GEMV
    for (int i0 = 0; i0 < nseg;) {
        int i1 = i0 + 1;
        while (i1 < nseg && segs[i1].fmt == segs[i0].fmt) ++i1;
        if (int e = gemv_multi_run(segs + i0, i1 - i0, x, K, ncol, (hipStream_t)stream)) return e;
        i0 = i1;
    }
    return QMM_OK;
}

int qmm_gemv_q4_K_f32(const void* W, const float* x, float* y, int N, int K, int ncol, int tpr, void* stream) {
    if (!W || !x || !y) return QMM_ERR_NULL;
    if (int e = check_gemv_shape(QMM_Q4_K, N, K)) return e;
    if (ncol < 1 || ncol > 8) return QMM_ERR_SHAPE;
    (void)tpr;   // the reference's threads per row (its other values take its default, gemv.hip:1486-1489)
    hipStream_t s = (hipStream_t)stream;
    // pair kernel: columns in launches of at most g (what fits the LDS budget); every column gets
    // the same arithmetic whatever ncol is
    const size_t per_col = (size_t)K * 4 + (size_t)(K >> 3);
    const int g = (int)min((size_t)3, kXLdsBudget / per_col);
    if (K <= 6144 && g >= 1) {
        for (int c0 = 0; c0 < ncol; c0 += g) {
            const int nc = min(g, ncol - c0);
            const float* xc = x + (size_t)c0 * K;
            float* yc = y + (size_t)c0 * N;
            const int e = nc == 1 ? launch_q4k_f32p<1>(W, xc, yc, N, K, s)
                        : nc == 2 ? launch_q4k_f32p<2>(W, xc, yc, N, K, s)
                                  : launch_q4k_f32p<3>(W, xc, yc, N, K, s);
            if (e != QMM_OK) return e;
        }
        return QMM_OK;
    }
    switch (ncol) {
        case 1: return launch_q4k_f32<1>(W, x, y, N, K, s);
        case 2: return launch_q4k_f32<2>(W, x, y, N, K, s);
        case 3: return launch_q4k_f32<3>(W, x, y, N, K, s);
        case 4: return launch_q4k_f32<4>(W, x, y, N, K, s);
        case 5: return launch_q4k_f32<5>(W, x, y, N, K, s);
        case 6: return launch_q4k_f32<6>(W, x, y, N, K, s);
        case 7: return launch_q4k_f32<7>(W, x, y, N, K, s);
        default: return launch_q4k_f32<8>(W, x, y, N, K, s);
    }
}

}  // extern "C"
