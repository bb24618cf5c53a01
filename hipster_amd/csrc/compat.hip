// compat.hip -- the rest of the reference's quantized-matmul call surface on gfx950, so that the
// engine and its validators compile and run against this library unchanged:
//
//   qmm_gemv_splitk        gemv_splitk     engine/kernels/gemv.h:55, gemv.hip:1397-1441
//   qmm_hc_up_fused        hc_up_fused     gemv.h:52 (declared only: returns QMM_ERR_UNSUPPORTED)
//   qmm_moe_gemm_q8        moe_gemm        gemv.h:49-50, gemv.hip:909-969,1377-1381 (q8 activations)
//   qmm_quantize_x_q8k     quantize_x_q8k  gemv.h:34, gemv.hip:686-705,1254-1257
//   qmm_gemv_q8k           gemv_wmma_q8k   gemv.h:35, gemv.hip:706-794,1259-1271
//
// All of them are built on the per-format units of fmt_unit.hpp: every (row, column) is the
// reference's q8 arithmetic (integer dot per scale group, the per-sub-block fix-up in f32), a lane
// accumulates its units in a fixed order and the wave reduces with a fixed butterfly, so a column's
// result does not depend on how many columns a call carries.  They are VALU kernels: the engine's
// hot calls go to the tuned kernels of gemv.hip / moe_prefill.hip; these keep the remaining call
// sites working with the reference's exact (not bf16-rounded) numerics.
#include "fmt_unit.hpp"
#include "qmm_common.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>

namespace qmm {
namespace {

constexpr int kCThreads = 256, kCWaves = kCThreads / 64, kCRpw = 2, kCCols = 8;

// ---- split-K GEMV: part[(c * ksplit + ks) * N + n] = W[n][K range ks] . x[c][K range ks] ----------
// The K range of split ks is the 256-weight blocks [ks*nb/ksplit, (ks+1)*nb/ksplit), nb = ceil(K/256)
// (gemv.hip:1404), so every partial covers the same weights as the reference's.
template <int F, int NC, int NIT>
__global__ void __launch_bounds__(kCThreads) k_gemv_splitk(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                           const float* __restrict__ xd, const float* __restrict__ xs,
                                                           float* __restrict__ part, int N, int K, int ksplit, int c0) {
    const int ks = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kCWaves + wave) * kCRpw;
    const int nb = (K + 255) >> 8, U = fmt_units<F>(K), upb = 256 / fmt_unit_weights<F>();
    const int ub = min(ks * nb / ksplit * upb, U), ue = min((ks + 1) * nb / ksplit * upb, U);
    const int nsb = K >> 5;
    XSrcQ8 src[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) src[c] = XSrcQ8{xq + (size_t)(c0 + c) * K, xd + (size_t)(c0 + c) * nsb, xs + (size_t)(c0 + c) * nsb};
    float acc[kCRpw][NC];
    fmt_rows<F, NC, NIT, kCRpw>(W, row0, N, K, src, acc, ub, ue);
#pragma unroll
    for (int r = 0; r < kCRpw; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = wave_sum(acc[r][c]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < kCRpw; ++r)
            if (row0 + r < N) {
#pragma unroll
                for (int c = 0; c < NC; ++c) part[((size_t)(c0 + c) * ksplit + ks) * N + row0 + r] = acc[r][c];
            }
    }
}

template <int F>
int launch_splitk(const void* W, qmm_xq8 x, float* part, int N, int K, int ksplit, int ncol, hipStream_t s) {
    const int nb = (K + 255) >> 8, upb = 256 / fmt_unit_weights<F>();
    const int per_split = (nb + ksplit - 1) / ksplit * upb;       // units of the longest split
    const dim3 grid((unsigned)((N + kCWaves * kCRpw - 1) / (kCWaves * kCRpw)), (unsigned)ksplit);
    for (int c0 = 0; c0 < ncol; c0 += kCCols) {
        const int nc = std::min(kCCols, ncol - c0);
#define QMM_SK(NC, NIT) hipLaunchKernelGGL((k_gemv_splitk<F, NC, NIT>), grid, dim3(kCThreads), 0, s, (const uint8_t*)W, x.q, x.d, x.s, part, N, K, ksplit, c0)
#define QMM_SKN(NIT) switch (nc) { case 1: QMM_SK(1, NIT); break; case 2: QMM_SK(2, NIT); break; case 3: QMM_SK(3, NIT); break; \
                                   case 4: QMM_SK(4, NIT); break; case 5: QMM_SK(5, NIT); break; case 6: QMM_SK(6, NIT); break; \
                                   case 7: QMM_SK(7, NIT); break; default: QMM_SK(8, NIT); break; }
        if (per_split <= 64) { QMM_SKN(1) } else { QMM_SKN(2) }
#undef QMM_SKN
#undef QMM_SK
        QMM_LAUNCH_CHECK();
    }
    return QMM_OK;
}

// ---- grouped expert GEMM over sorted slots with q8 activations (moe_gemm, gemv.hip:909-969) -------
// Workgroup (row block, tile): tile = (expert, k0, ncols); column r < ncols is x row rowtab[k0+r]
// (or k0+r), output row k0+r: y[(k0 + r) * N + n] = W_e[n] . x[row].  W_e = W + expert * ebytes in
// format F, or Wsh when expert < 0 (read in F too: the reference's routed launch does the same).
// Columns in passes of up to 8; rows of a wave as the plain GEMV of the format.
template <int F, int NIT, int NC>
__device__ __forceinline__ void moe_q8_pass(const uint8_t* wb, int row0, int N, int K, const int8_t* xq, const float* xd,
                                            const float* xs, const int* rowtab, int k0, int nc, float* __restrict__ y) {
    const int nsb = K >> 5, lane = threadIdx.x & 63;
    XSrcQ8 src[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int k = k0 + min(c, nc - 1);
        const size_t xr = (size_t)(rowtab ? rowtab[k] : k);
        src[c] = XSrcQ8{xq + xr * K, xd + xr * nsb, xs + xr * nsb};
    }
    float acc[kCRpw][NC];
    fmt_rows<F, NC, NIT, kCRpw>(wb, row0, N, K, src, acc, 0, fmt_units<F>(K));
#pragma unroll
    for (int r = 0; r < kCRpw; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = wave_sum(acc[r][c]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < kCRpw; ++r)
            if (row0 + r < N) {
#pragma unroll
                for (int c = 0; c < NC; ++c)
                    if (c < nc) y[(size_t)(k0 + c) * N + row0 + r] = acc[r][c];
            }
    }
}

template <int F, int NIT>
__global__ void __launch_bounds__(kCThreads) k_moe_gemm_q8(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Wsh, size_t ebytes,
                                                           const qmm_moe_tile* __restrict__ tiles, const int* __restrict__ rowtab,
                                                           const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                           const float* __restrict__ xs, float* __restrict__ y, int N, int K) {
    const qmm_moe_tile tl = tiles[blockIdx.y];
    if (tl.ncols <= 0) return;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kCWaves + wave) * kCRpw;
    const uint8_t* wb = tl.expert >= 0 ? W + (size_t)tl.expert * ebytes : Wsh;
    for (int c0 = 0; c0 < tl.ncols; c0 += kCCols) {
        const int nc = min(kCCols, tl.ncols - c0), k0 = tl.k0 + c0;
        if (nc == 1) moe_q8_pass<F, NIT, 1>(wb, row0, N, K, xq, xd, xs, rowtab, k0, nc, y);
        else if (nc == 2) moe_q8_pass<F, NIT, 2>(wb, row0, N, K, xq, xd, xs, rowtab, k0, nc, y);
        else if (nc <= 4) moe_q8_pass<F, NIT, 4>(wb, row0, N, K, xq, xd, xs, rowtab, k0, nc, y);
        else moe_q8_pass<F, NIT, 8>(wb, row0, N, K, xq, xd, xs, rowtab, k0, nc, y);
    }
}

template <int F>
int launch_moe_q8(const void* W, const void* Wsh, size_t ebytes, const qmm_moe_tile* tiles, int ntiles, const int* rowtab,
                  qmm_xq8 x, float* y, int N, int K, hipStream_t s) {
    if (ntiles <= 0) return QMM_OK;
    const dim3 grid((unsigned)((N + kCWaves * kCRpw - 1) / (kCWaves * kCRpw)), (unsigned)ntiles);
    if ((fmt_units<F>(K) + 63) / 64 <= 1)
        hipLaunchKernelGGL((k_moe_gemm_q8<F, 1>), grid, dim3(kCThreads), 0, s, (const uint8_t*)W, (const uint8_t*)Wsh, ebytes, tiles,
                           rowtab, x.q, x.d, x.s, y, N, K);
    else
        hipLaunchKernelGGL((k_moe_gemm_q8<F, 2>), grid, dim3(kCThreads), 0, s, (const uint8_t*)W, (const uint8_t*)Wsh, ebytes, tiles,
                           rowtab, x.q, x.d, x.s, y, N, K);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int moe_q8_dispatch(int fmt, const void* W, const void* Wsh, size_t ebytes, const qmm_moe_tile* tiles, int ntiles,
                    const int* rowtab, qmm_xq8 x, float* y, int N, int K, hipStream_t s) {
    switch (fmt) {
        case QMM_Q4_K: return launch_moe_q8<QMM_Q4_K>(W, Wsh, ebytes, tiles, ntiles, rowtab, x, y, N, K, s);
        case QMM_Q5_K: return launch_moe_q8<QMM_Q5_K>(W, Wsh, ebytes, tiles, ntiles, rowtab, x, y, N, K, s);
        case QMM_IQ4_XS: return launch_moe_q8<QMM_IQ4_XS>(W, Wsh, ebytes, tiles, ntiles, rowtab, x, y, N, K, s);
        case QMM_Q8_0_SOA: return launch_moe_q8<QMM_Q8_0_SOA>(W, Wsh, ebytes, tiles, ntiles, rowtab, x, y, N, K, s);
        case QMM_Q5_1_SOA: return launch_moe_q8<QMM_Q5_1_SOA>(W, Wsh, ebytes, tiles, ntiles, rowtab, x, y, N, K, s);
        default: return QMM_ERR_FORMAT;
    }
}

// ---- grouped expert GEMM with q8 activations on the int8 matrix cores (Q4_K experts) ---------------
// The arithmetic of the reference's moe_gemm (gemv.hip:804-953): per 32-weight sub-block the exact
// integer dot C = sum q * xq, then acc += (d sc) xd C - (dmin m) xs in fp32, sub-blocks in K order.
// Workgroup = (64 weight rows, tile); wave w owns rows n0 + 16w .. +15.  Per 256-weight block the pass's
// tokens (at most 48 columns of the tile) are staged in LDS as int8 with their per-32 scales,
// double-buffered (one barrier per block).  A sub-block is one v_mfma_i32_16x16x32_i8 per 16 tokens
// with A = x (16 tokens x 32) and B = 32 weights x 16 rows: lane l supplies token l%16 and weight row
// l%16, bytes k = 8(l/16)..+7 of the sub-block, and receives D[4(l/16) + r][l%16] -- four tokens of its
// own weight row, whose sub-block scales it decoded from the block header it loaded itself.
constexpr int kQmTok = 16, kQmMaxTok = 48, kQmRows = 64, kQmThreads = 256;
#ifndef QMM_QM_RG
#define QMM_QM_RG 2
#endif

struct QmLds {
    uint2 x[2][8][4][kQmMaxTok];     // [buffer][sub-block][k quarter][token]: 8 bytes of x
    float2 sd[2][8][kQmMaxTok];      // [buffer][sub-block][token]: {xd, xs}
};

struct QmArgs {
    const uint8_t* W;                // routed experts (expert e at W + e * ebytes)
    const uint8_t* Wsh;              // shared expert
    size_t ebytes;
    const qmm_moe_tile* tiles;       // blockIdx.y < ntiles: routed tiles; then the shared tiles
    const qmm_moe_tile* stiles;
    int ntiles;
    const int* rowtab;
    const int8_t* xq;
    const float* xd;
    const float* xs;
    float* y;
    int N, K;
};

// the x of block b for tokens [c0, c0 + 16 CB) of the tile (token c clamped to the last column) into
// registers: thread t loads 16-byte piece t + 256 i (token p / 16, piece p % 16) and scale pair
// t + 256 i (token p / 8, sub-block p % 8)
template <int CB>
struct QmXRegs { uint4 v[CB]; float2 sd[(CB * 128 + kQmThreads - 1) / kQmThreads]; };

template <int CB>
__device__ __forceinline__ void qm_x_load(const QmArgs& a, const qmm_moe_tile& tl, int c0, int ncl, int b, QmXRegs<CB>& R) {
    const int nsb = a.K >> 5;
#pragma unroll
    for (int i = 0; i < CB; ++i) {
        const int p = (int)threadIdx.x + kQmThreads * i, c = p >> 4, part = p & 15;
        const int k = tl.k0 + c0 + min(c, ncl - 1);
        const size_t xr = (size_t)(a.rowtab ? a.rowtab[k] : k);
        R.v[i] = *(const uint4*)(a.xq + xr * a.K + (size_t)b * 256 + 16 * part);
    }
#pragma unroll
    for (int i = 0; i < (CB * 128 + kQmThreads - 1) / kQmThreads; ++i) {
        const int p = min((int)threadIdx.x + kQmThreads * i, CB * 128 - 1), c = p >> 3, sb = p & 7;
        const int k = tl.k0 + c0 + min(c, ncl - 1);
        const size_t xr = (size_t)(a.rowtab ? a.rowtab[k] : k);
        R.sd[i] = make_float2(a.xd[xr * nsb + (size_t)b * 8 + sb], a.xs[xr * nsb + (size_t)b * 8 + sb]);
    }
}

template <int CB>
__device__ __forceinline__ void qm_x_store(QmLds& L, int buf, const QmXRegs<CB>& R) {
#pragma unroll
    for (int i = 0; i < CB; ++i) {
        const int p = (int)threadIdx.x + kQmThreads * i, c = p >> 4, part = p & 15, sb = part >> 1, kq = 2 * (part & 1);
        L.x[buf][sb][kq][c] = make_uint2(R.v[i].x, R.v[i].y);
        L.x[buf][sb][kq + 1][c] = make_uint2(R.v[i].z, R.v[i].w);
    }
#pragma unroll
    for (int i = 0; i < (CB * 128 + kQmThreads - 1) / kQmThreads; ++i) {
        const int p = (int)threadIdx.x + kQmThreads * i;
        if (p < CB * 128) L.sd[buf][p & 7][p >> 3] = R.sd[i];
    }
}

struct QmW { uint4 hd; uint2 q[4]; };

__device__ __forceinline__ void qm_w_load(const uint8_t* rp, int b, int kq, QmW& w) {
    const uint8_t* blk = rp + (size_t)b * 144;
    w.hd = *(const uint4*)blk;
#pragma unroll
    for (int j = 0; j < 4; ++j) w.q[j] = *(const uint2*)(blk + 16 + 32 * j + 8 * kq);
}

// one pass: tokens [c0, c0 + ncl) of the tile, ncl <= 16 CB, against the lane's RG weight rows (row
// groups of 16: the x fragment of a sub-block feeds RG MFMAs)
template <int CB, int RG>
__device__ __forceinline__ void qm_pass(const QmArgs& a, const qmm_moe_tile& tl, const uint8_t* const (&rp)[RG], const int (&row)[RG],
                                        int c0, int ncl, QmLds& L) {
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63, tok = lane & 15, kq = lane >> 4;
    const int nb = a.K >> 8;
    float acc[CB][RG][4];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int g = 0; g < RG; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[cb][g][r] = 0.f;
    QmXRegs<CB> R;
    QmW w[RG], wn[RG];
    qm_x_load<CB>(a, tl, c0, ncl, 0, R);
#pragma unroll
    for (int g = 0; g < RG; ++g) qm_w_load(rp[g], 0, kq, w[g]);
    __syncthreads();                                   // the previous pass's last reads of buffer 0 are done
    qm_x_store<CB>(L, 0, R);
    __syncthreads();
    for (int b = 0; b < nb; ++b) {
        const int cur = b & 1;
        if (b + 1 < nb) {                             // the next block's x and weights in flight during this one
            qm_x_load<CB>(a, tl, c0, ncl, b + 1, R);
#pragma unroll
            for (int g = 0; g < RG; ++g) qm_w_load(rp[g], b + 1, kq, wn[g]);
        }
        // per row group: d, dmin and the 8 scale / min bytes as 64-bit words, consumed two bytes (one pair)
        // per iteration from the bottom
        float d[RG], dmin[RG];
        uint64_t scb[RG], mnb[RG];
        uint2 q0[RG], q1[RG], q2[RG], q3[RG];
#pragma unroll
        for (int g = 0; g < RG; ++g) {
            d[g] = h2f(w[g].hd.x);
            dmin[g] = h2f(w[g].hd.x >> 16);
            const Q4kScaleBytes sbt = q4k_scale_bytes(w[g].hd.y, w[g].hd.z, w[g].hd.w);
            scb[g] = ((uint64_t)sbt.sc_hi << 32) | sbt.sc_lo;
            mnb[g] = ((uint64_t)sbt.m_hi << 32) | sbt.m_lo;
            q0[g] = w[g].q[0]; q1[g] = w[g].q[1]; q2[g] = w[g].q[2]; q3[g] = w[g].q[3];
        }
        // a loop, not unrolled: one qs pair (two sub-blocks) per iteration keeps the register count low
#pragma unroll 1
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int hi = 0; hi < 2; ++hi) {
                const int sb = 2 * j + hi;
                float ws[RG], wm[RG];
                long wb[RG];
#pragma unroll
                for (int g = 0; g < RG; ++g) {
                    ws[g] = d[g] * (float)(((uint32_t)scb[g] >> (8 * hi)) & 0xffu);
                    wm[g] = dmin[g] * (float)(((uint32_t)mnb[g] >> (8 * hi)) & 0xffu);
                    wb[g] = (long)(((uint64_t)((q0[g].y >> (4 * hi)) & 0x0f0f0f0fu) << 32) | (uint64_t)((q0[g].x >> (4 * hi)) & 0x0f0f0f0fu));
                }
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    const uint2 xv = L.x[cur][sb][kq][kQmTok * cb + tok];
                    const long xa = (long)(((uint64_t)xv.y << 32) | (uint64_t)xv.x);
                    const float4 s01 = *(const float4*)&L.sd[cur][sb][kQmTok * cb + 4 * kq];
                    const float4 s23 = *(const float4*)&L.sd[cur][sb][kQmTok * cb + 4 * kq + 2];
#pragma unroll
                    for (int g = 0; g < RG; ++g) {
                        const i32x4 z = {0, 0, 0, 0};
                        const i32x4 C = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa, wb[g], z, 0, 0, 0);
                        float* ac = acc[cb][g];
                        ac[0] = __builtin_fmaf(-wm[g], s01.y, __builtin_fmaf(ws[g] * s01.x, (float)C[0], ac[0]));
                        ac[1] = __builtin_fmaf(-wm[g], s01.w, __builtin_fmaf(ws[g] * s01.z, (float)C[1], ac[1]));
                        ac[2] = __builtin_fmaf(-wm[g], s23.y, __builtin_fmaf(ws[g] * s23.x, (float)C[2], ac[2]));
                        ac[3] = __builtin_fmaf(-wm[g], s23.w, __builtin_fmaf(ws[g] * s23.z, (float)C[3], ac[3]));
                    }
                }
            }
#pragma unroll
            for (int g = 0; g < RG; ++g) {
                q0[g] = q1[g];
                q1[g] = q2[g];
                q2[g] = q3[g];
                scb[g] >>= 16;
                mnb[g] >>= 16;
            }
        }
        if (b + 1 < nb) {
            qm_x_store<CB>(L, cur ^ 1, R);
#pragma unroll
            for (int g = 0; g < RG; ++g) w[g] = wn[g];
        }
        __syncthreads();
    }
#pragma unroll
    for (int g = 0; g < RG; ++g)
        if (row[g] < a.N) {
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int c = kQmTok * cb + 4 * kq + r;
                    if (c < ncl) a.y[(size_t)(tl.k0 + c0 + c) * a.N + row[g]] = acc[cb][g][r];
                }
        }
}

// CBMAX: 16-token blocks of the widest pass (1 when every tile has at most 16 columns); RG row groups
// of 16 per wave (a workgroup covers 64 RG weight rows)
template <int CBMAX, int RG>
__global__ void __launch_bounds__(kQmThreads) k_moe_gemm_q8_q4k(QmArgs a) {
    __shared__ __align__(16) QmLds L;
    const int ty = blockIdx.y;
    const bool routed = ty < a.ntiles;
    const qmm_moe_tile tl = routed ? a.tiles[ty] : a.stiles[ty - a.ntiles];
    if (tl.ncols <= 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint8_t* base = routed && tl.expert >= 0 ? a.W + (size_t)tl.expert * a.ebytes : a.Wsh;
    int row[RG];
    const uint8_t* rp[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) {
        row[g] = blockIdx.x * (kQmRows * RG) + 16 * (RG * wave + g) + (lane & 15);
        rp[g] = base + (size_t)min(row[g], a.N - 1) * (size_t)(a.K >> 8) * 144;
    }
    constexpr int kPass = kQmTok * CBMAX;
    for (int c0 = 0; c0 < tl.ncols; c0 += kPass) {
        const int ncl = min(kPass, tl.ncols - c0);
        if (CBMAX == 1 || ncl <= kQmTok) qm_pass<1, RG>(a, tl, rp, row, c0, ncl, L);
        else if (CBMAX == 2 || ncl <= 2 * kQmTok) qm_pass<(CBMAX >= 2 ? 2 : 1), RG>(a, tl, rp, row, c0, ncl, L);
        else qm_pass<(CBMAX >= 3 ? 3 : 1), RG>(a, tl, rp, row, c0, ncl, L);
    }
}

int launch_moe_q8_q4k(const void* W, const void* Wsh, size_t ebytes, const qmm_moe_tile* tiles, int ntiles,
                      const qmm_moe_tile* stiles, int nstiles, int ct, const int* rowtab, qmm_xq8 x, float* y, int N, int K,
                      hipStream_t s) {
    if (ntiles + nstiles <= 0) return QMM_OK;
    constexpr int RG = QMM_QM_RG;
    const QmArgs a = {(const uint8_t*)W, (const uint8_t*)Wsh, ebytes, tiles, stiles, ntiles, rowtab, x.q, x.d, x.s, y, N, K};
    const dim3 grid((unsigned)((N + kQmRows * RG - 1) / (kQmRows * RG)), (unsigned)(ntiles + nstiles));
    // tiles hold at most 16 ct columns (the reference's tiling): passes of up to 48 columns
    if (ct <= 1) hipLaunchKernelGGL((k_moe_gemm_q8_q4k<1, RG>), grid, dim3(kQmThreads), 0, s, a);
    else if (ct == 2) hipLaunchKernelGGL((k_moe_gemm_q8_q4k<2, RG>), grid, dim3(kQmThreads), 0, s, a);
    else hipLaunchKernelGGL((k_moe_gemm_q8_q4k<3, RG>), grid, dim3(kQmThreads), 0, s, a);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

// ---- Q8_K activations (gemv.hip:686-705): one scale per 256 weights, int16 sums per 32 ------------
// q [ncol][K] int8, d [K/256][16] f32, bs [K/256][16][8] int16; workgroup (block b, column c):
// d = amax/127 over the 256 values, q = rne(x * 127/amax) (0 when amax == 0), bs = sum of the 32 q.
__global__ void __launch_bounds__(256) k_quantize_x_q8k(const float* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ d,
                                                        int16_t* __restrict__ bs, int K) {
    __shared__ float red[8];
    const int b = blockIdx.x, col = blockIdx.y, tid = threadIdx.x, hw = tid >> 5, l = tid & 31;
    const size_t k = (size_t)col * K + (size_t)b * 256 + tid;
    const float v = x[k];
    const float m32 = g32_max(fabsf(v));
    if (l == 0) red[hw] = m32;
    __syncthreads();
    float amax = red[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) amax = fmaxf(amax, red[i]);
    const float dd = amax / 127.f, id = amax > 0.f ? 127.f / amax : 0.f;
    const int qi = __float2int_rn(v * id);
    const int sum = g32_isum(qi);
    q[k] = (int8_t)qi;
    if (l == 0) bs[((size_t)b * 16 + col) * 8 + hw] = (int16_t)sum;
    if (tid == 0) d[(size_t)b * 16 + col] = dd;
}

// q8 GEMV on Q8_K activations: the fmt_rows arithmetic with each sub-block's (d, s) = (block scale,
// block scale * bs); y[c][n] for c in [c0, c0 + NC).
template <int F, int NC, int NIT>
__global__ void __launch_bounds__(kCThreads) k_gemv_q8k(const uint8_t* __restrict__ W, const int8_t* __restrict__ q,
                                                        const float* __restrict__ d, const int16_t* __restrict__ bs,
                                                        float* __restrict__ y, int N, int K, int c0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kCWaves + wave) * kCRpw;
    XSrcQ8K src[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) src[c] = XSrcQ8K{q + (size_t)(c0 + c) * K, d, bs, c0 + c};
    float acc[kCRpw][NC];
    fmt_rows<F, NC, NIT, kCRpw>(W, row0, N, K, src, acc, 0, fmt_units<F>(K));
#pragma unroll
    for (int r = 0; r < kCRpw; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = wave_sum(acc[r][c]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < kCRpw; ++r)
            if (row0 + r < N) {
#pragma unroll
                for (int c = 0; c < NC; ++c) y[(size_t)(c0 + c) * N + row0 + r] = acc[r][c];
            }
    }
}

template <int F>
int launch_q8k(const void* W, const qmm_xq8k& x, float* y, int N, int K, int ncol, hipStream_t s) {
    const dim3 grid((unsigned)((N + kCWaves * kCRpw - 1) / (kCWaves * kCRpw)));
    const int per_lane = (fmt_units<F>(K) + 63) / 64;
    for (int c0 = 0; c0 < ncol; c0 += kCCols) {
        const int nc = std::min(kCCols, ncol - c0);
#define QMM_QK(NC, NIT) hipLaunchKernelGGL((k_gemv_q8k<F, NC, NIT>), grid, dim3(kCThreads), 0, s, (const uint8_t*)W, x.q, x.d, x.bs, y, N, K, c0)
#define QMM_QKN(NIT) switch (nc) { case 1: QMM_QK(1, NIT); break; case 2: QMM_QK(2, NIT); break; case 3: QMM_QK(3, NIT); break; \
                                   case 4: QMM_QK(4, NIT); break; case 5: QMM_QK(5, NIT); break; case 6: QMM_QK(6, NIT); break; \
                                   case 7: QMM_QK(7, NIT); break; default: QMM_QK(8, NIT); break; }
        if (per_lane <= 1) { QMM_QKN(1) } else { QMM_QKN(2) }
#undef QMM_QKN
#undef QMM_QK
        QMM_LAUNCH_CHECK();
    }
    return QMM_OK;
}

// K granule of a format for these kernels (the block formats whole 256-weight blocks; Q6_K_SOA
// 512 so that its rows stay dword aligned; the 32-weight SoA formats as qmm_gemv_q8)
int kgran(int f) {
    switch (f) {
        case QMM_Q8_0_SOA: return 64;
        case QMM_Q5_1_SOA: return 32;
        case QMM_Q6_K_SOA: return 512;
        default: return 256;
    }
}

}  // namespace
}  // namespace qmm

using namespace qmm;

extern "C" {

int qmm_gemv_splitk(int fmt, const void* W, qmm_xq8 x, float* part, int N, int K, int ksplit, int ncol, void* stream) {
    if (!W || !x.q || !x.d || !x.s || !part) return QMM_ERR_NULL;
    if (N <= 0 || K <= 0 || K % kgran(fmt) != 0 || ncol < 1 || ksplit < 1 || ksplit > (K + 255) / 256) return QMM_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    switch (fmt) {
        case QMM_Q4_K: return launch_splitk<QMM_Q4_K>(W, x, part, N, K, ksplit, ncol, s);
        case QMM_Q5_K: return launch_splitk<QMM_Q5_K>(W, x, part, N, K, ksplit, ncol, s);
        case QMM_IQ4_XS: return launch_splitk<QMM_IQ4_XS>(W, x, part, N, K, ksplit, ncol, s);
        case QMM_Q6_K_SOA: return launch_splitk<QMM_Q6_K_SOA>(W, x, part, N, K, ksplit, ncol, s);
        case QMM_Q8_0_SOA: return launch_splitk<QMM_Q8_0_SOA>(W, x, part, N, K, ksplit, ncol, s);
        case QMM_Q5_1_SOA: return launch_splitk<QMM_Q5_1_SOA>(W, x, part, N, K, ksplit, ncol, s);
        default: return QMM_ERR_FORMAT;
    }
}

// the Flash-Next hyper-connection prologue is a neighbour of the path, not part of it (declared only)
int qmm_hc_up_fused(const void*, const float*, int, float*, int, int, void*) { return QMM_ERR_UNSUPPORTED; }

int qmm_moe_gemm_q8(int fmt, int shared_fmt, const void* W, const void* Wsh, size_t ebytes, const qmm_moe_tile* tiles, int ntiles,
                    const qmm_moe_tile* stiles, int nstiles, int ct, const int* rowtab, qmm_xq8 x, float* y, int N, int K,
                    void* stream) {
    auto fmt_ok = [](int f) { return f == QMM_Q4_K || f == QMM_Q5_K || f == QMM_IQ4_XS || f == QMM_Q8_0_SOA || f == QMM_Q5_1_SOA; };
    if (!fmt_ok(fmt) || (nstiles > 0 && !fmt_ok(shared_fmt))) return QMM_ERR_FORMAT;
    if (!x.q || !x.d || !x.s || !y || (ntiles > 0 && (!W || !tiles)) || (nstiles > 0 && (!Wsh || !stiles))) return QMM_ERR_NULL;
    if (N <= 0 || K <= 0 || K % kgran(fmt) != 0 || (nstiles > 0 && K % kgran(shared_fmt) != 0) || ntiles < 0 || nstiles < 0 ||
        ct < 1 || ntiles > 65535 || nstiles > 65535)
        return QMM_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    // Q4_K tile lists run on the int8 matrix cores (routed and shared tiles in one launch when both are
    // Q4_K); the other formats on the q8 GEMV units
    const bool mr = fmt == QMM_Q4_K, ms = nstiles > 0 && shared_fmt == QMM_Q4_K;
    if (mr && ms && ntiles + nstiles > 65535) {              // one grid row per tile: two launches
        int rc = launch_moe_q8_q4k(W, Wsh, ebytes, tiles, ntiles, stiles, 0, ct, rowtab, x, y, N, K, s);
        if (rc == QMM_OK) rc = launch_moe_q8_q4k(W, Wsh, ebytes, tiles, 0, stiles, nstiles, ct, rowtab, x, y, N, K, s);
        if (rc != QMM_OK) return rc;
    } else if (mr || ms) {
        const int rc = launch_moe_q8_q4k(W, Wsh, ebytes, tiles, mr ? ntiles : 0, stiles, ms ? nstiles : 0, ct, rowtab, x, y, N, K, s);
        if (rc != QMM_OK) return rc;
    }
    if (!mr) {
        const int rc = moe_q8_dispatch(fmt, W, Wsh, ebytes, tiles, ntiles, rowtab, x, y, N, K, s);
        if (rc != QMM_OK) return rc;
    }
    if (!ms) return moe_q8_dispatch(shared_fmt, Wsh, Wsh, 0, stiles, nstiles, rowtab, x, y, N, K, s);
    return QMM_OK;
}

int qmm_quantize_x_q8k(const float* x, qmm_xq8k out, int ncol, int K, void* stream) {
    if (!x || !out.q || !out.d || !out.bs) return QMM_ERR_NULL;
    if (K <= 0 || K % 256 != 0 || ncol < 1 || ncol > 16) return QMM_ERR_SHAPE;
    hipLaunchKernelGGL(k_quantize_x_q8k, dim3((unsigned)(K / 256), (unsigned)ncol), dim3(256), 0, (hipStream_t)stream, x, out.q,
                       out.d, out.bs, K);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_gemv_q8k(const qmm_gemv_seg* segs, int nseg, qmm_xq8k x, int ncol, void* stream) {
    if (!segs || !x.q || !x.d || !x.bs) return QMM_ERR_NULL;
    if (nseg < 1 || ncol < 1 || ncol > 16) return QMM_ERR_SHAPE;
    for (int i = 0; i < nseg; ++i) {
        const qmm_gemv_seg& g = segs[i];
        if (!g.w || !g.y) return QMM_ERR_NULL;
        if (g.N <= 0 || g.K <= 0 || g.K % 256 != 0 || g.K % kgran(g.fmt) != 0 || g.K != segs[0].K) return QMM_ERR_SHAPE;
        if (!(g.fmt == QMM_Q4_K || g.fmt == QMM_Q5_K || g.fmt == QMM_IQ4_XS || g.fmt == QMM_Q6_K_SOA || g.fmt == QMM_Q8_0_SOA))
            return QMM_ERR_FORMAT;
    }
    hipStream_t s = (hipStream_t)stream;
    for (int i = 0; i < nseg; ++i) {
        const qmm_gemv_seg& g = segs[i];
        int rc = QMM_ERR_FORMAT;
        switch (g.fmt) {
            case QMM_Q4_K: rc = launch_q8k<QMM_Q4_K>(g.w, x, g.y, g.N, g.K, ncol, s); break;
            case QMM_Q5_K: rc = launch_q8k<QMM_Q5_K>(g.w, x, g.y, g.N, g.K, ncol, s); break;
            case QMM_IQ4_XS: rc = launch_q8k<QMM_IQ4_XS>(g.w, x, g.y, g.N, g.K, ncol, s); break;
            case QMM_Q6_K_SOA: rc = launch_q8k<QMM_Q6_K_SOA>(g.w, x, g.y, g.N, g.K, ncol, s); break;
            case QMM_Q8_0_SOA: rc = launch_q8k<QMM_Q8_0_SOA>(g.w, x, g.y, g.N, g.K, ncol, s); break;
        }
        if (rc != QMM_OK) return rc;
    }
    return QMM_OK;
}

}  // extern "C"
