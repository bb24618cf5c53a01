// router.hip -- the MoE router matmul on gfx950 (wave64), and the router matmul + routing in one call:
//
//   this library        reference
//   qmm_f32_gemv        fn::f32_gemv            engine/kernels/fn.h:37, fn.hip:251-277
//   qmm_moe_router      fn::f32_gemv + fn::moe_route (engine/src/qwen4exp.cpp:346-347)
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
