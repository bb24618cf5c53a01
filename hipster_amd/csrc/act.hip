// act.hip -- the activation producers that feed the quantized matmuls, on gfx950 (wave64):
//
//   this library              reference (engine/kernels)
//   qmm_add_rmsnorm_quant     add_rmsnorm_quant   ops.h:14, ops.hip:62-98,760-762
//   qmm_add_rmsnorm_bf16      add_rmsnorm_bf16    ops.h:18, ops.hip:111-120,763
//   qmm_silu_mul_quant        silu_mul_quant      ops.h:24, ops.hip:146-151,770-772
//   qmm_silu_mul_bf16         silu_mul_bf16       ops.h:20, ops.hip:131,765
//
// Norm rows reproduce the reference's 1024-thread workgroup (ops.hip:62-98,111-120): its thread t
// (wave32 w = t/32, lane t%32) owns elements t, t+1024, ..., accumulates their squares with fma in
// that order, and the row sum is block_sum1024's pairwise tree (xor butterfly over the 32 lanes of a
// wave32, then over the 32 wave sums), so the sum is bit for bit the reference's.  The one
// deliberate difference is the scale: 1/sqrt(mean + eps) is computed in double and rounded once
// (correctly rounded in all but astronomically rare cases, and reproducible off the GPU), where the
// reference calls rsqrtf, a hardware approximation within about 1 ulp whose exact value only the
// GPU that ran it knows.
//
// Two layouts play those 1024 logical threads:
//  - vector (rows of n <= 6144, n % 4 == 0, 16-byte aligned rows): 256 lanes, lane p holding logical
//    threads 4p..4p+3, whose elements 4p+k+1024c are contiguous: x, y, w and xn move as 16-byte
//    accesses, q as one dword, and a q8 sub-block is 8 lanes.  Logical lane 4(p&7)+k of logical
//    wave p>>3 makes the tree's steps 16, 8, 4 physical swizzles to lanes p^4, p^2, p^1 and its
//    steps 2, 1 additions inside the lane (k^2, then k^1): the same pairs in the same order;
//  - scalar (any other row up to 16384 values): 1024 lanes, lane t playing logical thread t.
// Both load x (+ y, written back) and w before the one barrier, so a row costs one memory round
// trip and moves the algorithmic bytes once.
#include "qmm_common.hpp"

namespace qmm {
namespace {

constexpr int kNormMaxN = 16384;
constexpr int kNormVecMaxN = 6144;       // 6 float4 per lane and array

// ---- vector layout -------------------------------------------------------------------------
template <int C, bool HASY>
__device__ __forceinline__ float norm_row4(float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ w,
                                           int n, float eps, float4 (&v)[C], float4 (&wv)[C], float* part) {
    const int p = threadIdx.x;
    float4 a[C], b[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {            // every load first (past the row: clamped, zeroed below)
        const int i = min(4 * p + 1024 * c, n - 4);
        a[c] = *(const float4*)(x + i);
        if (HASY) b[c] = *(const float4*)(y + i);
        wv[c] = *(const float4*)(w + i);
    }
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;   // logical threads 4p + 0..3
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int i = 4 * p + 1024 * c;
        float4 t = a[c];
        if (HASY) {
            t.x += b[c].x; t.y += b[c].y; t.z += b[c].z; t.w += b[c].w;
            if (i < n) *(float4*)(x + i) = t;
        }
        if (i >= n) t = make_float4(0.f, 0.f, 0.f, 0.f);   // a zero square adds nothing
        v[c] = t;
        s0 = fmaf(t.x, t.x, s0); s1 = fmaf(t.y, t.y, s1); s2 = fmaf(t.z, t.z, s2); s3 = fmaf(t.w, t.w, s3);
    }
    s0 += swz_xor<4>(s0); s1 += swz_xor<4>(s1); s2 += swz_xor<4>(s2); s3 += swz_xor<4>(s3);   // logical l^16
    s0 += swz_xor<2>(s0); s1 += swz_xor<2>(s1); s2 += swz_xor<2>(s2); s3 += swz_xor<2>(s3);   // l^8
    s0 += swz_xor<1>(s0); s1 += swz_xor<1>(s1); s2 += swz_xor<1>(s2); s3 += swz_xor<1>(s3);   // l^4
    const float wsum = (s0 + s2) + (s1 + s3);                                                  // l^2, l^1
    if ((p & 7) == 0) part[p >> 3] = wsum;
    __syncthreads();
    const float tot = hw32_sum(part[p & 31]);       // the same tree over the 32 wave sums
    return (float)(1.0 / sqrt((double)(tot / (float)n + eps)));
}

template <int C, bool HASY>
__global__ void __launch_bounds__(256) k_add_rmsnorm_q8v(float* __restrict__ x, const float* __restrict__ y,
                                                         const float* __restrict__ w, float* __restrict__ xn,
                                                         int8_t* __restrict__ q, float* __restrict__ qd, float* __restrict__ qs,
                                                         float2* __restrict__ qds, int n, float eps) {
    __shared__ float part[32];
    const size_t row = blockIdx.x;
    const int nsb = n >> 5;
    float4 v[C], wv[C];
    const float sc = norm_row4<C, HASY>(x + row * n, HASY ? y + row * n : nullptr, w, n, eps, v, wv, part);
    const int p = threadIdx.x;
    xn += row * n;
    int8_t* qr = q + row * n;
    float* dr = qd + row * nsb;
    float* sr = qs + row * nsb;
    float2* dsr = qds ? qds + row * nsb : nullptr;
    float4 o[C];
    float dd[C];
    uint32_t qp[C];
    int sm[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {            // q8 per 32 as hw32_quant, the sub-block in 8 lanes
        o[c] = make_float4(v[c].x * sc * wv[c].x, v[c].y * sc * wv[c].y, v[c].z * sc * wv[c].z, v[c].w * sc * wv[c].w);
        const float am = g8_max(fmaxf(fmaxf(fabsf(o[c].x), fabsf(o[c].y)), fmaxf(fabsf(o[c].z), fabsf(o[c].w))));
        dd[c] = am / 127.f;
        const float id = am > 0.f ? 127.f / am : 0.f;
        const int q0 = __float2int_rn(o[c].x * id), q1 = __float2int_rn(o[c].y * id), q2 = __float2int_rn(o[c].z * id),
                  q3 = __float2int_rn(o[c].w * id);
        qp[c] = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)q3 << 24);
        sm[c] = g8_isum(q0 + q1 + q2 + q3);
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int i = 4 * p + 1024 * c;
        if (i < n) {                         // uniform over the 8 lanes of a sub-block
            *(float4*)(xn + i) = o[c];
            *(uint32_t*)(qr + i) = qp[c];
            if ((p & 7) == 0) {
                const int sb = i >> 5;
                const float ss = dd[c] * (float)sm[c];
                dr[sb] = dd[c]; sr[sb] = ss;
                if (dsr) dsr[sb] = make_float2(dd[c], ss);
            }
        }
    }
}

template <int C, bool HASY>
__global__ void __launch_bounds__(256) k_add_rmsnorm_bf16v(float* __restrict__ x, const float* __restrict__ y,
                                                           const float* __restrict__ w, uint16_t* __restrict__ xb, int n,
                                                           float eps) {
    __shared__ float part[32];
    const size_t row = blockIdx.x;
    float4 v[C], wv[C];
    const float sc = norm_row4<C, HASY>(x + row * n, HASY ? y + row * n : nullptr, w, n, eps, v, wv, part);
    xb += row * n;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int i = 4 * threadIdx.x + 1024 * c;
        if (i < n) {
            const uint32_t lo = f2bf_bits(v[c].x * sc * wv[c].x) | (f2bf_bits(v[c].y * sc * wv[c].y) << 16);
            const uint32_t hi = f2bf_bits(v[c].z * sc * wv[c].z) | (f2bf_bits(v[c].w * sc * wv[c].w) << 16);
            *(uint2*)(xb + i) = make_uint2(lo, hi);
        }
    }
}

// ---- scalar layout (lane t = logical thread t) ------------------------------------------------
template <int J, bool HASY>
__device__ __forceinline__ float norm_row1(float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ w,
                                           int n, float eps, float (&v)[J], float (&wv)[J], float* part) {
    const int t = threadIdx.x, l = t & 31;
    float a[J], b[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = min(t + 1024 * j, n - 1);
        a[j] = x[i];
        if (HASY) b[j] = y[i];
        wv[j] = w[i];
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = t + 1024 * j;
        float u = a[j];
        if (HASY) {
            u += b[j];
            if (i < n) x[i] = u;
        }
        u = i < n ? u : 0.f;
        v[j] = u;
        ss = fmaf(u, u, ss);
    }
    ss = hw32_sum(ss);
    if (l == 0) part[t >> 5] = ss;
    __syncthreads();
    const float tot = hw32_sum(part[l]);
    return (float)(1.0 / sqrt((double)(tot / (float)n + eps)));
}

template <int J, bool HASY>
__global__ void __launch_bounds__(1024) k_add_rmsnorm_q8(float* __restrict__ x, const float* __restrict__ y,
                                                         const float* __restrict__ w, float* __restrict__ xn,
                                                         int8_t* __restrict__ q, float* __restrict__ qd, float* __restrict__ qs,
                                                         float2* __restrict__ qds, int n, float eps) {
    __shared__ float part[32];
    const size_t row = blockIdx.x;
    const int nsb = n >> 5;
    float v[J], wv[J];
    const float sc = norm_row1<J, HASY>(x + row * n, HASY ? y + row * n : nullptr, w, n, eps, v, wv, part);
    const int t = threadIdx.x, l = t & 31;
    xn += row * n;
    int8_t* qr = q + row * n;
    float* dr = qd + row * nsb;
    float* sr = qs + row * nsb;
    float2* dsr = qds ? qds + row * nsb : nullptr;
    float o[J], dd[J];
    int qi[J], sm[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {            // q8 per 32 as hw32_quant (element t + 1024j: sub-block 32j + t/32)
        o[j] = v[j] * sc * wv[j];
        const float am = g32_max(fabsf(o[j]));
        dd[j] = am / 127.f;
        const float id = am > 0.f ? 127.f / am : 0.f;
        qi[j] = __float2int_rn(o[j] * id);
        sm[j] = g32_isum(qi[j]);
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = t + 1024 * j;
        if (i < n) {                         // uniform over the half-wave (n % 32 == 0)
            xn[i] = o[j];
            qr[i] = (int8_t)qi[j];
            if (l == 0) {
                const int sb = i >> 5;
                const float ss = dd[j] * (float)sm[j];
                dr[sb] = dd[j]; sr[sb] = ss;
                if (dsr) dsr[sb] = make_float2(dd[j], ss);
            }
        }
    }
}

template <int J, bool HASY>
__global__ void __launch_bounds__(1024) k_add_rmsnorm_bf16(float* __restrict__ x, const float* __restrict__ y,
                                                           const float* __restrict__ w, uint16_t* __restrict__ xb, int n,
                                                           float eps) {
    __shared__ float part[32];
    const size_t row = blockIdx.x;
    float v[J], wv[J];
    const float sc = norm_row1<J, HASY>(x + row * n, HASY ? y + row * n : nullptr, w, n, eps, v, wv, part);
    xb += row * n;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = threadIdx.x + 1024 * j;
        if (i < n) xb[i] = (uint16_t)f2bf_bits(v[j] * sc * wv[j]);
    }
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// xq = q8(silu(g) * u) per 32 (ops.hip:146-151): one half-wave per sub-block.
__device__ __forceinline__ float silu_f(float x) { return x / (1.f + __expf(-x)); }

__global__ void __launch_bounds__(256) k_silu_mul_q8(const float* __restrict__ g, const float* __restrict__ u,
                                                     int8_t* __restrict__ q, float* __restrict__ d, float* __restrict__ s,
                                                     float2* __restrict__ ds, size_t nsb) {
    const size_t sb = (size_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int l = threadIdx.x & 31;
    if (sb >= nsb) return;                   // whole half-waves leave together
    const size_t i = sb * 32 + l;
    hw32_quant(silu_f(g[i]) * u[i], q, d, s, ds, sb, l);
}

// The same with four values per lane and eight lanes per sub-block: 16-byte loads of g and u, the
// four q8 bytes stored as one dword, two divisions per four values, 8-lane DPP reductions.  amax and the integer sum are
// exact whatever the reduction order, so the result is bit for bit that of k_silu_mul_q8.
// Needs g, u 16-byte and q 4-byte aligned (the host checks).
__global__ void __launch_bounds__(256) k_silu_mul_q8x4(const float* __restrict__ g, const float* __restrict__ u,
                                                       int8_t* __restrict__ q, float* __restrict__ d, float* __restrict__ s,
                                                       float2* __restrict__ ds, size_t nsb) {
    const size_t sb = (size_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    const int l = threadIdx.x & 7;
    if (sb >= nsb) return;                   // whole 8-lane groups leave together
    const size_t i = sb * 32 + l * 4;
    const float4 a = *(const float4*)(g + i), b = *(const float4*)(u + i);
    const float h0 = silu_f(a.x) * b.x, h1 = silu_f(a.y) * b.y, h2 = silu_f(a.z) * b.z, h3 = silu_f(a.w) * b.w;
    const float amax = g8_max(fmaxf(fmaxf(fabsf(h0), fabsf(h1)), fmaxf(fabsf(h2), fabsf(h3))));
    const float dd = amax / 127.f, id = amax > 0.f ? 127.f / amax : 0.f;
    const int q0 = __float2int_rn(h0 * id), q1 = __float2int_rn(h1 * id), q2 = __float2int_rn(h2 * id),
              q3 = __float2int_rn(h3 * id);
    const int sum = g8_isum(q0 + q1 + q2 + q3);
    *(uint32_t*)(q + i) = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
                          ((uint32_t)q3 << 24);
    if (l == 0) {
        const float ss = dd * (float)sum;
        d[sb] = dd; s[sb] = ss;
        if (ds) ds[sb] = make_float2(dd, ss);
    }
}

// out = bf16(silu(g) * u) (ops.hip:131), four elements per thread
__global__ void __launch_bounds__(256) k_silu_mul_bf16(const float* __restrict__ g, const float* __restrict__ u,
                                                       uint16_t* __restrict__ o, size_t n) {
    const size_t i0 = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i0 + 4 <= n && ((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(u)) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(o) & 7) == 0) {
        const float4 a = *(const float4*)(g + i0), b = *(const float4*)(u + i0);
        const uint32_t lo = f2bf_bits(silu_f(a.x) * b.x) | (f2bf_bits(silu_f(a.y) * b.y) << 16);
        const uint32_t hi = f2bf_bits(silu_f(a.z) * b.z) | (f2bf_bits(silu_f(a.w) * b.w) << 16);
        *(uint2*)(o + i0) = make_uint2(lo, hi);
        return;
    }
    for (size_t i = i0; i < n && i < i0 + 4; ++i) o[i] = (uint16_t)f2bf_bits(silu_f(g[i]) * u[i]);
}

}  // namespace
}  // namespace qmm

using namespace qmm;

extern "C" {

int qmm_add_rmsnorm_quant(float* x, const float* y, const float* w, float* xn, qmm_xq8 xq, int T, int n, float eps,
                          void* stream) {
    if (!x || !w || !xn || !xq.q || !xq.d || !xq.s) return QMM_ERR_NULL;
    if (T < 0 || n <= 0 || n % 32 != 0 || n > kNormMaxN) return QMM_ERR_SHAPE;
    if (T == 0) return QMM_OK;
    hipStream_t s = (hipStream_t)stream;
    float2* ds = (float2*)xq.ds;
    const bool vec = n <= kNormVecMaxN && aligned(x, 16) && (!y || aligned(y, 16)) && aligned(w, 16) && aligned(xn, 16) &&
                     aligned(xq.q, 4);
#define QMM_NORM_Q8(KER, C, NT)                                                                                          \
    do {                                                                                                              \
        if (y)                                                                                                        \
            hipLaunchKernelGGL((KER<C, true>), dim3(T), dim3(NT), 0, s, x, y, w, xn, xq.q, xq.d, xq.s, ds, n, eps);      \
        else                                                                                                          \
            hipLaunchKernelGGL((KER<C, false>), dim3(T), dim3(NT), 0, s, x, y, w, xn, xq.q, xq.d, xq.s, ds, n, eps);     \
    } while (0)
    if (vec)
        QMM_NORM_Q8(k_add_rmsnorm_q8v, 6, 256);
    else if (n <= 6144)
        QMM_NORM_Q8(k_add_rmsnorm_q8, 6, 1024);
    else
        QMM_NORM_Q8(k_add_rmsnorm_q8, 16, 1024);
#undef QMM_NORM_Q8
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_add_rmsnorm_bf16(float* x, const float* y, const float* w, uint16_t* xb, int T, int n, float eps, void* stream) {
    if (!x || !w || !xb) return QMM_ERR_NULL;
    if (T < 0 || n <= 0 || n > kNormMaxN) return QMM_ERR_SHAPE;
    if (T == 0) return QMM_OK;
    hipStream_t s = (hipStream_t)stream;
    const bool vec = n <= kNormVecMaxN && n % 4 == 0 && aligned(x, 16) && (!y || aligned(y, 16)) && aligned(w, 16) &&
                     aligned(xb, 8);
#define QMM_NORM_BF(KER, C, NT)                                                                                          \
    do {                                                                                                              \
        if (y)                                                                                                        \
            hipLaunchKernelGGL((KER<C, true>), dim3(T), dim3(NT), 0, s, x, y, w, xb, n, eps);                            \
        else                                                                                                          \
            hipLaunchKernelGGL((KER<C, false>), dim3(T), dim3(NT), 0, s, x, y, w, xb, n, eps);                           \
    } while (0)
    if (vec)
        QMM_NORM_BF(k_add_rmsnorm_bf16v, 6, 256);
    else if (n <= 6144)
        QMM_NORM_BF(k_add_rmsnorm_bf16, 6, 1024);
    else
        QMM_NORM_BF(k_add_rmsnorm_bf16, 16, 1024);
#undef QMM_NORM_BF
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_silu_mul_quant(const float* gate, const float* up, qmm_xq8 xq, int n, void* stream) {
    if (!gate || !up || !xq.q || !xq.d || !xq.s) return QMM_ERR_NULL;
    if (n < 0 || n % 32 != 0) return QMM_ERR_SHAPE;
    const size_t nsb = (size_t)n / 32;
    if (nsb == 0) return QMM_OK;
    const bool vec = ((reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up)) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(xq.q) & 3) == 0;
    if (vec)
        hipLaunchKernelGGL(k_silu_mul_q8x4, dim3((unsigned)((nsb + 31) / 32)), dim3(256), 0, (hipStream_t)stream, gate, up,
                           xq.q, xq.d, xq.s, (float2*)xq.ds, nsb);
    else
        hipLaunchKernelGGL(k_silu_mul_q8, dim3((unsigned)((nsb + 7) / 8)), dim3(256), 0, (hipStream_t)stream, gate, up,
                           xq.q, xq.d, xq.s, (float2*)xq.ds, nsb);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_silu_mul_bf16(const float* gate, const float* up, uint16_t* out, size_t n, void* stream) {
    if (!gate || !up || !out) return QMM_ERR_NULL;
    if (n == 0) return QMM_OK;
    const size_t blocks = (n + 1023) / 1024;
    if (blocks > 0x7fffffffu) return QMM_ERR_SHAPE;
    hipLaunchKernelGGL(k_silu_mul_bf16, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, gate, up, out, n);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

}  // extern "C"
