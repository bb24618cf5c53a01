// roofs.hip -- MI355X roof microbenchmarks behind bench.py --roofs (libhipster_roofs.so, separate from
// the product library).  The method of the reference's bench/roofline/bandwidth.hip (every thread
// streams 16-byte loads over a buffer and folds them into a register that is stored only when an
// impossible value comes out, so no load is dead) and wmma_rate.hip (register-only matrix
// instructions in independent accumulator chains, 8 waves per workgroup), re-targeted at gfx950:
//
//   qmm_roof_read  variant 0: grid-stride loop (bandwidth.hip); variant 1: each thread issues U
//                  loads up front, lanes of a wave on consecutive 16-byte pieces (the GEMV's
//                  pattern); variant 2: as 1 with nontemporal loads
//   qmm_roof_mfma  op 0: v_mfma_f32_32x32x16_bf16, 1: v_mfma_f32_16x16x32_bf16,
//                  2: v_mfma_i32_32x32x32_i8, 3: v_mfma_f32_32x32x2_f32, 4: v_mfma_i32_16x16x64_i8
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ void __launch_bounds__(256) k_read_stride(const uint4* __restrict__ p, size_t n, uint32_t* __restrict__ sink) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    for (; i < n; i += stride) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x7fffffffu) sink[0] = acc;
}

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

template <int U, bool NT>
__global__ void __launch_bounds__(256) k_read_burst(const uint4* __restrict__ p, size_t n, uint32_t* __restrict__ sink) {
    // workgroup w reads pieces [w * 256 * U, (w + 1) * 256 * U): load u of thread t is piece
    // base + u * 256 + t, so each load instruction of a wave covers 1 KiB of contiguous memory
    const size_t base = (size_t)blockIdx.x * 256 * U + threadIdx.x;
    u32x4v v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t i = base + (size_t)u * 256;
        const u32x4v* q = (const u32x4v*)(p + (i < n ? i : n - 1));
        if constexpr (NT) v[u] = __builtin_nontemporal_load(q);
        else v[u] = *q;
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == 0x7fffffffu) sink[0] = acc;
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef long i64x2 __attribute__((ext_vector_type(2)));

template <int OP>
__global__ void __launch_bounds__(512) k_mfma(float* __restrict__ out, int iters) {
    constexpr int CH = 4;            // independent accumulator chains per wave
    const float s = 0.001f * (float)threadIdx.x;
    bf16x8 a, b;
    for (int i = 0; i < 8; ++i) { a[i] = (__bf16)(s + 0.01f * i); b[i] = (__bf16)(0.002f * i); }
    i32x4 ai = {(int)(0x01020304u * (threadIdx.x + 1)), 0x05060708, 0x11223344, (int)threadIdx.x};
    f32x16 c[CH];
    f32x4 c4[CH];
    i32x16 ci[CH];
    i32x4 ci4[CH];
    for (int j = 0; j < CH; ++j) {
        for (int e = 0; e < 16; ++e) { c[j][e] = 0.f; ci[j][e] = 0; }
        for (int e = 0; e < 4; ++e) { c4[j][e] = 0.f; ci4[j][e] = 0; }
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            if constexpr (OP == 0) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[j], 0, 0, 0);
            else if constexpr (OP == 1) c4[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c4[j], 0, 0, 0);
            else if constexpr (OP == 2) ci[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ai, ai, ci[j], 0, 0, 0);
            else if constexpr (OP == 3) c[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(s, s, c[j], 0, 0, 0);
            else ci4[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ai, ai, ci4[j], 0, 0, 0);
        }
    }
    float t = 0.f;
    for (int j = 0; j < CH; ++j) t += c[j][0] + c4[j][0] + (float)ci[j][0] + (float)ci4[j][0];
    if (t == 12345.f) out[0] = t;
}

// LDS read rate: WAVES waves per workgroup (one workgroup per CU: 128 KiB of LDS), each issuing
// ds_read_b128 of 16 consecutive bytes per lane (conflict-free: a wave reads 1 KiB of consecutive
// addresses), 16 reads per iteration folded into registers stored only on an impossible value
template <int WAVES>
__global__ void __launch_bounds__(64 * WAVES) k_lds_read(uint32_t* __restrict__ sink, int iters) {
    __shared__ __align__(16) uint4 lds[8192];
    for (int i = threadIdx.x; i < 8192; i += 64 * WAVES) lds[i] = make_uint4(i, 3 * i, 5 * i, 7 * i);
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint4 acc = make_uint4(0, 0, 0, 0);
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const uint4 v = lds[((it * 16 + u) * 64 + wave * 1024 + lane) & 8191];
            acc.x ^= v.x; acc.y += v.y; acc.z ^= v.z; acc.w += v.w;
        }
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x12345678u) sink[0] = acc.x;
}

}  // namespace

extern "C" {

// variant 0: grid workgroups of 256 threads striding over the buffer; 1 / 2: U loads per thread,
// grid = ceil(bytes / (4096 U)) (unroll U in {4, 8, 16}).  Returns 0, or -1 on bad arguments / launch.
int qmm_roof_read(const void* src, size_t bytes, int variant, int grid, int unroll, uint32_t* sink, void* stream) {
    if (!src || !sink || bytes < 16) return -1;
    const size_t n = bytes / 16;
    hipStream_t s = (hipStream_t)stream;
    if (variant == 0) {
        if (grid < 1) return -1;
        hipLaunchKernelGGL(k_read_stride, dim3((unsigned)grid), dim3(256), 0, s, (const uint4*)src, n, sink);
    } else {
        const unsigned g = (unsigned)((n + 256 * (size_t)unroll - 1) / (256 * (size_t)unroll));
#define QMM_RB(U, NT) hipLaunchKernelGGL((k_read_burst<U, NT>), dim3(g), dim3(256), 0, s, (const uint4*)src, n, sink)
        const bool nt = variant == 2;
        switch (unroll) {
            case 4: if (nt) QMM_RB(4, true); else QMM_RB(4, false); break;
            case 8: if (nt) QMM_RB(8, true); else QMM_RB(8, false); break;
            case 16: if (nt) QMM_RB(16, true); else QMM_RB(16, false); break;
            default: return -1;
        }
#undef QMM_RB
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// grid workgroups of 8 waves, iters rounds of 4 independent matrix instructions per wave
int qmm_roof_mfma(int op, int iters, int grid, float* sink, void* stream) {
    if (!sink || iters < 1 || grid < 1) return -1;
    hipStream_t s = (hipStream_t)stream;
    switch (op) {
        case 0: hipLaunchKernelGGL(k_mfma<0>, dim3(grid), dim3(512), 0, s, sink, iters); break;
        case 1: hipLaunchKernelGGL(k_mfma<1>, dim3(grid), dim3(512), 0, s, sink, iters); break;
        case 2: hipLaunchKernelGGL(k_mfma<2>, dim3(grid), dim3(512), 0, s, sink, iters); break;
        case 3: hipLaunchKernelGGL(k_mfma<3>, dim3(grid), dim3(512), 0, s, sink, iters); break;
        case 4: hipLaunchKernelGGL(k_mfma<4>, dim3(grid), dim3(512), 0, s, sink, iters); break;
        default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// grid workgroups of `waves` waves (4, 8 or 16), iters rounds of 16 ds_read_b128 per wave
int qmm_roof_lds(int waves, int iters, int grid, uint32_t* sink, void* stream) {
    if (!sink || iters < 1 || grid < 1) return -1;
    hipStream_t s = (hipStream_t)stream;
    switch (waves) {
        case 4: hipLaunchKernelGGL(k_lds_read<4>, dim3(grid), dim3(256), 0, s, sink, iters); break;
        case 8: hipLaunchKernelGGL(k_lds_read<8>, dim3(grid), dim3(512), 0, s, sink, iters); break;
        case 16: hipLaunchKernelGGL(k_lds_read<16>, dim3(grid), dim3(1024), 0, s, sink, iters); break;
        default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
