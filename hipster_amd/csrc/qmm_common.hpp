// qmm_common.hpp -- device helpers shared by the gfx950 kernels of libhipster_qmm.
// Wave64 throughout (CDNA4).  Nothing here allocates; all state lives in caller buffers.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hipster_qmm.h"

namespace qmm {

constexpr int kWave = 64;

// 16-byte and 8-byte vectors that only promise 4-byte alignment: GGUF Q6_K rows (210-byte
// blocks) are 2- or 4-byte aligned, and CDNA global loads accept dword-aligned multi-dword
// accesses, so these still compile to one global_load_dwordx4 / dwordx2.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffffu)));
}
__device__ __forceinline__ uint4 ld16(const void* p) { return *(const uint4*)p; }
__device__ __forceinline__ uint4 ld16_a4(const void* p) {
    const u32x4_a4 v = *(const u32x4_a4*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);   // v_dot4_i32_i8
}
__device__ __forceinline__ uint32_t alignbyte(uint32_t hi, uint32_t lo, uint32_t shift_bytes) {
    return __builtin_amdgcn_alignbyte(hi, lo, shift_bytes);     // ({hi,lo} >> 8*shift)[31:0]
}

// The 12 packed scale bytes of a Q4_K block (engine/src/quant.h:37-40) as four byte-vectors:
// sc[0..3], sc[4..7], m[0..3], m[4..7].  For j<4 the 6-bit values sit in bytes j / j+4; for j>=4
// the low nibble of byte j+4 carries the low 4 bits and the top two bits of byte j-4 (scale) or
// byte j (min) carry bits 4-5.
struct Q4kScaleBytes { uint32_t sc_lo, sc_hi, m_lo, m_hi; };
__device__ __forceinline__ Q4kScaleBytes q4k_scale_bytes(uint32_t s0, uint32_t s1, uint32_t s2) {
    Q4kScaleBytes r;
    r.sc_lo = s0 & 0x3f3f3f3fu;
    r.m_lo = s1 & 0x3f3f3f3fu;
    r.sc_hi = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
    r.m_hi = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
    return r;
}
// byte i (0..7) of the 8-byte vector {lo, hi}
__device__ __forceinline__ uint32_t byte8(uint32_t lo, uint32_t hi, int i) {
    const uint32_t v = i < 4 ? lo : hi;
    return (v >> (8 * (i & 3))) & 0xffu;
}

// the 16 signed levels of IQ4 (quant.h:35) as bytes, four per little-endian word: levels 0-3, 4-7,
// 8-11, 12-15
constexpr uint32_t kIq4L0 = 0xBFAD9881u, kIq4L1 = 0xF6EADDCFu, kIq4H0 = 0x26190D01u, kIq4H1 = 0x71594535u;
// four nibbles (one per byte, 0..15) -> four signed levels: one byte permute per half of the table,
// then a per-byte select on bit 3
__device__ __forceinline__ uint32_t iq4_levels4(uint32_t nib) {
    const uint32_t sel = nib & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kIq4L1, kIq4L0, sel), hi = __builtin_amdgcn_perm(kIq4H1, kIq4H0, sel);
    const uint32_t m = ((nib >> 3) & 0x01010101u) * 0xffu;
    return (hi & m) | (lo & ~m);
}
// Q6_K: 6-bit values (0..63, one per byte) -> signed q-32 per byte without carries between bytes.
__device__ __forceinline__ uint32_t q6_signed(uint32_t q) { return (q + 0x60606060u) ^ 0x80808080u; }

// v / d for 0 <= v < 2^20, d >= 1, rd = 1 / d within a few ulp: the float quotient is then within 1/4
// of v / d, so its truncation is off by at most one, which the two integer checks correct
__device__ __forceinline__ int div_small(int v, int d, float rd) {
    int c = (int)((float)v * rd);
    c += (c + 1) * d <= v;
    c -= c * d > v;
    return c;
}

// LDS byte address of a pointer into __shared__ memory
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Global -> LDS DMA of 16 bytes per lane (global_load_lds_dwordx4): lane i writes lds + 16*i, lds
// wave-uniform.  Issued as inline assembly on purpose: the compiler tracks the builtin form as an
// LDS store and, unable to tell the stages of a ring apart, puts s_waitcnt vmcnt(0) before the next
// LDS read, which waits for the DMA just issued for a later step and serialises the prefetch.  The
// callers order DMA and LDS reads themselves (s_waitcnt vmcnt(n), then a barrier).  Loads the
// compiler issues itself stay correct: a vmcnt it computes without counting these only waits longer.
//
// Every inline-assembly memory instruction here starts with s_nop 4 (5 wait states).  The compiler
// cannot see that the assembly is a vector memory instruction, so it does not insert the wait states
// the ISA requires between a VALU write of an SGPR and a vector memory instruction reading it (5),
// or between an SALU write of M0 and an LDS DMA (1).  Without them a base address the compiler has
// just reloaded with v_readlane (an SGPR spill) or moved into M0 can be read stale: a garbage global
// address or LDS slot.
#define QMM_VMEM_ASM_GUARD "s_nop 4\n\t"
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
    asm volatile(QMM_VMEM_ASM_GUARD "global_load_lds_dwordx4 %0, off" : : "v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
// The same with a wave-uniform 64-bit base in SGPRs and a per-lane 32-bit byte offset: per-step
// address changes then cost scalar adds only.  base and lds must be wave-uniform.
__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile(QMM_VMEM_ASM_GUARD "global_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(base), "{m0}"(lds) : "memory");
}

// A value the optimiser cannot see through (keeps a byte mask from being folded into the
// byte-select of v_cvt_f32_ubyte{1,2,3}, which would turn each conversion into bfe + cvt)
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm("" : "+v"(v));
    return v;
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() is a release/acquire fence
// at workgroup scope over all address spaces, which makes every wave wait for all of its
// outstanding global loads (vmcnt(0)) before the barrier; a kernel that issued its weight loads
// ahead of the barrier would lose all overlap.  With the fences restricted to LDS ("local") the
// barrier waits for LDS traffic only.  The scheduling barriers keep the compiler from hoisting
// work that consumes those loads above the barrier (which would reintroduce the wait).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_sched_barrier(0);
}

// Stage q8 x of NCOL columns into LDS: [xq NCOL*K][xd NCOL*K/32][xs NCOL*K/32].
template <int NCOL>
__device__ __forceinline__ void stage_xq8(uint8_t* lds, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                          const float* __restrict__ xs, int K) {
    const int nq = NCOL * K / 16, ns = NCOL * (K / 32) / 4;
    uint4* dq = (uint4*)lds;
    for (int i = threadIdx.x; i < nq; i += blockDim.x) dq[i] = ld16(xq + (size_t)i * 16);
    float4* dd = (float4*)(lds + (size_t)NCOL * K);
    float4* dsv = dd + ns;
    for (int i = threadIdx.x; i < ns; i += blockDim.x) {
        dd[i] = *(const float4*)(xd + (size_t)i * 4);
        dsv[i] = *(const float4*)(xs + (size_t)i * 4);
    }
    __syncthreads();
}

// ---- wave reductions (wave64) ----
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, width);
    return v;
}

// ---- half-wave (32-lane) butterflies ----
// ds_swizzle in bit mode (offset[15] = 0: and_mask 0x1f, or_mask 0, xor_mask O) reads lane l^O
// within each group of 32 lanes without touching LDS memory.
template <int O>
__device__ __forceinline__ float swz_xor(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (O << 10) | 0x1f));
}
// Reductions whose result does not depend on the order (max, integer sum) over 8 or 32 lanes, on the
// VALU instead of the LDS pipe: DPP quad_perm [1,0,3,2] and [2,3,0,1] (lanes l^1, l^2), row_half_mirror
// (lane 7-l of each 8-lane half-row: the other quad), row_mirror (lane 15-l of each 16-lane row: the
// other half-row), then v_permlane16_swap, which exchanges the odd rows of one operand with the even
// rows of the other: swapping a value with itself yields the row pair (r0, r1) in one result and
// (r1, r0) in the other, so combining the two gives every lane of a half-wave its 32-lane total.
// Every source lane lies inside the group being reduced.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false); }
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) { return __int_as_float(dpp_i<CTRL>(__float_as_int(v))); }
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;
constexpr int kDppQuadReverse = 0x1B, kDppRor8 = 0x128;

// The 32-lane sum as the pairwise tree that pairs lane l with l^16 first, then l^8, l^4, l^2, l^1
// (every lane of the half-wave ends with the same value; addition commutes, so both partners of a
// step compute the same sum), with the partners read on the VALU: l^16 from v_permlane16_swap of the
// value with itself (one result holds row r, the other row r^1: their sum is the step), l^8 by a
// rotation of the 16-lane row by 8, l^4 as (l^7)^3 (row_half_mirror, then the reversed quad), l^2 and
// l^1 by quad permutes.  The same partners as the xor swizzles, so the same bits.
__device__ __forceinline__ float hw32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    v += dpp_f<kDppRor8>(v);
    v += dpp_f<kDppQuadReverse>(dpp_f<kDppHalfMirror>(v));
    v += dpp_f<kDppXor2>(v);
    v += dpp_f<kDppXor1>(v);
    return v;
}

__device__ __forceinline__ float g8_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v)); v = fmaxf(v, dpp_f<kDppXor2>(v));
    return fmaxf(v, dpp_f<kDppHalfMirror>(v));
}
__device__ __forceinline__ int g8_isum(int v) {
    v += dpp_i<kDppXor1>(v); v += dpp_i<kDppXor2>(v);
    return v + dpp_i<kDppHalfMirror>(v);
}
__device__ __forceinline__ float g32_max(float v) {
    v = g8_max(v);
    v = fmaxf(v, dpp_f<kDppMirror>(v));
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ int g32_isum(int v) {
    v = g8_isum(v);
    v += dpp_i<kDppMirror>(v);
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    return (int)r[0] + (int)r[1];
}

// q8 per 32 (engine/kernels/ops.hip:48-59, == gemv.hip:36-51): lane l of a half-wave holds value l
// of sub-block sb.  d = amax/127, id = 127/amax (0 when amax == 0), q = round-half-even(v*id),
// s = d * sum(q); ds (optional) receives the packed (d, s) pair.
__device__ __forceinline__ void hw32_quant(float v, int8_t* __restrict__ q, float* __restrict__ d, float* __restrict__ s,
                                           float2* __restrict__ ds, size_t sb, int l) {
    const float amax = g32_max(fabsf(v));
    const float dd = amax / 127.f, id = amax > 0.f ? 127.f / amax : 0.f;
    const int qi = __float2int_rn(v * id);
    const int sum = g32_isum(qi);
    q[sb * 32 + l] = (int8_t)qi;
    if (l == 0) {
        const float ss = dd * (float)sum;
        d[sb] = dd; s[sb] = ss;
        if (ds) ds[sb] = make_float2(dd, ss);
    }
}

// MoE decode dedup over the slots of a step, run by the 64 lanes of the first wave: slot te leads its
// expert when no earlier slot routes to it (the shared expert: every id < 0); the leader lists, in
// order, every slot >= te routed to the same expert (at most 64) in s_cols[0..*s_n).  *s_dup = 1
// when te does not lead.
__device__ __forceinline__ void moe_slot_columns(const int* __restrict__ ids, int nslot, int te, int id, int* s_cols,
                                                 int* s_n, int* s_dup) {
    const int tid = threadIdx.x;
    int n = 0, dup = 0;
    for (int base = 0; base < nslot; base += 64) {
        const int sl = base + tid;
        const int sid0 = ids[min(sl, nslot - 1)];
        const int sid = sl < nslot ? sid0 : 0x7fffffff;
        const bool m = sl < nslot && (sid == id || (sid < 0 && id < 0));
        const unsigned long long bal = __ballot(m);
        // slots before te that match -> duplicate
        const unsigned long long before = base + 64 <= te ? ~0ull : (te > base ? ((1ull << (te - base)) - 1ull) : 0ull);
        if (bal & before) dup = 1;
        // slots >= te that match, in order
        const unsigned long long from = te <= base ? ~0ull : (te - base >= 64 ? 0ull : ~((1ull << (te - base)) - 1ull));
        unsigned long long mm = bal & from;
        while (mm && n < 64) {
            const int b = __builtin_ctzll(mm);
            if (tid == 0) s_cols[n] = base + b;
            ++n;
            mm &= mm - 1;
        }
    }
    if (tid == 0) { *s_n = n; *s_dup = dup; }
}
constexpr int kMoeMaxSlots = 16;    // slots per token (10 routed + shared in the reference)

// bf16 round-to-nearest-even of the top half (no NaN special case, as engine/kernels/gemm.hip:12)
__device__ __forceinline__ uint32_t f2bf_bits(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }

// ---- host side ----------------------------------------------------------------------------
// CUs of the current device (cached after the first call)
inline int device_cu_count() {
    static int n = 0;
    if (n == 0) {
        int dev = 0, v = 0;
        n = (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) ? v : 256;
    }
    return n;
}
// D[m][n] (row stride ldd) = A[m][:] . dequant(W[n][:]) for m < M, n < N with the grouped-GEMM kernel of
// moe_prefill.hip over implicit tiles of `trows` consecutive rows (one Q4_K matrix, no row gather):
// the dense GEMM hands it the columns that would leave its last round of 256 x 256 tiles thin.
int launch_q4k_rows_gemm(const void* W, const uint16_t* A, float* D, int M, int N, int K, int ldd, int trows, hipStream_t s);
// q8 GEMV of gemv_fmt.hip for QMM_Q5_K, QMM_IQ4_XS, QMM_Q8_0_SOA, QMM_Q5_1_SOA (ncol 1..8, K % 256 == 0)
int gemv_fmt_dispatch(int fmt, const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, hipStream_t s);
int gemv_il_dispatch(int rows, int fmt, const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, hipStream_t s);
int gemv_fmt_dispatch_segs(int fmt, const qmm_gemv_seg* segs, int nseg, qmm_xq8 x, int K, int ncol, hipStream_t s);
// prefill grouped GEMM (qmm_moe_gemm_bf16) for the formats other than all-Q4_K (moe_gemm_fmt.hip)
int launch_moe_gemm_fmt(int fmt, int sfmt, const void* W, const void* Wsh, size_t ebytes, const qmm_moe_tile* tiles,
                        const int* counts, int max_tiles, const int* rowtab, const uint16_t* A, float* D, int N, int K,
                        hipStream_t s);
// Q4_K GEMV of 1..16 columns over 1..4 segments sharing K on the int8 matrix cores, one launch
// (gemv_mfma.hip); bitwise the dot4 kernels.  The dispatch of gemv.hip sends Q4_K calls of at least
// g_mfma_min_ncol columns there.
int gemv_q4k_mfma(const qmm_gemv_seg* segs, int nseg, qmm_xq8 x, int K, int ncol, hipStream_t s);
size_t gemv_q4k_mfma_lds(int K, int ncol);     // its LDS bytes; it runs when they are <= kMfmaLdsMax
constexpr size_t kMfmaLdsMax = 120 * 1024;
extern int g_mfma_min_ncol;
// Q6_K_SOA GEMV of 2..8 columns on the int8 matrix cores (gemv_mfma.hip), bitwise the unit kernel;
// the dispatch sends Q6_K_SOA calls of at least g_q6_mfma_min_ncol columns there (K % 512 == 0,
// 16-byte aligned x scales)
int gemv_q6k_mfma(const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, hipStream_t s);
bool gemv_q6k_mfma_fits(int K, int ncol);     // its one-pass staging of x scales, block scales and d (K <= 20480)
extern int g_q6_mfma_min_ncol;
// Q8_0_SOA GEMV of 1..8 columns on the int8 matrix cores (gemv_mfma.hip), bitwise the unit kernel;
// the dispatch sends Q8_0_SOA calls of at least g_q80_mfma_min_ncol columns there when the kernel stages
// their x, d and x scales in one pass (gemv_q80_mfma_fits: ncol * K <= 40960, K <= 8192, K % 64 == 0)
// and the x scales are 8-byte aligned
int gemv_q80_mfma(const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, hipStream_t s);
bool gemv_q80_mfma_fits(int K, int ncol);
extern int g_q80_mfma_min_ncol;

// the MoE decode step of qmm_moe_decode (moe.hip): argument checks, and the two launches with the gate /
// up rows in gu (2 * T * (topk + 1) * F floats)
int moe_decode_check(int fmt, const void* Wg, const void* Wu, const void* Wd, const void* Sg, const void* Su, const void* Sd,
                     const float* logits, int stride, int nexp_total, int topk, qmm_xq8 x, int T, int H, int F, const int* ids,
                     const float* w, const float* y);
int moe_decode_run(const void* Wg, const void* Wu, const void* Wd, size_t ebytes_gu, size_t ebytes_d, const void* Sg, const void* Su,
                   const void* Sd, const float* logits, int stride, int nexp_total, int topk, qmm_xq8 x, int T, int H, int F, int* ids,
                   float* w, float* gu, float* y, hipStream_t s);
// MoE decode gather / down (qmm_gemv_moe) for the routed formats other than all-Q4_K (gemv_fmt.hip)
int moe_fmt_dispatch(int fmt, int sfmt, const qmm_moe_segs* a, int nseg, const int* ids, int nexp, qmm_xq8 x, int N, int K,
                     int T, int xrow_te, hipStream_t s);

// ------------------------------------------------------------------------------------------
// Q4_K nibbles -> bf16 through v_fma_mix_f32 (the grouped and dense prefill GEMMs)
typedef __bf16 qmm_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// fma(value of the f16 half, s, c) -- v_fma_mix_f32.  A half whose bits are a small integer q
// (exponent field 0) is the subnormal q * 2^-24, exactly, so with s = x * 2^24 the product is
// exactly q * x and the result is the single rounding of q * x + c: fmaf(x, q, c) bit for bit.
__device__ __forceinline__ float mix_lo(uint32_t v, float s, float c) {
    return __builtin_fmaf((float)__builtin_bit_cast(f16x2, v)[0], s, c);
}
__device__ __forceinline__ float mix_hi(uint32_t v, float s, float c) {
    return __builtin_fmaf((float)__builtin_bit_cast(f16x2, v)[1], s, c);
}
// 8 weights bf16(fma(dl, q, -ml)) from the nibbles of bytes 0..7 of {u0, u1} (k order = byte
// order).  m = 0x000f000f takes the low nibbles (s24 = dl * 2^24), m = 0x00f000f0 the high ones in
// place, 16q (s24 = dl * 2^20).  Bit for bit the dequantisation bf16(fmaf(dl, (float)q, -ml)) (RNE),
// in 17 VALU per 8 weights (byte-to-float conversions, fma and packing take 22).  Relies on f16
// subnormals being kept, the kernels' default mode (float_denorm_mode_16_64 = 3).
__device__ __forceinline__ qmm_bf16x8 q4_bf16x8_mix(uint32_t u0, uint32_t u1, uint32_t m, float s24, float c) {
    const uint32_t e0 = u0 & m, o0 = (u0 >> 8) & m, e1 = u1 & m, o1 = (u1 >> 8) & m;
    qmm_bf16x8 r;
    r[0] = (__bf16)mix_lo(e0, s24, c);
    r[1] = (__bf16)mix_lo(o0, s24, c);
    r[2] = (__bf16)mix_hi(e0, s24, c);
    r[3] = (__bf16)mix_hi(o0, s24, c);
    r[4] = (__bf16)mix_lo(e1, s24, c);
    r[5] = (__bf16)mix_lo(o1, s24, c);
    r[6] = (__bf16)mix_hi(e1, s24, c);
    r[7] = (__bf16)mix_hi(o1, s24, c);
    return r;
}

}  // namespace qmm

// Host-side launch check shared by the C-ABI wrappers.
#define QMM_LAUNCH_CHECK()                                                   \
    do {                                                                     \
        if (hipGetLastError() != hipSuccess) return QMM_ERR_LAUNCH;          \
    } while (0)
