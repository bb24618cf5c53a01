// gemv_fmt.hip -- q8-activation GEMV on gfx950 for the other weight formats of the call surface:
// Q5_K and IQ4_XS (GGUF blocks) and Q8_0_SOA / Q5_1_SOA (the engine's load-time row-SoA repacks of
// Q8_0 and Q5_1 / Q5_0 rows).  Reached through qmm_gemv_q8 / qmm_gemv_multi (gemv.hip), which is
// the reference's gemv_q8 / gemv_multi (engine/kernels/gemv.h:25,28) for these formats; the
// per-format arithmetic is the reference's (block decoders gemv.hip:90-163,214-268).
//
// RPW rows per wave (4; 2 for Q5_K).  A unit is one scale's worth of weights -- 32 (one sub-block) for IQ4_XS,
// Q8_0_SOA and Q5_1_SOA, 64 for Q5_K (the two sub-blocks sharing one 32-byte qs pair) -- and lane l
// takes units l, l + 64, ... of the row, NIT at a time, with all of a pass's weight loads issued
// before its compute.  The q8 x of a unit (32 bytes per sub-block, its d and s) is read from
// global memory (L1) once per wave and used for all of the wave's rows.  Per sub-block the
// weights become int8 lanes of a dword, the integer dot with the q8 x uses v_dot4_i32_i8, and the
// reference's fix-up follows:
//   Q5_K    acc += (d sc) xd isum - (dmin m) xs          (q = nibble | fifth bit << 4, 0..31)
//   IQ4_XS  acc += (d (ls - 32)) xd isum                 (q = level[nibble], signed)
//   Q8_0    acc += d xd isum
//   Q5_1    acc += d xd isum + m xs                      (q = nibble | fifth bit << 4)
// A lane accumulates its units in a fixed order and the wave reduces with a fixed butterfly, so a
// column's result does not depend on ncol (T-invariant).  K % 256 == 0 for the block formats, K % 64
// (Q8_0_SOA) or K % 32 (Q5_1_SOA) for the row-SoA ones (checked by the caller).
#include "qmm_common.hpp"

#include <hip/hip_runtime.h>

namespace qmm {
namespace {

constexpr int kFmtBlock = 256, kFmtWaves = kFmtBlock / 64;

template <int F>
__device__ __forceinline__ size_t fmt_row_bytes(int K) {
    if constexpr (F == QMM_Q4_K) return (size_t)K / 256 * 144;
    else if constexpr (F == QMM_Q5_K) return (size_t)K / 256 * 176;
    else if constexpr (F == QMM_IQ4_XS) return (size_t)K / 256 * 136;
    else if constexpr (F == QMM_Q8_0_SOA) return (size_t)K + (size_t)K / 16;
    else return (size_t)K / 32 * 24;                        // QMM_Q5_1_SOA
}
template <int F>
__host__ __device__ __forceinline__ int fmt_units(int K) { return (F == QMM_Q5_K || F == QMM_Q4_K) ? K / 64 : K / 32; }

// four bits h (0..15) -> bit 4 of each byte: h * 0x02040810 puts bit i of h at bit 8i + 4 (and the
// other partial products at positions that are not 4 mod 8, none overlapping), the mask keeps those
__device__ __forceinline__ uint32_t bits4_to_byte_bit4(uint32_t h) { return (h * 0x02040810u) & 0x10101010u; }

// 32 int8 weights (8 dwords) against 32 q8 x bytes
__device__ __forceinline__ int dot32(const uint32_t (&w)[8], const uint4 a, const uint4 b) {
    int s = sdot4(w[0], a.x, 0);
    s = sdot4(w[1], a.y, s);
    s = sdot4(w[2], a.z, s);
    s = sdot4(w[3], a.w, s);
    s = sdot4(w[4], b.x, s);
    s = sdot4(w[5], b.y, s);
    s = sdot4(w[6], b.z, s);
    return sdot4(w[7], b.w, s);
}

// q8 x of one 32-weight sub-block of one column: its 32 bytes, d and s
struct X32 { uint4 a, b; float d, s; };
__device__ __forceinline__ void x32_load(const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                         const float* __restrict__ xs, int sb, X32& x) {
    x.a = ld16(xq + 32 * (size_t)sb);
    x.b = ld16(xq + 32 * (size_t)sb + 16);
    x.d = xd[sb];
    x.s = xs[sb];
}

// ---- per-format unit: its raw weight bytes and load, its x, and its contribution to a column ----
// The loads (weights once, x per column) are issued before any arithmetic, so a unit never waits
// for one memory access after another.
template <int F> struct FmtUnit;

template <> struct FmtUnit<QMM_Q8_0_SOA> {            // row = [qs K][d (K/32) x f16]
    struct Raw { uint4 a, b; uint32_t d; };
    typedef X32 X;
    static __device__ __forceinline__ void load(const uint8_t* rp, int K, int u, Raw& r) {   // rows dword aligned
        r.a = ld16_a4(rp + 32 * (size_t)u);
        r.b = ld16_a4(rp + 32 * (size_t)u + 16);
        r.d = *(const uint16_t*)(rp + K + 2 * (size_t)u);
    }
    static __device__ __forceinline__ void xload(const int8_t* xq, const float* xd, const float* xs, int u, X& x) {
        x32_load(xq, xd, xs, u, x);
    }
    static __device__ __forceinline__ float col(const Raw& r, const X& x, int) {
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        return h2f(r.d) * x.d * (float)dot32(w, x.a, x.b);
    }
};

template <> struct FmtUnit<QMM_Q5_1_SOA> {            // row = [qs K/2][qh K/8][d K/32 x f16][m K/32 x f16]
    struct Raw { uint4 qs; uint32_t qh, d, m; };
    typedef X32 X;
    static __device__ __forceinline__ void load(const uint8_t* rp, int K, int u, Raw& r) {   // rows 8-byte aligned
        r.qs = ld16_a4(rp + 16 * (size_t)u);
        r.qh = *(const uint32_t*)(rp + K / 2 + 4 * (size_t)u);
        r.d = *(const uint16_t*)(rp + K / 2 + K / 8 + 2 * (size_t)u);
        r.m = *(const uint16_t*)(rp + K / 2 + K / 8 + K / 16 + 2 * (size_t)u);
    }
    static __device__ __forceinline__ void xload(const int8_t* xq, const float* xd, const float* xs, int u, X& x) {
        x32_load(xq, xd, xs, u, x);
    }
    static __device__ __forceinline__ float col(const Raw& r, const X& x, int) {
        // weight j (< 16): low nibble of qs byte j, fifth bit = qh bit j; weight j + 16: high nibble,
        // qh bit j + 16 (quant.h:82-88)
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            w[k] = (q[k] & 0x0f0f0f0fu) | bits4_to_byte_bit4((r.qh >> (4 * k)) & 0xfu);
            w[4 + k] = ((q[k] >> 4) & 0x0f0f0f0fu) | bits4_to_byte_bit4((r.qh >> (16 + 4 * k)) & 0xfu);
        }
        return h2f(r.d) * x.d * (float)dot32(w, x.a, x.b) + h2f(r.m) * x.s;
    }
};

template <> struct FmtUnit<QMM_IQ4_XS> {              // block = {f16 d, u16 scales_h, u8 scales_l[4], qs[128]}
    struct Raw { uint2 hd; uint4 qs; };
    typedef X32 X;
    static __device__ __forceinline__ void load(const uint8_t* rp, int, int u, Raw& r) {
        const uint8_t* blk = rp + (size_t)(u >> 3) * 136;
        r.hd = *(const uint2*)blk;
        r.qs = ld16_a4(blk + 8 + 16 * (u & 7));              // 136-byte blocks: 8-byte aligned
    }
    static __device__ __forceinline__ void xload(const int8_t* xq, const float* xd, const float* xs, int u, X& x) {
        x32_load(xq, xd, xs, u, x);
    }
    static __device__ __forceinline__ float col(const Raw& r, const X& x, int u) {
        const int ib = u & 7;
        const int ls = (int)((r.hd.y >> (4 * ib)) & 0xfu) | (int)(((r.hd.x >> (16 + 2 * ib)) & 3u) << 4);
        const float dl = h2f(r.hd.x) * (float)(ls - 32);
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            w[k] = iq4_levels4(q[k] & 0x0f0f0f0fu);            // weights 4k..4k+3
            w[4 + k] = iq4_levels4((q[k] >> 4) & 0x0f0f0f0fu); // weights 16+4k..
        }
        return dl * x.d * (float)dot32(w, x.a, x.b);
    }
};

template <> struct FmtUnit<QMM_Q5_K> {                // block = {f16 d, dmin, scales[12], qh[32], qs[128]}
    struct Raw { uint4 hd, h0, h1, q0, q1; };
    struct X { X32 lo, hi; };                          // sub-blocks 2j and 2j + 1
    static __device__ __forceinline__ void load(const uint8_t* rp, int, int u, Raw& r) {
        const uint8_t* blk = rp + (size_t)(u >> 2) * 176;     // 176-byte blocks: 16-byte aligned
        r.hd = ld16(blk);
        r.h0 = ld16(blk + 16);
        r.h1 = ld16(blk + 32);
        r.q0 = ld16(blk + 48 + 32 * (u & 3));
        r.q1 = ld16(blk + 64 + 32 * (u & 3));
    }
    static __device__ __forceinline__ void xload(const int8_t* xq, const float* xd, const float* xs, int u, X& x) {
        x32_load(xq, xd, xs, 2 * u, x.lo);                    // unit u = 4b + j: sub-blocks 8b + 2j = 2u, 2u + 1
        x32_load(xq, xd, xs, 2 * u + 1, x.hi);
    }
    static __device__ __forceinline__ float col(const Raw& r, const X& x, int u) {
        // pair j of block b: weights 64j + l (sub-block 2j) = low nibble of qs[32j + l] with bit 2j of
        // qh[l] as the fifth bit, 64j + 32 + l (sub-block 2j + 1) = high nibble with bit 2j + 1
        const int j = u & 3;
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t h[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
        uint32_t wl[8], wh[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            wl[k] = (q[k] & 0x0f0f0f0fu) | (((h[k] >> (2 * j)) & 0x01010101u) << 4);
            wh[k] = ((q[k] >> 4) & 0x0f0f0f0fu) | (((h[k] >> (2 * j + 1)) & 0x01010101u) << 4);
        }
        const int i0 = dot32(wl, x.lo.a, x.lo.b), i1 = dot32(wh, x.hi.a, x.hi.b);
        const float d = h2f(r.hd.x), dmin = h2f(r.hd.x >> 16);
        const Q4kScaleBytes s = q4k_scale_bytes(r.hd.y, r.hd.z, r.hd.w);
        const float d0 = d * (float)byte8(s.sc_lo, s.sc_hi, 2 * j), m0 = dmin * (float)byte8(s.m_lo, s.m_hi, 2 * j);
        const float d1 = d * (float)byte8(s.sc_lo, s.sc_hi, 2 * j + 1), m1 = dmin * (float)byte8(s.m_lo, s.m_hi, 2 * j + 1);
        return d0 * x.lo.d * (float)i0 - m0 * x.lo.s + (d1 * x.hi.d * (float)i1 - m1 * x.hi.s);
    }
};

template <> struct FmtUnit<QMM_Q4_K> {                // block = {f16 d, dmin, scales[12], qs[128]}
    struct Raw { uint4 hd, q0, q1; };
    struct X { X32 lo, hi; };                          // sub-blocks 2j and 2j + 1
    static __device__ __forceinline__ void load(const uint8_t* rp, int, int u, Raw& r) {
        const uint8_t* blk = rp + (size_t)(u >> 2) * 144;     // 144-byte blocks: 16-byte aligned
        r.hd = ld16(blk);
        r.q0 = ld16(blk + 16 + 32 * (u & 3));
        r.q1 = ld16(blk + 32 + 32 * (u & 3));
    }
    static __device__ __forceinline__ void xload(const int8_t* xq, const float* xd, const float* xs, int u, X& x) {
        x32_load(xq, xd, xs, 2 * u, x.lo);
        x32_load(xq, xd, xs, 2 * u + 1, x.hi);
    }
    static __device__ __forceinline__ float col(const Raw& r, const X& x, int u) {
        // pair j of block b (quant.h:44-53): weights 64j + l = low nibble of qs[32j + l] (sub-block
        // 2j), 64j + 32 + l = its high nibble (sub-block 2j + 1)
        const int j = u & 3;
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        uint32_t wl[8], wh[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            wl[k] = q[k] & 0x0f0f0f0fu;
            wh[k] = (q[k] >> 4) & 0x0f0f0f0fu;
        }
        const int i0 = dot32(wl, x.lo.a, x.lo.b), i1 = dot32(wh, x.hi.a, x.hi.b);
        const float d = h2f(r.hd.x), dmin = h2f(r.hd.x >> 16);
        const Q4kScaleBytes s = q4k_scale_bytes(r.hd.y, r.hd.z, r.hd.w);
        const float d0 = d * (float)byte8(s.sc_lo, s.sc_hi, 2 * j), m0 = dmin * (float)byte8(s.m_lo, s.m_hi, 2 * j);
        const float d1 = d * (float)byte8(s.sc_lo, s.sc_hi, 2 * j + 1), m1 = dmin * (float)byte8(s.m_lo, s.m_hi, 2 * j + 1);
        return d0 * x.lo.d * (float)i0 - m0 * x.lo.s + (d1 * x.hi.d * (float)i1 - m1 * x.hi.s);
    }
};

// RPW rows per wave: the q8 x of a unit is loaded once into registers and used by all RPW rows
// (x traffic per row / RPW; with one row per wave the x reads outweigh the weight bytes).  Column c
// reads its q8 x at xq[c], xd[c], xs[c]; acc[r][c] is lane-partial (the caller reduces over the wave).
template <int F, int NCOL, int NIT, int RPW>
__device__ __forceinline__ void fmt_rows(const uint8_t* __restrict__ W, int row0, int N, int K,
                                         const int8_t* const (&xq)[NCOL], const float* const (&xd)[NCOL],
                                         const float* const (&xs)[NCOL], float (&acc)[RPW][NCOL]) {
    typedef FmtUnit<F> FU;
    const int lane = threadIdx.x & 63;
    const size_t rb = fmt_row_bytes<F>(K);
    const int U = fmt_units<F>(K);
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int c = 0; c < NCOL; ++c) acc[r][c] = 0.f;
    for (int base = 0; base < U; base += 64 * NIT) {
        typename FU::Raw R[RPW][NIT];
        typename FU::X X[NIT];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int i = 0; i < NIT; ++i) FU::load(W + (size_t)min(row0 + r, N - 1) * rb, K, min(base + lane + 64 * i, U - 1), R[r][i]);
#pragma unroll
        for (int c = 0; c < NCOL; ++c) {
#pragma unroll
            for (int i = 0; i < NIT; ++i) FU::xload(xq[c], xd[c], xs[c], min(base + lane + 64 * i, U - 1), X[i]);
            // all loads issued before any arithmetic (the scheduler would otherwise sink each load
            // to its use to save registers, one memory latency after another)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < NIT; ++i) {
                const int u = base + lane + 64 * i;
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const float v = FU::col(R[r][i], X[i], min(u, U - 1));
                    acc[r][c] += u < U ? v : 0.f;
                }
            }
        }
    }
}

template <int F, int NCOL, int NIT, int RPW>
__global__ void __launch_bounds__(kFmtBlock) k_gemv_fmt(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                        const float* __restrict__ xd, const float* __restrict__ xs,
                                                        float* __restrict__ y, int N, int K) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kFmtWaves + wave) * RPW;
    const int nsb = K / 32;
    const int8_t* xqc[NCOL];
    const float *xdc[NCOL], *xsc[NCOL];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
        xqc[c] = xq + (size_t)c * K;
        xdc[c] = xd + (size_t)c * nsb;
        xsc[c] = xs + (size_t)c * nsb;
    }
    float acc[RPW][NCOL];
    fmt_rows<F, NCOL, NIT, RPW>(W, row0, N, K, xqc, xdc, xsc, acc);
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int c = 0; c < NCOL; ++c) acc[r][c] = wave_sum(acc[r][c]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r)
            if (row0 + r < N) {
#pragma unroll
                for (int c = 0; c < NCOL; ++c) y[(size_t)c * N + row0 + r] = acc[r][c];
            }
    }
}

// ---- MoE decode for the formats above (reference: gemv_moe, gemv.h:44, gemv.hip:1385-1394) ----
// Routed experts in format F, the shared expert in FS (F, or Q8_0_SOA as the reference allows).  A
// slot's rows are computed by fmt_rows like the plain GEMV of its expert (same per-row order, so
// the same bits as qmm_gemv_q8 on that expert), two rows per wave.
constexpr int kMoeRpw = 2, kMoeCols = 8;

template <int F, int FS, int NIT, int NC>
__device__ __forceinline__ void moe_fmt_pass(const uint8_t* wbase, bool shared, int row0, int N, int K, const int8_t* xq,
                                             const float* xd, const float* xs, const int* cols, int nc, int nexp,
                                             int xrow_te, float* __restrict__ y) {
    const int nsb = K / 32, lane = threadIdx.x & 63;
    const int8_t* xqc[NC];
    const float *xdc[NC], *xsc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int sl = cols[min(c, nc - 1)];
        const size_t xr = (size_t)(xrow_te ? sl : sl / nexp);
        xqc[c] = xq + xr * K;
        xdc[c] = xd + xr * nsb;
        xsc[c] = xs + xr * nsb;
    }
    float acc[kMoeRpw][NC];
    if (shared) fmt_rows<FS, NC, NIT, kMoeRpw>(wbase, row0, N, K, xqc, xdc, xsc, acc);
    else fmt_rows<F, NC, NIT, kMoeRpw>(wbase, row0, N, K, xqc, xdc, xsc, acc);
#pragma unroll
    for (int r = 0; r < kMoeRpw; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = wave_sum(acc[r][c]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < kMoeRpw; ++r)
            if (row0 + r < N) {
#pragma unroll
                for (int c = 0; c < NC; ++c)
                    if (c < nc) y[(size_t)cols[c] * N + row0 + r] = acc[r][c];
            }
    }
}

// gather (gate|up): grid = (row blocks of 4 waves x 2 rows, slots, segments).
template <int F, int FS, int NIT>
__global__ void __launch_bounds__(kFmtBlock) k_gemv_moe_fmt(qmm_moe_segs a, const int* __restrict__ ids, int nexp,
                                                            const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                            const float* __restrict__ xs, int N, int K, int nslot,
                                                            int xrow_te) {
    __shared__ int s_cols[64 + kMoeCols];
    __shared__ int s_n, s_dup;
    const int te = blockIdx.y, seg = blockIdx.z;
    const int id = ids[te];
    if (threadIdx.x < 64) moe_slot_columns(ids, nslot, te, id, s_cols, &s_n, &s_dup);
    __syncthreads();
    if (s_dup) return;
    const int ncols = s_n, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kFmtWaves + wave) * kMoeRpw;
    const uint8_t* wbase = id >= 0 ? (const uint8_t*)a.w[seg] + (size_t)id * a.ebytes : (const uint8_t*)a.shared[seg];
    float* y = a.y[seg];
    for (int c0 = 0; c0 < ncols; c0 += kMoeCols) {
        const int nc = min(kMoeCols, ncols - c0);
        const int* cols = s_cols + c0;
        if (nc == 1) moe_fmt_pass<F, FS, NIT, 1>(wbase, id < 0, row0, N, K, xq, xd, xs, cols, nc, nexp, xrow_te, y);
        else if (nc == 2) moe_fmt_pass<F, FS, NIT, 2>(wbase, id < 0, row0, N, K, xq, xd, xs, cols, nc, nexp, xrow_te, y);
        else if (nc <= 4) moe_fmt_pass<F, FS, NIT, 4>(wbase, id < 0, row0, N, K, xq, xd, xs, cols, nc, nexp, xrow_te, y);
        else moe_fmt_pass<F, FS, NIT, 8>(wbase, id < 0, row0, N, K, xq, xd, xs, cols, nc, nexp, xrow_te, y);
    }
}

// down projection + weighted combine: grid = (row blocks of 2 rows, tokens); wave w takes the slots
// e = w, w + 4, ... of the token; lane r < 2 then sums row r over the slots in order (the combine of
// the Q4_K kernel, the same expression).
template <int F, int FS, int NIT>
__global__ void __launch_bounds__(kFmtBlock) k_gemv_moe_down_fmt(qmm_moe_segs a, const int* __restrict__ ids, int nexp,
                                                                 const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                                 const float* __restrict__ xs, int N, int K) {
    __shared__ float vres[kMoeMaxSlots][kMoeRpw];
    const int tok = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int row0 = blockIdx.x * kMoeRpw, nsb = K / 32;
    for (int e = wave; e < nexp; e += kFmtWaves) {
        const int id = ids[tok * nexp + e];
        const uint8_t* wbase = id >= 0 ? (const uint8_t*)a.w[0] + (size_t)id * a.ebytes : (const uint8_t*)a.shared[0];
        const size_t xr = (size_t)tok * nexp + e;
        const int8_t* xqc[1] = {xq + xr * K};
        const float* xdc[1] = {xd + xr * nsb};
        const float* xsc[1] = {xs + xr * nsb};
        float acc[kMoeRpw][1];
        if (id < 0) fmt_rows<FS, 1, NIT, kMoeRpw>(wbase, row0, N, K, xqc, xdc, xsc, acc);
        else fmt_rows<F, 1, NIT, kMoeRpw>(wbase, row0, N, K, xqc, xdc, xsc, acc);
#pragma unroll
        for (int r = 0; r < kMoeRpw; ++r) {
            const float v = wave_sum(acc[r][0]);
            if (lane == 0) vres[e][r] = v;
        }
    }
    __syncthreads();
    if (tid < kMoeRpw && row0 + tid < N) {
        float acc = 0.f;
        for (int e = 0; e < nexp; ++e) acc += a.slotw[tok * nexp + e] * vres[e][tid];
        a.y[0][(size_t)tok * N + row0 + tid] = acc;
    }
}

template <int F, int FS>
int launch_moe_fmt(const qmm_moe_segs& a, int nseg, const int* ids, int nexp, qmm_xq8 x, int N, int K, int T, int xrow_te,
                   hipStream_t s) {
    const int per_lane = (max(fmt_units<F>(K), fmt_units<FS>(K)) + 63) / 64;
    if (a.slotw) {
        const dim3 grid((unsigned)((N + kMoeRpw - 1) / kMoeRpw), (unsigned)T);
        if (per_lane <= 1) hipLaunchKernelGGL((k_gemv_moe_down_fmt<F, FS, 1>), grid, dim3(kFmtBlock), 0, s, a, ids, nexp, x.q, x.d, x.s, N, K);
        else hipLaunchKernelGGL((k_gemv_moe_down_fmt<F, FS, 2>), grid, dim3(kFmtBlock), 0, s, a, ids, nexp, x.q, x.d, x.s, N, K);
    } else {
        const dim3 grid((unsigned)((N + kFmtWaves * kMoeRpw - 1) / (kFmtWaves * kMoeRpw)), (unsigned)(T * nexp), (unsigned)nseg);
        if (per_lane <= 1)
            hipLaunchKernelGGL((k_gemv_moe_fmt<F, FS, 1>), grid, dim3(kFmtBlock), 0, s, a, ids, nexp, x.q, x.d, x.s, N, K, T * nexp, xrow_te);
        else
            hipLaunchKernelGGL((k_gemv_moe_fmt<F, FS, 2>), grid, dim3(kFmtBlock), 0, s, a, ids, nexp, x.q, x.d, x.s, N, K, T * nexp, xrow_te);
    }
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

template <int F, int NCOL>
int launch_fmt(const void* W, qmm_xq8 x, float* y, int N, int K, hipStream_t s) {
    // rows per wave: 2 at one column (more waves in flight), 4 above (the shared x pays more), 2 for
    // Q5_K (its units hold 20 registers of raw weights)
    constexpr int RPW = (F == QMM_Q5_K || NCOL == 1) ? 2 : 4;
    const int grid = (N + kFmtWaves * RPW - 1) / (kFmtWaves * RPW);
    const int per_lane = (fmt_units<F>(K) + 63) / 64;
#define QMM_FMTL(IV) hipLaunchKernelGGL((k_gemv_fmt<F, NCOL, IV, RPW>), dim3(grid), dim3(kFmtBlock), 0, s, (const uint8_t*)W, x.q, x.d, x.s, y, N, K)
    // units per lane and pass: all of them when they are few, else passes of two (registers: RPW
    // rows x NIT units of raw weights are live at once)
    if (per_lane <= 1) QMM_FMTL(1);
    else if (per_lane == 3 && F != QMM_Q5_K) QMM_FMTL(3);
    else QMM_FMTL(2);
#undef QMM_FMTL
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

template <int NCOL>
int launch_fmt_ncol(int fmt, const void* W, qmm_xq8 x, float* y, int N, int K, hipStream_t s) {
    switch (fmt) {
        case QMM_Q5_K: return launch_fmt<QMM_Q5_K, NCOL>(W, x, y, N, K, s);
        case QMM_IQ4_XS: return launch_fmt<QMM_IQ4_XS, NCOL>(W, x, y, N, K, s);
        case QMM_Q8_0_SOA: return launch_fmt<QMM_Q8_0_SOA, NCOL>(W, x, y, N, K, s);
        case QMM_Q5_1_SOA: return launch_fmt<QMM_Q5_1_SOA, NCOL>(W, x, y, N, K, s);
        default: return QMM_ERR_FORMAT;
    }
}

}  // namespace

int gemv_fmt_dispatch(int fmt, const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, hipStream_t s) {
    switch (ncol) {
        case 1: return launch_fmt_ncol<1>(fmt, W, x, y, N, K, s);
        case 2: return launch_fmt_ncol<2>(fmt, W, x, y, N, K, s);
        case 3: return launch_fmt_ncol<3>(fmt, W, x, y, N, K, s);
        case 4: return launch_fmt_ncol<4>(fmt, W, x, y, N, K, s);
        case 5: return launch_fmt_ncol<5>(fmt, W, x, y, N, K, s);
        case 6: return launch_fmt_ncol<6>(fmt, W, x, y, N, K, s);
        case 7: return launch_fmt_ncol<7>(fmt, W, x, y, N, K, s);
        case 8: return launch_fmt_ncol<8>(fmt, W, x, y, N, K, s);
        default: return QMM_ERR_SHAPE;
    }
}

// routed format fmt, shared format sfmt (fmt, or Q8_0_SOA); fmt may be Q4_K only with a Q8_0_SOA
// shared expert (the all-Q4_K case has its own kernels).
int moe_fmt_dispatch(int fmt, int sfmt, const qmm_moe_segs* a, int nseg, const int* ids, int nexp, qmm_xq8 x, int N, int K,
                     int T, int xrow_te, hipStream_t s) {
#define QMM_MF(F)                                                                                                    \
    case F:                                                                                                          \
        return sfmt == QMM_Q8_0_SOA ? launch_moe_fmt<F, QMM_Q8_0_SOA>(*a, nseg, ids, nexp, x, N, K, T, xrow_te, s) \
                                    : launch_moe_fmt<F, F>(*a, nseg, ids, nexp, x, N, K, T, xrow_te, s);
    if (sfmt != fmt && sfmt != QMM_Q8_0_SOA) return QMM_ERR_FORMAT;
    switch (fmt) {
        case QMM_Q4_K:
            if (sfmt != QMM_Q8_0_SOA) return QMM_ERR_FORMAT;
            return launch_moe_fmt<QMM_Q4_K, QMM_Q8_0_SOA>(*a, nseg, ids, nexp, x, N, K, T, xrow_te, s);
        QMM_MF(QMM_Q5_K)
        QMM_MF(QMM_IQ4_XS)
        QMM_MF(QMM_Q5_1_SOA)
        case QMM_Q8_0_SOA:
            return launch_moe_fmt<QMM_Q8_0_SOA, QMM_Q8_0_SOA>(*a, nseg, ids, nexp, x, N, K, T, xrow_te, s);
        default:
            return QMM_ERR_FORMAT;
    }
#undef QMM_MF
}

}  // namespace qmm
