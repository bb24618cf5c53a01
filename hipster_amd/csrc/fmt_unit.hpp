// fmt_unit.hpp -- per-format "units" of the q8-activation GEMV: the raw weight bytes of one scale's
// worth of weights, their load, the matching activations and the unit's contribution to one
// column, in the reference's arithmetic (block decoders engine/kernels/gemv.hip:58-268; formats
// engine/src/quant.h:22-100).  The unit arithmetic and the lane accumulation are compiled without
// floating-point contraction (explicit fmaf where one is meant), so every kernel built on them
// rounds the same way and their results agree bit for bit.  Shared by the decode GEMV of the other formats (gemv_fmt.hip) and the
// compatibility entry points (compat.hip: split-K GEMV, grouped q8 expert GEMM, Q8_K GEMV).
// Device code only.
#pragma once
#include "qmm_common.hpp"

namespace qmm {

template <int F>
__device__ __forceinline__ size_t fmt_row_bytes(int K) {
    if constexpr (F == QMM_Q4_K) return (size_t)K / 256 * 144;
    else if constexpr (F == QMM_Q5_K) return (size_t)K / 256 * 176;
    else if constexpr (F == QMM_IQ4_XS) return (size_t)K / 256 * 136;
    else if constexpr (F == QMM_Q8_0_SOA) return (size_t)K + (size_t)K / 16;
    else if constexpr (F == QMM_Q6_K_SOA) return (size_t)K / 256 * 210;
    else return (size_t)K / 32 * 24;                        // QMM_Q5_1_SOA
}
// weights per unit: 64 for the formats whose unit is a Q4_K-style qs pair or a Q6_K quarter block,
// else 32 (one sub-block)
template <int F>
__host__ __device__ constexpr int fmt_unit_weights() { return (F == QMM_Q5_K || F == QMM_Q4_K || F == QMM_Q6_K_SOA) ? 64 : 32; }
template <int F>
__host__ __device__ __forceinline__ int fmt_units(int K) { return K / fmt_unit_weights<F>(); }

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

// q8 x of one 32-weight sub-block of one column: its 32 bytes, d and s (s = d * sum(q))
struct X32 { uint4 a, b; float d, s; };

// Sources of one column's activations.  XSrcQ8: the reference's XQ8 (per 32: d, s = d*sum q;
// engine/kernels/gemv.h:8).  XSrcQ8K: the reference's XQ8K (gemv.h:33: one scale per 256,
// d[b*16 + col], int16 sums per 32 bs[(b*16 + col)*8 + j]); its sub-block view has d = the block
// scale and s = d * bs, the same q8 fix-up terms.
struct XSrcQ8 {
    const int8_t* q; const float* d; const float* s;
    __device__ __forceinline__ void sub(int sb, X32& x) const {
        x.a = ld16(q + 32 * (size_t)sb);
        x.b = ld16(q + 32 * (size_t)sb + 16);
        x.d = d[sb];
        x.s = s[sb];
    }
    __device__ __forceinline__ uint4 bytes16(size_t off) const { return ld16(q + off); }
    __device__ __forceinline__ float scale(int sb) const { return d[sb]; }
};
struct XSrcQ8K {
    const int8_t* q; const float* d; const int16_t* bs; int col;
    __device__ __forceinline__ void sub(int sb, X32& x) const {
        x.a = ld16(q + 32 * (size_t)sb);
        x.b = ld16(q + 32 * (size_t)sb + 16);
        const size_t bc = (size_t)(sb >> 3) * 16 + col;
        x.d = d[bc];
        x.s = x.d * (float)bs[bc * 8 + (sb & 7)];
    }
    __device__ __forceinline__ uint4 bytes16(size_t off) const { return ld16(q + off); }
    __device__ __forceinline__ float scale(int sb) const { return d[(size_t)(sb >> 3) * 16 + col]; }
};

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
    template <class XS>
    static __device__ __forceinline__ void xload(const XS& xs, int u, X& x) { xs.sub(u, x); }
    static __device__ __forceinline__ float col(const Raw& r, const X& x, int) {
#pragma clang fp contract(off)
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
    template <class XS>
    static __device__ __forceinline__ void xload(const XS& xs, int u, X& x) { xs.sub(u, x); }
    static __device__ __forceinline__ float col(const Raw& r, const X& x, int) {
#pragma clang fp contract(off)
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
    template <class XS>
    static __device__ __forceinline__ void xload(const XS& xs, int u, X& x) { xs.sub(u, x); }
    static __device__ __forceinline__ float col(const Raw& r, const X& x, int u) {
#pragma clang fp contract(off)
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
    template <class XS>
    static __device__ __forceinline__ void xload(const XS& xs, int u, X& x) {
        xs.sub(2 * u, x.lo);                                   // unit u = 4b + j: sub-blocks 8b + 2j = 2u, 2u + 1
        xs.sub(2 * u + 1, x.hi);
    }
    static __device__ __forceinline__ float col(const Raw& r, const X& x, int u) {
#pragma clang fp contract(off)
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
    template <class XS>
    static __device__ __forceinline__ void xload(const XS& xs, int u, X& x) {
        xs.sub(2 * u, x.lo);
        xs.sub(2 * u + 1, x.hi);
    }
    static __device__ __forceinline__ float col(const Raw& r, const X& x, int u) {
#pragma clang fp contract(off)
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

template <> struct FmtUnit<QMM_Q6_K_SOA> {            // row = [ql K/2][qh K/4][sc K/16 x i8][d K/256 x f16]
    // unit u = quarter block: block b = u/4, half n = (u/2)&1, lh = u&1; its 64 weights are
    // b*256 + 128n + 32g + 16lh + (0..15) for g = 0..3 (quant.h:65-80: ql[l] low/high nibble and
    // ql[l+32] low/high nibble with qh[l] bit pairs 0/2/4/6, scale sc[is + 2g], is = lh)
    struct Raw { uint4 a, b, h; uint32_t sc0, sc1; float d; };
    struct X { uint4 v[4]; float d[4]; };
    static __device__ __forceinline__ void load(const uint8_t* rp, int K, int u, Raw& o) {   // rows 2-byte aligned:
        const int nb = K >> 8, b = u >> 2, n = (u >> 1) & 1, lh = u & 1;                     // dword-aligned loads
        const uint8_t* ql = rp + (size_t)b * 128 + 64 * n + 16 * lh;                         // (K % 512 == 0 keeps
        o.a = ld16_a4(ql);                                                                     //  rows dword aligned)
        o.b = ld16_a4(ql + 32);
        o.h = ld16_a4(rp + (size_t)nb * 128 + (size_t)b * 64 + 32 * n + 16 * lh);
        const u32x2_a4 sc = *(const u32x2_a4*)(rp + (size_t)nb * 192 + (size_t)b * 16 + 8 * n);
        o.sc0 = sc.x; o.sc1 = sc.y;
        o.d = h2f(*(const uint16_t*)(rp + (size_t)nb * 208 + 2 * b));
    }
    template <class XS>
    static __device__ __forceinline__ void xload(const XS& xs, int u, X& x) {
        const int b = u >> 2, n = (u >> 1) & 1, lh = u & 1;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            x.v[g] = xs.bytes16((size_t)b * 256 + 128 * n + 32 * g + 16 * lh);
            x.d[g] = xs.scale(8 * b + 4 * n + g);
        }
    }
    static __device__ __forceinline__ float col(const Raw& q, const X& x, int u) {
#pragma clang fp contract(off)
        const int lh = u & 1;
        const uint32_t A[4] = {q.a.x, q.a.y, q.a.z, q.a.w}, B[4] = {q.b.x, q.b.y, q.b.z, q.b.w}, H[4] = {q.h.x, q.h.y, q.h.z, q.h.w};
        // scales sc[lh + 2g] of the unit's 8-byte run {sc0, sc1}: bytes lh, lh+2, lh+4, lh+6
        const uint32_t scr = __builtin_amdgcn_perm(q.sc1, q.sc0, lh ? 0x07050301u : 0x06040200u);
        float v = 0.f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint32_t w[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = g == 0 ? (A[k] & 0x0f0f0f0fu) : g == 1 ? (B[k] & 0x0f0f0f0fu)
                                  : g == 2 ? ((A[k] >> 4) & 0x0f0f0f0fu) : ((B[k] >> 4) & 0x0f0f0f0fu);
                const uint32_t hi = (g == 0 ? H[k] << 4 : g == 1 ? H[k] << 2 : g == 2 ? H[k] : H[k] >> 2) & 0x30303030u;
                w[k] = q6_signed(lo | hi);
            }
            int is = sdot4(w[0], x.v[g].x, 0);
            is = sdot4(w[1], x.v[g].y, is);
            is = sdot4(w[2], x.v[g].z, is);
            is = sdot4(w[3], x.v[g].w, is);
            const int scg = (int)(int8_t)((scr >> (8 * g)) & 0xffu);
            v = __builtin_fmaf(q.d * x.d[g], (float)(scg * is), v);
        }
        return v;
    }
};

// ---- where a unit's weight bytes are: the loaders of fmt_rows ----
// FmtRowLoad: row `row` at W + row * rb in the format's own layout (every GEMV of the library).
template <int F>
struct FmtRowLoad {
    static __device__ __forceinline__ void load(const uint8_t* W, int row, size_t rb, int K, int u, typename FmtUnit<F>::Raw& r) {
        FmtUnit<F>::load(W + (size_t)row * rb, K, u, r);
    }
};
// FmtIl8Load (Q4_K, Q5_K, IQ4_XS): the 8-row interleaved layout of the reference's layout experiment
// (repack_interleave8, engine/kernels/gemv.hip:1442-1446): rows in groups of 8, a group's blocks
// stored block-major, so block b of row r is block (r / 8) * 8 * nb + 8 b + r % 8 of W.  A block's own
// bytes are unchanged: the format's load of unit u % (units per block) on that one block.
template <int F>
struct FmtIl8Load {
    static __device__ __forceinline__ void load(const uint8_t* W, int row, size_t, int K, int u, typename FmtUnit<F>::Raw& r) {
        static_assert(F == QMM_Q4_K || F == QMM_Q5_K || F == QMM_IQ4_XS, "block formats only");
        constexpr int BB = F == QMM_Q4_K ? 144 : F == QMM_Q5_K ? 176 : 136, UPB = 256 / fmt_unit_weights<F>();
        const int nb = K >> 8;
        const uint8_t* blk = W + ((size_t)(row >> 3) * 8 * nb + (size_t)(u / UPB) * 8 + (row & 7)) * BB;
        FmtUnit<F>::load(blk, 256, u % UPB, r);
    }
};
// FmtIl16Load: the 16-row interleaved layout of the reference's matrix-core GEMV experiment
// (repack_wmma_il, gemv.hip:1277-1303): rows in groups of 16 (the last padded with zero rows); per group
// and 256-weight block, 16 x BB bytes G = W + ((row / 16) * nb + b) * 16 * BB hold the 16 rows' bytes
// piece-major: 16-byte piece i of row r16 at G + 256 i + 16 r16 (IQ4_XS: 8-byte pieces at
// G + 128 i + 8 r16; Q6_K_SOA: ql pieces 0..7, qh pieces at G + 2048, the 16 scale bytes at G + 3072, d at
// G + 3328 + 2 r16; Q8_0_SOA: q pieces 0..15, the 8 sub-block d at G + 4096 + 16 r16).  Piece numbers are
// the byte offsets in the row's own layout / 16.
template <int F>
struct FmtIl16Load {
    static __device__ __forceinline__ size_t group(int row, int K, int b, int BB) {
        return ((size_t)(row >> 4) * (K >> 8) + b) * 16 * BB;
    }
    static __device__ __forceinline__ void load(const uint8_t* W, int row, size_t, int K, int u, typename FmtUnit<F>::Raw& r) {
        const int r16 = row & 15;
        if constexpr (F == QMM_Q4_K) {                 // hd = piece 0, pair j: qs pieces 1 + 2j, 2 + 2j
            const uint8_t* g = W + group(row, K, u >> 2, 144) + 16 * r16;
            const int j = u & 3;
            r.hd = ld16(g);
            r.q0 = ld16(g + 256 * (1 + 2 * j));
            r.q1 = ld16(g + 256 * (2 + 2 * j));
        } else if constexpr (F == QMM_Q5_K) {          // hd, qh halves = pieces 0..2, pair j: 3 + 2j, 4 + 2j
            const uint8_t* g = W + group(row, K, u >> 2, 176) + 16 * r16;
            const int j = u & 3;
            r.hd = ld16(g);
            r.h0 = ld16(g + 256);
            r.h1 = ld16(g + 512);
            r.q0 = ld16(g + 256 * (3 + 2 * j));
            r.q1 = ld16(g + 256 * (4 + 2 * j));
        } else if constexpr (F == QMM_IQ4_XS) {        // 8-byte pieces: header 0, sub-block k: 1 + 2k, 2 + 2k
            const uint8_t* g = W + group(row, K, u >> 3, 136) + 8 * r16;
            const int k = u & 7;
            r.hd = *(const uint2*)g;
            const uint2 lo = *(const uint2*)(g + 128 * (1 + 2 * k)), hi = *(const uint2*)(g + 128 * (2 + 2 * k));
            r.qs = make_uint4(lo.x, lo.y, hi.x, hi.y);
        } else if constexpr (F == QMM_Q6_K_SOA) {      // quarter (n, lh): ql pieces 4n + lh, + 2; qh 2n + lh
            const uint8_t* g = W + group(row, K, u >> 2, 210);
            const int n = (u >> 1) & 1, lh = u & 1;
            r.a = ld16(g + 256 * (4 * n + lh) + 16 * r16);
            r.b = ld16(g + 256 * (4 * n + lh + 2) + 16 * r16);
            r.h = ld16(g + 2048 + 256 * (2 * n + lh) + 16 * r16);
            const uint2 sc = *(const uint2*)(g + 3072 + 16 * r16 + 8 * n);
            r.sc0 = sc.x;
            r.sc1 = sc.y;
            r.d = h2f(*(const uint16_t*)(g + 3328 + 2 * r16));
        } else {                                       // Q8_0_SOA, sub-block s: q pieces 2s, 2s + 1
            static_assert(F == QMM_Q8_0_SOA, "no 16-row interleaved layout for this format");
            const uint8_t* g = W + group(row, K, u >> 3, 272);
            const int sb = u & 7;
            r.a = ld16(g + 256 * (2 * sb) + 16 * r16);
            r.b = ld16(g + 256 * (2 * sb + 1) + 16 * r16);
            r.d = *(const uint16_t*)(g + 4096 + 16 * r16 + 2 * sb);
        }
    }
};

// Lane-partial sums of RPW rows (row0..row0+RPW-1, clamped to N) x NCOL columns over units
// [ub, ue): lane l takes units ub + l, ub + l + 64, ..., NIT at a time, every load of a pass issued
// before its arithmetic.  xs[c] is column c's activation source; acc[r][c] is the lane's partial
// (the caller reduces over the wave).  Rows of format F start rb bytes apart (0 = the format's own
// row size for K) unless the loader LD places them otherwise.  pre() runs once, after the first pass's
// weight loads are issued and before its x is read (a caller that stages x in LDS finishes the staging
// there, so its weights are already in flight); FmtNoPre does nothing.
struct FmtNoPre {
    static constexpr bool active = false;
    __device__ __forceinline__ void operator()() const {}
};
template <int F, int NCOL, int NIT, int RPW, class XS, class Pre = FmtNoPre, class LD = FmtRowLoad<F>>
__device__ __forceinline__ void fmt_rows(const uint8_t* __restrict__ W, int row0, int N, int K, const XS (&xs)[NCOL],
                                         float (&acc)[RPW][NCOL], int ub, int ue, size_t rb = 0, const Pre& pre = Pre()) {
#pragma clang fp contract(off)
    typedef FmtUnit<F> FU;
    const int lane = threadIdx.x & 63;
    if (rb == 0) rb = fmt_row_bytes<F>(K);
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int c = 0; c < NCOL; ++c) acc[r][c] = 0.f;
    for (int base = ub; base < ue; base += 64 * NIT) {
        typename FU::Raw R[RPW][NIT];
        typename FU::X X[NIT];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int i = 0; i < NIT; ++i) LD::load(W, min(row0 + r, N - 1), rb, K, min(base + lane + 64 * i, ue - 1), R[r][i]);
        if constexpr (Pre::active) {
            if (base == ub) {
                __builtin_amdgcn_sched_barrier(0);
                pre();
            }
        }
#pragma unroll
        for (int c = 0; c < NCOL; ++c) {
#pragma unroll
            for (int i = 0; i < NIT; ++i) FU::xload(xs[c], min(base + lane + 64 * i, ue - 1), X[i]);
            // all loads issued before any arithmetic (the scheduler would otherwise sink each load
            // to its use to save registers, one memory latency after another)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < NIT; ++i) {
                const int u = base + lane + 64 * i;
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const float v = FU::col(R[r][i], X[i], min(u, ue - 1));
                    acc[r][c] += u < ue ? v : 0.f;
                }
            }
        }
    }
}

}  // namespace qmm
