// gemv_mfma.hip -- Q4_K decode GEMV for 2..16 columns on the int8 matrix cores of gfx950.
//
// Replaces, for Q4_K weights, the per-column dot4 work of the reference's gemv_q8 / gemv_multi /
// gemv_wmma (engine/kernels/gemv.hip:602-682 is the reference's int8 WMMA form for gfx1151).
//
// v_mfma_i32_16x16x32_i8 multiplies A [16 x 32] by B [32 x 16]: lane l supplies A row l%16 and B
// column l%16, k = 8(l/16)..8(l/16)+7 of each, and gets D[i][l%16] for i = 4(l/16)..+3.  Here A holds
// x (rows = token slots) and B one 32-weight sub-block of 16 weight rows: a Q4_K pair j (qs bytes
// 32j..32j+31 of a block) is two instructions, its low nibbles against sub-block 2j of x and its high
// nibbles against sub-block 2j+1, on the same 8 bytes of row l%16 in lane l.  The int32 results are the
// exact sub-block dots ia, ib of the dot4 kernels.
//
// Bitwise the dot4 kernels (q4k_pair.hpp): there, lane t of a row's 16 lanes adds the values of pair
// tasks t, t+16, t+32, ... (task = 4 * block + j) in that order, and the 16 partial sums meet in the
// xor butterfly 8, 4, 2, 1.  Here wave w of a workgroup takes blocks w, w+4, w+8, ... of one 16-row
// tile, which are exactly the tasks of partial sums t = 4w + j, in the same order; each value is
// q4k_pair_value of the same scales, x pair scales and integer dots; the 16 partial sums are then
// combined in LDS in the butterfly's association order.  So every column is the same float as the
// one-column kernels give, whatever the number of columns (T-invariant with them).
//
// Token slots: with MV = 1, 2 or 4 slots per lane group (ncol <= 4, 8, 16), token c sits in A row
// 4(c / MV) + c % MV, so lane l's D values v < MV are tokens MV(l/16) + v: the float epilogue costs
// MV evaluations per pair per lane whatever the slot rows left empty.
#include "q4k_pair.hpp"
#include "qmm_common.hpp"

#include <hip/hip_runtime.h>

namespace qmm {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kMfmaMaxSeg = 4;
constexpr int kScaleRegs = 4;      // x pair-scale quadruples each thread loads ahead of the weights

struct MSegs {
    const uint8_t* w[kMfmaMaxSeg];
    float* y[kMfmaMaxSeg];
    int N[kMfmaMaxSeg];
    int t0[kMfmaMaxSeg + 1];       // first 16-row tile of each segment; t0[nseg] = all tiles
    int nseg;
};

__device__ __forceinline__ uint2 ld8(const void* p) { return *(const uint2*)p; }
__device__ __forceinline__ long as_long(uint2 v) { return (long)(((unsigned long)v.y << 32) | v.x); }

// One block (256 weights) of the lane's row: its header and 16 qs bytes of each pair couple (pairs
// 2c, 2c+1 = qs bytes 64c..64c+63): lane group h reads bytes 64c + 16h..+15, whole 16-byte pieces.
// A permlane32 swap of their second halves (groups 0, 1) with the first halves of groups 2, 3 leaves
// every lane 8 bytes of pair 2c and 8 of pair 2c+1, at k offsets 8 kperm(h) within the pair,
// kperm = {0, 2, 1, 3}; the A operand (x) is read at the same k offsets, so each MFMA sums the same
// products as with k in order.
struct MBlk {
    uint4 hd;
    uint4 q[2];
    uint4 x[4];        // x of the lane's token slot, bytes 64j + 16h..+15 of the block (pair j)
};

__device__ __forceinline__ int kperm(int h) { return ((h & 1) << 1) | (h >> 1); }

typedef unsigned u32x4v __attribute__((ext_vector_type(4)));

// x through a buffer resource over the call's x: lanes of empty token slots use an offset past its
// end, which reads zeros without touching memory
__device__ __forceinline__ uint4 xload(__amdgpu_buffer_rsrc_t rx, uint32_t off) {
    const u32x4v v = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// XL: x comes from LDS at compute time (only the weights are loaded here)
template <bool XL>
__device__ __forceinline__ void mblk_load(MBlk& B, const uint8_t* rp, __amdgpu_buffer_rsrc_t rx, uint32_t xo, int b, int h) {
    const uint8_t* bp = rp + (size_t)b * 144;
    B.hd = ld16(bp);
    B.q[0] = ld16(bp + 16 + 16 * h);
    B.q[1] = ld16(bp + 80 + 16 * h);
    if constexpr (!XL) {
#pragma unroll
        for (int j = 0; j < 4; ++j) B.x[j] = xload(rx, xo + (uint32_t)(b * 256 + 64 * j));
    }
}

// {lane's 8 bytes of pair 2c, lane's 8 bytes of pair 2c+1} from the couple's 16-byte piece
__device__ __forceinline__ void couple_split(const uint4 v, uint2& p0, uint2& p1) {
    const auto sx = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
    const auto sy = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
    p0 = make_uint2(sx[0], sy[0]);
    p1 = make_uint2(sx[1], sy[1]);
}

// adds block b's pair values to acc; a block past the row's end (live = false, b clamped by the
// caller) adds +0, which leaves every partial sum unchanged (a sum started at +0 is never -0)
// The x piece of pair j (sub-block 2j = bytes 0..31, 2j+1 = bytes 32..63) splits the same way as a
// weight couple: after the swap the lane holds 8 bytes of each sub-block at k offsets 8 kperm(h).
// Every lane decodes the scales of the four pairs of its row's block itself: an exchange of one
// quadruple per lane through LDS costs less VALU but puts an LDS round trip into every block's chain
// (measured: 18.6 against 17.8 us at 4 columns, 17408 x 5120).
// XL: the x piece of pair j is the 16 bytes at xl + 64 j (LDS)
template <int MV, bool XL>
__device__ __forceinline__ void mblk_compute(const MBlk& B, int b, int h, bool live, const float4* __restrict__ sds,
                                             const uint8_t* xl, float (&acc)[4][MV]) {
    constexpr int NS = 4 * MV;
    uint2 q[4];
    couple_split(B.q[0], q[0], q[1]);
    couple_split(B.q[1], q[2], q[3]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint2 lo = make_uint2(q[j].x & 0x0f0f0f0fu, q[j].y & 0x0f0f0f0fu);
        const uint2 hi = make_uint2((q[j].x >> 4) & 0x0f0f0f0fu, (q[j].y >> 4) & 0x0f0f0f0fu);
        uint2 x0, x1;
        if constexpr (XL) couple_split(*(const uint4*)(xl + 64 * j), x0, x1);
        else couple_split(B.x[j], x0, x1);
        const i32x4 z = {0, 0, 0, 0};
        const i32x4 ca = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(x0), as_long(lo), z, 0, 0, 0);
        const i32x4 cb = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(x1), as_long(hi), z, 0, 0, 0);
        const Q4kPairScales sc = q4k_pair_scales(B.hd, Q4kPairDecode(j));
        const float4* dsp = sds + (size_t)(4 * b + j) * NS + h * MV;
#pragma unroll
        for (int v = 0; v < MV; ++v) acc[j][v] += live ? q4k_pair_value(sc, dsp[v], ca[v], cb[v]) : 0.f;
    }
}

constexpr int kMfmaMaxK = 32768;

// LDS of the x pair scales [K/64][4 MV] float4, reused for the partial sums [16][4 MV][16] float
__host__ __device__ inline size_t gemv_q4k_mfma_main_lds(int K, int mv) {
    const size_t scales = (size_t)(K / 64) * (4 * mv) * 16, parts = (size_t)16 * (4 * mv) * 16 * 4;
    return scales > parts ? scales : parts;
}
// x staged in LDS (XL) for ncol <= 8 and ncol * K <= xl_max(MV): token c at c * (K + 64) (the 64-byte skew
// spreads the tokens over the banks), then 256 bytes of zeros read by the empty token slots; staged
// by xl_regs(MV) 16-byte pieces per thread, loaded before the first weights: 8 up to 4 columns, 10 (all
// of 8 columns at K = 5120) for 5..8 (10 at 4 columns measured 0.8 us slower at 17408 x 5120: 106
// against 94 VGPRs; x in LDS at 5..8 columns: 20.8-21.4 -> 20.1-20.4 us, config-1 layer at M = 8
// 100.7 -> 99.4 us)
__host__ __device__ constexpr int xl_regs(int mv) { return mv == 1 ? 8 : 10; }
__host__ __device__ constexpr int xl_max(int mv) { return 256 * 16 * xl_regs(mv); }
__host__ __device__ inline size_t gemv_q4k_mfma_xl_bytes(int K, int ncol) { return (size_t)ncol * (K + 64) + 256; }

// grid = all 16-row tiles of all segments, 256 threads; LDS: x pair scales [K/64][4 MV] float4, after
// the main loop reused for the partial sums [16][4 MV][16] float; with XL the staged x.  XL takes the x loads out of the main loop (fewer load instructions, 32 fewer VGPRs).
template <int MV, bool XL>
__global__ void __launch_bounds__(256) k_gemv_q4k_mfma(MSegs sg, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                       const float* __restrict__ xs, int K, int ncol) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NS = 4 * MV;
    const int tile = blockIdx.x;
    int si = 0;
#pragma unroll
    for (int i = 1; i < kMfmaMaxSeg; ++i)
        if (i < sg.nseg && tile >= sg.t0[i]) si = i;
    const int N = sg.N[si], row0 = (tile - sg.t0[si]) * 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane & 15, h = lane >> 4;
    const int nb = K >> 8, nsb = K >> 5, npair = K >> 6;
    const uint8_t* rp = sg.w[si] + (size_t)min(row0 + r, N - 1) * ((size_t)nb * 144);
    float4* sds = (float4*)smem;
    float* part = (float*)smem;
    // A operand source of this lane: x of the token in slot r (zeros for an empty slot), 16-byte
    // piece h of each pair
    const int ca = (r >> 2) * MV + (r & 3);
    const bool aval = (r & 3) < MV && ca < ncol;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)xq, (short)0, ncol * K, 0x00020000);
    const uint32_t xo = aval ? (uint32_t)(ca * K + 16 * h) : 0x40000000u;
    // XL: the lane's x in LDS for block b at xlb + b * xls (the zero area for an empty slot)
    uint8_t* const xlds = smem + gemv_q4k_mfma_main_lds(K, MV);
    const int kp = K + 64;
    const uint8_t* const xlb = aval ? xlds + ca * kp + 16 * h : xlds + ncol * kp + 16 * h;
    const int xls = aval ? 256 : 0;

    // x pair scales {d[2p], d[2p+1], s[2p], s[2p+1]} of every (pair, token): item e = c * npair + p,
    // thread tid taking items tid + 256 u, loaded (unconditionally, clamped) before the first weights
    // so that their LDS stores wait for them only (loads retire in issue order).  c = e / npair by a
    // float reciprocal, exact for these small integers.
    const int nitem = npair * ncol;
    const float inv_np = 1.f / (float)npair;
    float4 sv[kScaleRegs];
#pragma unroll
    for (int u = 0; u < kScaleRegs; ++u) {
        const int e = min(tid + 256 * u, nitem - 1), c = (int)(((float)e + 0.5f) * inv_np), pp = e - c * npair;
        const float2 dd = *(const float2*)(xd + (size_t)c * nsb + 2 * pp), ss = *(const float2*)(xs + (size_t)c * nsb + 2 * pp);
        sv[u] = make_float4(dd.x, dd.y, ss.x, ss.y);
    }
    // XL: the x of every column, 16-byte piece e = c * (K / 16) + o (token c by a float reciprocal,
    // exact for these small integers), loaded (clamped) ahead of the weights as well
    const int nxq = XL ? ncol * (K >> 4) : 1;
    const float inv_kq = 1.f / (float)(K >> 4);
    constexpr int XR = XL ? xl_regs(MV) : 1;
    uint4 xv[XR];
    if constexpr (XL) {
#pragma unroll
        for (int u = 0; u < XR; ++u) xv[u] = ld16(xq + (size_t)min(tid + 256 * u, nxq - 1) * 16);
    }
    // every load below is unconditional (block indices clamped to the last block): with the same
    // loads on every path the wait counts stay exact and each prefetch stays in flight
    MBlk A, B;
    mblk_load<XL>(A, rp, rx, xo, min(wave, nb - 1), h);
#pragma unroll
    for (int u = 0; u < kScaleRegs; ++u) {
        const int e = tid + 256 * u, c = (int)(((float)e + 0.5f) * inv_np), pp = e - c * npair;
        if (e < nitem) sds[pp * NS + c] = sv[u];
    }
    for (int e = tid + 256 * kScaleRegs; e < nitem; e += 256) {     // K * ncol > 128 K: the rest in a loop
        const int c = (int)(((float)e + 0.5f) * inv_np), pp = e - c * npair;
        const float2 dd = *(const float2*)(xd + (size_t)c * nsb + 2 * pp), ss = *(const float2*)(xs + (size_t)c * nsb + 2 * pp);
        sds[pp * NS + c] = make_float4(dd.x, dd.y, ss.x, ss.y);
    }
    if constexpr (XL) {
#pragma unroll
        for (int u = 0; u < XR; ++u) {                    // no branch: a clamped piece stores its own value
            const int e = min(tid + 256 * u, nxq - 1), c = (int)(((float)e + 0.5f) * inv_kq), o = e - c * (K >> 4);
            *(uint4*)(xlds + c * kp + 16 * o) = xv[u];
        }
        if (tid < 16) *(uint4*)(xlds + ncol * kp + 16 * tid) = make_uint4(0, 0, 0, 0);
    }
    lds_barrier();

    float acc[4][MV];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < MV; ++v) acc[j][v] = 0.f;
    // two register sets in turn; no branch around a load or a compute (the compiler would sink the
    // prefetch into it), and scheduling barriers keep each prefetch ahead of the compute it overlaps
    for (int b = wave; b < nb; b += 8) {                  // wave-uniform
        mblk_load<XL>(B, rp, rx, xo, min(b + 4, nb - 1), h);
        __builtin_amdgcn_sched_barrier(0);
        mblk_compute<MV, XL>(A, b, h, true, sds, xlb + b * xls, acc);
        mblk_load<XL>(A, rp, rx, xo, min(b + 8, nb - 1), h);
        __builtin_amdgcn_sched_barrier(0);
        mblk_compute<MV, XL>(B, min(b + 4, nb - 1), h, b + 4 < nb, sds, xlb + min(b + 4, nb - 1) * xls, acc);
    }
    __syncthreads();                                      // every wave is done with the scales
    // partial sum t = 4 wave + j of token MV h + v, row r
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < MV; ++v) part[((4 * wave + j) * NS + h * MV + v) * 16 + r] = acc[j][v];
    __syncthreads();
    const int orow = tid & 15, oc = tid >> 4;
    if (oc < ncol && row0 + orow < N) {
        float a[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) a[t] = part[(t * NS + oc) * 16 + orow];
        // the association order of the xor butterfly 8, 4, 2, 1 (group_sum over 16 lanes)
        float q[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) q[t] = a[t] + a[t + 8];
#pragma unroll
        for (int t = 0; t < 4; ++t) q[t] = q[t] + q[t + 4];
        q[0] = q[0] + q[2];
        q[1] = q[1] + q[3];
        sg.y[si][(size_t)oc * N + row0 + orow] = q[0] + q[1];
    }
}


// ------------------------------------------------------------------------------------------
// Q6_K_SOA GEMV for 2..8 columns on the int8 matrix cores, bitwise the unit kernel of gemv.hip
// (k_gemv_q6k_u / k_gemv_q6k_w: lane l of a row's wave adds the values of quarter-block units l,
// l+64, ... in that order, each value the fma chain over the unit's four 16-weight groups g of
// (d * xd[g]) * (float)(sc[g] * isum_g), and the 64 partial sums meet in the xor butterfly 32, 16,
// 8, 4, 2, 1).  Unit u = 4b + 2n + lh holds weights 256b + 128n + 16lh + l' + 32g, l' < 16: group g
// is the low (g < 2) or high nibble of ql run A (g even, ql[64n + l]) or run B (g odd, ql[64n + 32 +
// l]) with bits 2g, 2g+1 of qh[32n + l], l = 16lh + l' (quant.h:65-80).
//
// v_mfma_i32_16x16x64_i8, one instruction per group g and 4 tokens: lane (j, q) = (l % 16, l / 16)
// supplies 16 bytes of A row j and of B column j, the same 16 k for both.  B column j is weight row j
// of the 16-row tile and lane group q supplies group g of unit q of the block, so every lane loads
// bytes of its own (ql runs A and B and qh of its unit: three 16-byte loads per block, none
// repeated).  A row 4t + s is token t against unit s alone (its x of group g in the lanes of group
// q = s, zeros elsewhere), so D[4t + s][j] is the exact integer isum of unit s, group g, and lane
// (j, q) receives D[4q + v][j], v = 0..3: token q (q + 4 in the second token block), units 0..3.
// A workgroup is 16 rows x kQ6MWaves waves (W); wave w takes blocks b = w + Wm, whose units 4b + v belong
// to the unit kernel's lanes 4w + v + 4Wk, k = m % (16 / W), in the same order: acc[k][v] is lane
// (4w + v + 4Wk)'s partial sum.  The 64 partials of each (row, token) meet in LDS in the butterfly's
// association order.  The tile's block scales and d are staged in LDS with the x scales before the
// main loop, which loads only the lanes' weight bytes and x (5120 x 17408 at 4 columns: 34.2 -> 28.1 us).
struct Q6MBlk {
    uint4 a, b, h;      // the lane's unit: 16 bytes of ql run A, of run B and of qh
};

template <int NT>
__device__ __forceinline__ void q6m_load(Q6MBlk& B, uint4 (&X)[NT][4], const uint8_t* qlp, const uint8_t* qhp,
                                         __amdgpu_buffer_rsrc_t rx, const uint32_t (&xo)[NT], int b) {
    B.a = ld16_a4(qlp + b * 128);
    B.b = ld16_a4(qlp + b * 128 + 32);
    B.h = ld16_a4(qhp + b * 64);
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) X[i][g] = xload(rx, xo[i] + (uint32_t)(b * 256 + 32 * g));
}

// the block's unit values for the lane's tokens q + 4i added to acc[v][i] (live = false adds +0)
template <int NT>
__device__ __forceinline__ void q6m_compute(const Q6MBlk& B, const uint4 (&X)[NT][4], int b, int q, const uint8_t* scl, const uint16_t* dl,
                                            const float* sxd, int nsb,
                                            int ncol, bool live, float (&acc)[4][NT]) {
    const uint32_t aw[4] = {B.a.x, B.a.y, B.a.z, B.a.w}, bw[4] = {B.b.x, B.b.y, B.b.z, B.b.w};
    const uint32_t hw[4] = {B.h.x, B.h.y, B.h.z, B.h.w};
    i32x4 bop[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        bop[0][w] = (int)q6_signed((aw[w] & 0x0f0f0f0fu) | ((hw[w] << 4) & 0x30303030u));
        bop[1][w] = (int)q6_signed((bw[w] & 0x0f0f0f0fu) | ((hw[w] << 2) & 0x30303030u));
        bop[2][w] = (int)q6_signed(((aw[w] >> 4) & 0x0f0f0f0fu) | (hw[w] & 0x30303030u));
        bop[3][w] = (int)q6_signed(((bw[w] >> 4) & 0x0f0f0f0fu) | ((hw[w] >> 2) & 0x30303030u));
    }
    const float d = h2f(dl[b]);                           // the row's staged d and scales of block b
    const uint4 sc = *(const uint4*)(scl + 16 * b);
    const uint32_t scw[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        i32x4 c[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const i32x4 a = {(int)X[i][g].x, (int)X[i][g].y, (int)X[i][g].z, (int)X[i][g].w};
            const i32x4 z = {0, 0, 0, 0};
            c[g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bop[g], z, 0, 0, 0);
        }
        const float* xs = sxd + (size_t)min(q + 4 * i, ncol - 1) * nsb + 8 * b;
        const float4 x0 = *(const float4*)xs, x1 = *(const float4*)(xs + 4);
        const float xsn[2][4] = {{x0.x, x0.y, x0.z, x0.w}, {x1.x, x1.y, x1.z, x1.w}};
#pragma unroll
        for (int v = 0; v < 4; ++v) {              // unit v = (n, lh) = (v >> 1, v & 1)
            const int n = v >> 1, lh = v & 1;
            float val = 0.f;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int si = 8 * n + lh + 2 * g;  // scale byte of the unit's group g
                const int scg = (int)(int8_t)((scw[si >> 2] >> (8 * (si & 3))) & 0xffu);
                val = __builtin_fmaf(d * xsn[n][g], (float)(scg * c[g][v]), val);
            }
            acc[v][i] += live ? val : 0.f;
        }
    }
}

constexpr int kQ6MWaves = 4;
constexpr int kQ6MParts = 16 / kQ6MWaves;   // partial sums per lane and unit position
constexpr int kQ6MUnroll = kQ6MParts < 2 ? 2 : kQ6MParts;   // blocks per loop pass: the 2-block ring and acc[m % kQ6MParts]
constexpr int kQ6MScaleRegs = 8;      // x-scale float4 per thread loaded ahead of the weights
constexpr int kQ6MScRegs = 5;         // 16-byte pieces of the tile's block scales per thread, staged ahead of the weights
constexpr int kQ6MDRegs = 3;          // dwords of the tile's block d per thread, staged ahead of the weights

// LDS: x scales [ncol][K/32] float, the tile's block scales [16][K/16 + 16] bytes and d [16][K/256 + 2]
// f16; after the main loop the partials [64][4 NT][16] float from offset 0
__host__ __device__ inline size_t gemv_q6k_mfma_sc_row(int K) { return (size_t)K / 16 + 16; }
__host__ __device__ inline size_t gemv_q6k_mfma_d_row(int K) { return (size_t)K / 256 + 2; }   // f16 elements
__host__ __device__ inline size_t gemv_q6k_mfma_lds(int K, int ncol) {
    const size_t st = (size_t)ncol * (K / 32) * 4 + 16 * gemv_q6k_mfma_sc_row(K) + 16 * gemv_q6k_mfma_d_row(K) * 2;
    const size_t parts = (size_t)64 * (ncol <= 4 ? 4 : 8) * 16 * 4;
    return st > parts ? st : parts;
}

template <int NT>
__global__ void __launch_bounds__(64 * kQ6MWaves) k_gemv_q6k_mfma(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                                 const float* __restrict__ xd, float* __restrict__ y, int N, int K,
                                                                 int ncol) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NS = 4 * NT;
    const int nb = K >> 8, nsb = K >> 5;
    const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: a scalar block loop
    const int row0 = blockIdx.x * 16;
    const uint8_t* rp = W + (size_t)min(row0 + j, N - 1) * ((size_t)nb * 210);
    const int un = q >> 1, ulh = q & 1;                      // the lane's unit (n, lh) = q of each block
    const uint8_t* qlp = rp + 64 * un + 16 * ulh;
    const uint8_t* qhp = rp + (size_t)nb * 128 + 32 * un + 16 * ulh;
    // A source: token 4i + (j >> 2) against unit s = j & 3 of the block, from the lanes of group q = s
    // only (an offset past the end of x reads zeros)
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)xq, (short)0, ncol * K, 0x00020000);
    uint32_t xo[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int t = 4 * i + (j >> 2), sv = j & 3;
        xo[i] = (sv == q && t < ncol) ? (uint32_t)(t * K + 128 * (sv >> 1) + 16 * (sv & 1)) : 0x40000000u;
    }
    // x scales of every column to LDS, kQ6MScaleRegs float4 per thread (the launcher checks that they
    // cover them), loaded before the weights: loads retire in issue order, so their LDS stores wait
    // for them only
    float* sxd = (float*)smem;
    const int nx4 = ncol * (nsb >> 2);
    float4 sv[kQ6MScaleRegs];
#pragma unroll
    for (int r = 0; r < kQ6MScaleRegs; ++r) sv[r] = ((const float4*)xd)[min(tid + 64 * kQ6MWaves * r, nx4 - 1)];
    // the tile's block scales (nb 16-byte pieces per row) and d (nb / 2 dwords per row), staged the same
    // way, so the main loop loads weights and x only
    uint8_t* const scl = (uint8_t*)(sxd + (size_t)ncol * nsb);
    uint16_t* const dlds = (uint16_t*)(scl + 16 * gemv_q6k_mfma_sc_row(K));
    const int scrs = (int)gemv_q6k_mfma_sc_row(K), drs = (int)gemv_q6k_mfma_d_row(K);
    const size_t rbytes = (size_t)nb * 210;
    const int nsc = 16 * nb, ndw = 16 * (nb >> 1);
    const float rnb = __builtin_amdgcn_rcpf((float)nb), rnh = __builtin_amdgcn_rcpf((float)(nb >> 1));
    uint4 scv[kQ6MScRegs];
    uint32_t dv[kQ6MDRegs];
#pragma unroll
    for (int r = 0; r < kQ6MScRegs; ++r) {                 // piece e: row e / nb, block e % nb
        const int e = min(tid + 64 * kQ6MWaves * r, nsc - 1), rr = div_small(e, nb, rnb);
        scv[r] = ld16_a4(W + (size_t)min(row0 + rr, N - 1) * rbytes + (size_t)nb * 192 + (size_t)(e - rr * nb) * 16);
    }
#pragma unroll
    for (int r = 0; r < kQ6MDRegs; ++r) {                  // dword e: row e / (nb/2), blocks 2 (e % (nb/2)) + 0, 1
        const int e = min(tid + 64 * kQ6MWaves * r, ndw - 1), rr = div_small(e, nb >> 1, rnh);
        dv[r] = *(const uint32_t*)(W + (size_t)min(row0 + rr, N - 1) * rbytes + (size_t)nb * 208 + (size_t)(e - rr * (nb >> 1)) * 4);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int nm = (nb - wave + kQ6MWaves - 1) / kQ6MWaves;  // blocks b = wave + W m of this wave (may be 0)
    auto blk = [&](int m) { return min(wave + kQ6MWaves * min(m, max(nm - 1, 0)), nb - 1); };
    // two blocks in flight (weights three blocks ahead measured no faster); every load unconditional
    // (clamped block), so the wait counts stay exact
    Q6MBlk R[2];
    uint4 X[2][NT][4];
    q6m_load<NT>(R[0], X[0], qlp, qhp, rx, xo, blk(0));
    q6m_load<NT>(R[1], X[1], qlp, qhp, rx, xo, blk(1));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < kQ6MScaleRegs; ++r)                 // no branch: a clamped item stores its own value
        ((float4*)sxd)[min(tid + 64 * kQ6MWaves * r, nx4 - 1)] = sv[r];
#pragma unroll
    for (int r = 0; r < kQ6MScRegs; ++r) {
        const int e = min(tid + 64 * kQ6MWaves * r, nsc - 1), rr = div_small(e, nb, rnb);
        *(uint4*)(scl + rr * scrs + 16 * (e - rr * nb)) = scv[r];
    }
#pragma unroll
    for (int r = 0; r < kQ6MDRegs; ++r) {
        const int e = min(tid + 64 * kQ6MWaves * r, ndw - 1), rr = div_small(e, nb >> 1, rnh);
        *(uint32_t*)(dlds + rr * drs + 2 * (e - rr * (nb >> 1))) = dv[r];
    }
    lds_barrier();
    const uint8_t* const scr = scl + j * scrs;            // the lane's row
    const uint16_t* const dr = dlds + j * drs;
    float acc[kQ6MParts][4][NT];
#pragma unroll
    for (int k = 0; k < kQ6MParts; ++k)
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int i = 0; i < NT; ++i) acc[k][v][i] = 0.f;
    // at least one pass: a loop that might not run would let the compiler sink the ring's loads past
    // the barrier into its entry
    int m0 = 0;
    do {                                                     // wave-uniform
#pragma unroll
        for (int k = 0; k < kQ6MUnroll; ++k) {
            const int m = m0 + k;
            q6m_compute<NT>(R[k & 1], X[k & 1], blk(m), q, scr, dr, sxd, nsb, ncol, m < nm, acc[k % kQ6MParts]);
            // the refill stays right here: the scheduler would otherwise move the ring's loads next to
            // their uses and drain the queue
            __builtin_amdgcn_sched_barrier(0);
            q6m_load<NT>(R[k & 1], X[k & 1], qlp, qhp, rx, xo, blk(m + 2));
            __builtin_amdgcn_sched_barrier(0);
        }
        m0 += kQ6MUnroll;
    } while (m0 < nm);
    lds_barrier();                                           // every wave is done with the x scales
    float* part = (float*)smem;                              // [slot l][token][row]
#pragma unroll
    for (int k = 0; k < kQ6MParts; ++k)
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int i = 0; i < NT; ++i) part[((4 * wave + v + 4 * kQ6MWaves * k) * NS + 4 * i + q) * 16 + j] = acc[k][v][i];
    lds_barrier();
    for (int e = tid; e < 16 * ncol; e += 64 * kQ6MWaves) {
        const int orow = e & 15, oc = e >> 4;
        if (row0 + orow >= N) continue;
        // the association order of the butterfly over the 64 lanes of the unit kernel's row wave
        float a[32];
#pragma unroll
        for (int t = 0; t < 32; ++t) a[t] = part[(t * NS + oc) * 16 + orow] + part[((t + 32) * NS + oc) * 16 + orow];
#pragma unroll
        for (int t = 0; t < 16; ++t) a[t] = a[t] + a[t + 16];
#pragma unroll
        for (int t = 0; t < 8; ++t) a[t] = a[t] + a[t + 8];
#pragma unroll
        for (int t = 0; t < 4; ++t) a[t] = a[t] + a[t + 4];
        a[0] = a[0] + a[2];
        a[1] = a[1] + a[3];
        y[(size_t)oc * N + row0 + orow] = a[0] + a[1];
    }
}

// ------------------------------------------------------------------------------------------
// Q8_0_SOA GEMV for 1..8 columns on the int8 matrix cores (the dispatch uses it from 4 columns on),
// bitwise the unit kernel of gemv_fmt.hip
// (k_gemv_fmt with FmtUnit<QMM_Q8_0_SOA>: lane l of a row's wave adds (d * xd) * isum of the 32-weight
// sub-blocks l, l + 64, ... in that order, and the 64 partial sums meet in the xor butterfly 32, 16, 8,
// 4, 2, 1).  Row = [qs K][d K/32 x f16] (the engine's load-time SoA repack of Q8_0).
//
// v_mfma_i32_16x16x64_i8 over one 64-byte chunk c (sub-blocks 2c, 2c + 1) of 16 weight rows and up to
// 8 tokens: lane (j, q) = (l % 16, l / 16) supplies as B column j the chunk bytes 16q..16q+15 of
// weight row j (half q & 1 of sub-block q >> 1), and as A row j -- token j >> 1 against sub-block j & 1
// alone -- that token's x bytes at the same chunk offset when q >> 1 == j & 1, zeros elsewhere (16 zero
// bytes in LDS).  So D[2t + s][j] is the exact isum of sub-block 2c + s of row j with token
// t, and lane (j, q) receives D[4q + v][j]: token 2q + (v >> 1), sub-block 2c + (v & 1).  Wave w of
// kQ8MWaves (4) takes chunks c = w + 4i; sub-block 2c + s belongs to the unit kernel's lane
// (2c + s) % 64 = 2w + s + 8 (i % 8), so acc[i % 8][v] is that lane's partial sum, its sub-blocks
// added in the same order.  The 64 partials of each (row, token) meet in LDS in the butterfly's order.
// x, the tile's d and the x scales are staged in LDS before the main loop, whose only loads are the
// weights (reading x and d from global memory per chunk measured 32-37 against 25 us at 17408 x 5120).
constexpr int kQ8MWaves = 4;
constexpr int kQ8MRing = 8;          // weight pieces in flight per lane
constexpr int kQ8MScaleRegs = 8;     // x-scale pairs per thread, staged ahead of the weights
constexpr int kQ8MXRegs = 10;        // 16-byte x pieces per thread, staged ahead of the weights
constexpr int kQ8MDRegs = 8;         // dwords of the tile's d per thread, staged ahead of the weights

// LDS: x [ncol][K + 64] bytes (the skew spreads the tokens over the banks) and 16 zero bytes (the A
// pieces of the lanes that hold no x), the tile's d [16][K/16 + 4] bytes, the x scales [ncol][K/32]
// float; after the main loop the partials [64][8][16] float from offset 0
__host__ __device__ inline size_t gemv_q80_mfma_x_bytes(int K, int ncol) { return (size_t)ncol * (K + 64) + 16; }
__host__ __device__ inline size_t gemv_q80_mfma_d_bytes(int K) { return (size_t)16 * (K / 16 + 4); }
__host__ __device__ inline size_t gemv_q80_mfma_lds(int K, int ncol) {
    const size_t st = gemv_q80_mfma_x_bytes(K, ncol) + gemv_q80_mfma_d_bytes(K) + (size_t)ncol * (K / 32) * 4;
    const size_t parts = (size_t)64 * 8 * 16 * 4;
    return st > parts ? st : parts;
}

__device__ __forceinline__ void q8m_compute(uint4 w, const uint8_t* xa, int xs, int c, int q, const uint8_t* da, const float* sxd, int nsb,
                                            int ncol, bool live, float (&acc)[4]) {
#pragma clang fp contract(off)
    const uint4 xv = *(const uint4*)(xa + xs * c);
    const uint32_t dd = *(const uint32_t*)(da + 4 * c);
    const i32x4 a = {(int)xv.x, (int)xv.y, (int)xv.z, (int)xv.w}, b = {(int)w.x, (int)w.y, (int)w.z, (int)w.w};
    const i32x4 z = {0, 0, 0, 0};
    const i32x4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, z, 0, 0, 0);
    const float d0 = h2f(dd), d1 = h2f(dd >> 16);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int t = min(2 * q + (v >> 1), ncol - 1), sb = 2 * c + (v & 1);
        const float val = ((v & 1) ? d1 : d0) * sxd[t * nsb + sb] * (float)D[v];
        acc[v] += live ? val : 0.f;
    }
}

__global__ void __launch_bounds__(64 * kQ8MWaves) k_gemv_q80_mfma(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                                const float* __restrict__ xd, float* __restrict__ y, int N, int K,
                                                                int ncol) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int nsb = K >> 5, nch = K >> 6, kp = K + 64, drs = (K >> 4) + 4;
    const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: a scalar chunk loop
    const int row0 = blockIdx.x * 16;
    const size_t rb = (size_t)K + (size_t)(K >> 4);
    const uint8_t* rp = W + (size_t)min(row0 + j, N - 1) * rb;
    uint8_t* const xl = smem;
    uint8_t* const dl = smem + gemv_q80_mfma_x_bytes(K, ncol);
    float* const sxd = (float*)(dl + gemv_q80_mfma_d_bytes(K));
    // staged ahead of the weights (loads retire in issue order, so the LDS stores wait for them only),
    // every item clamped to the last one (a clamped item stores its own bytes again): x scales, x, d
    const int nx2 = ncol * (nsb >> 1), nxq = ncol * (K >> 4), ndq = 16 * (K >> 6);
    const float rk = __builtin_amdgcn_rcpf((float)(K >> 4)), rd = __builtin_amdgcn_rcpf((float)(K >> 6));
    float2 sv[kQ8MScaleRegs];
    uint4 xv[kQ8MXRegs];
    uint32_t dv[kQ8MDRegs];
#pragma unroll
    for (int r = 0; r < kQ8MScaleRegs; ++r) sv[r] = ((const float2*)xd)[min(tid + 64 * kQ8MWaves * r, nx2 - 1)];
#pragma unroll
    for (int r = 0; r < kQ8MXRegs; ++r) xv[r] = ld16(xq + (size_t)min(tid + 64 * kQ8MWaves * r, nxq - 1) * 16);
#pragma unroll
    for (int r = 0; r < kQ8MDRegs; ++r) {                   // dword e: row e / (K/64), K/64 dwords per row
        const int e = min(tid + 64 * kQ8MWaves * r, ndq - 1), rr = div_small(e, K >> 6, rd);
        dv[r] = *(const uint32_t*)(W + (size_t)min(row0 + rr, N - 1) * rb + K + (size_t)(e - rr * (K >> 6)) * 4);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int nm = (nch - wave + kQ8MWaves - 1) / kQ8MWaves;    // chunks c = wave + W m of this wave (may be 0)
    auto chk = [&](int m) { return min(wave + kQ8MWaves * min(m, max(nm - 1, 0)), nch - 1); };
    // every weight load unconditional (clamped chunk), so the wait counts stay exact
    uint4 R[kQ8MRing];
#pragma unroll
    for (int r = 0; r < kQ8MRing; ++r) R[r] = ld16_a4(rp + 64 * (size_t)chk(r) + 16 * q);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < kQ8MScaleRegs; ++r) ((float2*)sxd)[min(tid + 64 * kQ8MWaves * r, nx2 - 1)] = sv[r];
#pragma unroll
    for (int r = 0; r < kQ8MXRegs; ++r) {
        const int e = min(tid + 64 * kQ8MWaves * r, nxq - 1), c = div_small(e, K >> 4, rk);
        *(uint4*)(xl + c * kp + 16 * (e - c * (K >> 4))) = xv[r];
    }
#pragma unroll
    for (int r = 0; r < kQ8MDRegs; ++r) {
        const int e = min(tid + 64 * kQ8MWaves * r, ndq - 1), rr = div_small(e, K >> 6, rd);
        *(uint32_t*)(dl + rr * drs + 4 * (e - rr * (K >> 6))) = dv[r];
    }
    if (tid == 0) *(uint4*)(xl + ncol * kp) = make_uint4(0, 0, 0, 0);
    lds_barrier();
    // the lane's A piece: token j >> 1 at chunk offset 16q when q >> 1 == j & 1, else the zero bytes
    const int t = j >> 1;
    const bool xa_on = (q >> 1) == (j & 1) && t < ncol;
    const uint8_t* const xa = xa_on ? xl + t * kp + 16 * q : xl + ncol * kp;
    const int xs = xa_on ? 64 : 0;
    const uint8_t* const da = dl + j * drs;
    float acc[8][4];
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[k][v] = 0.f;
    // at least one pass: a loop that might not run would let the compiler sink the ring's loads past
    // the barrier into its entry
    int m0 = 0;
    do {                                                     // wave-uniform
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int m = m0 + k;
            q8m_compute(R[k % kQ8MRing], xa, xs, chk(m), q, da, sxd, nsb, ncol, m < nm, acc[k]);
            // the refill stays right here: the scheduler would otherwise move the ring's loads next to
            // their uses and drain the queue
            __builtin_amdgcn_sched_barrier(0);
            R[k % kQ8MRing] = ld16_a4(rp + 64 * (size_t)chk(m + kQ8MRing) + 16 * q);
            __builtin_amdgcn_sched_barrier(0);
        }
        m0 += 8;
    } while (m0 < nm);
    lds_barrier();                                           // every wave is done with the staged x, d and scales
    float* part = (float*)smem;                              // [unit-kernel lane L][token][row]
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int v = 0; v < 4; ++v) part[((2 * wave + (v & 1) + 8 * k) * 8 + 2 * q + (v >> 1)) * 16 + j] = acc[k][v];
    lds_barrier();
    for (int e = tid; e < 16 * ncol; e += 64 * kQ8MWaves) {
        const int orow = e & 15, oc = e >> 4;
        if (row0 + orow >= N) continue;
        // the association order of the butterfly over the 64 lanes of the unit kernel's row wave
        float a[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) a[u] = part[(u * 8 + oc) * 16 + orow] + part[((u + 32) * 8 + oc) * 16 + orow];
#pragma unroll
        for (int u = 0; u < 16; ++u) a[u] = a[u] + a[u + 16];
#pragma unroll
        for (int u = 0; u < 8; ++u) a[u] = a[u] + a[u + 8];
#pragma unroll
        for (int u = 0; u < 4; ++u) a[u] = a[u] + a[u + 4];
        a[0] = a[0] + a[2];
        a[1] = a[1] + a[3];
        y[(size_t)oc * N + row0 + orow] = a[0] + a[1];
    }
}
}  // namespace

// x in LDS: up to 8 columns whose x fits the staging registers
static bool gemv_q4k_mfma_xl(int K, int ncol) { return ncol <= 8 && ncol * K <= xl_max(ncol <= 4 ? 1 : 2); }

size_t gemv_q4k_mfma_lds(int K, int ncol) {
    const int mv = ncol <= 4 ? 1 : ncol <= 8 ? 2 : 4;
    return K > kMfmaMaxK ? SIZE_MAX
                         : gemv_q4k_mfma_main_lds(K, mv) +
                               (gemv_q4k_mfma_xl(K, ncol) ? gemv_q4k_mfma_xl_bytes(K, ncol) : 0);
}

// ncol (1..16) columns of q8 x against nseg (1..4) Q4_K segments sharing K, in one launch.  Shapes are
// checked by the caller (K % 256 == 0, N > 0).
int gemv_q4k_mfma(const qmm_gemv_seg* segs, int nseg, qmm_xq8 x, int K, int ncol, hipStream_t s) {
    if (nseg < 1 || nseg > kMfmaMaxSeg || ncol < 1 || ncol > 16) return QMM_ERR_SHAPE;
    MSegs sg = {};
    sg.nseg = nseg;
    sg.t0[0] = 0;
    for (int i = 0; i < nseg; ++i) {
        sg.w[i] = (const uint8_t*)segs[i].w;
        sg.y[i] = segs[i].y;
        sg.N[i] = segs[i].N;
        sg.t0[i + 1] = sg.t0[i] + (segs[i].N + 15) / 16;
    }
    const int mv = ncol <= 4 ? 1 : ncol <= 8 ? 2 : 4;
    const size_t lds = gemv_q4k_mfma_lds(K, ncol);
    if (lds > kMfmaLdsMax) return QMM_ERR_SHAPE;
    const dim3 grid((unsigned)sg.t0[nseg]);
    switch (mv) {
        case 1:
            if (gemv_q4k_mfma_xl(K, ncol))
                hipLaunchKernelGGL((k_gemv_q4k_mfma<1, true>), grid, dim3(256), lds, s, sg, x.q, x.d, x.s, K, ncol);
            else
                hipLaunchKernelGGL((k_gemv_q4k_mfma<1, false>), grid, dim3(256), lds, s, sg, x.q, x.d, x.s, K, ncol);
            break;
        case 2:
            if (gemv_q4k_mfma_xl(K, ncol))
                hipLaunchKernelGGL((k_gemv_q4k_mfma<2, true>), grid, dim3(256), lds, s, sg, x.q, x.d, x.s, K, ncol);
            else
                hipLaunchKernelGGL((k_gemv_q4k_mfma<2, false>), grid, dim3(256), lds, s, sg, x.q, x.d, x.s, K, ncol);
            break;
        default: hipLaunchKernelGGL((k_gemv_q4k_mfma<4, false>), grid, dim3(256), lds, s, sg, x.q, x.d, x.s, K, ncol); break;
    }
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

// the shapes whose x scales, block scales and d the Q6_K_SOA kernel stages in one pass
bool gemv_q6k_mfma_fits(int K, int ncol) {
    return (size_t)ncol * (K / 128) <= (size_t)64 * kQ6MWaves * kQ6MScaleRegs && (size_t)16 * (K / 256) <= (size_t)64 * kQ6MWaves * kQ6MScRegs &&
           (size_t)8 * (K / 256) <= (size_t)64 * kQ6MWaves * kQ6MDRegs;
}

// ncol (1..8) columns of q8 x against a Q6_K_SOA matrix (K % 512 == 0, 512 <= K, gemv_q6k_mfma_fits),
// bitwise the unit kernel's columns
int gemv_q6k_mfma(const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, hipStream_t s) {
    if (ncol < 1 || ncol > 8 || K < 512 || K % 512 || N < 1) return QMM_ERR_SHAPE;
    if (!gemv_q6k_mfma_fits(K, ncol)) return QMM_ERR_SHAPE;   // x scales, block scales and d in one staging pass
    const size_t lds = gemv_q6k_mfma_lds(K, ncol);
    if (lds > kMfmaLdsMax) return QMM_ERR_SHAPE;
    const dim3 grid((unsigned)((N + 15) / 16));
    if (ncol <= 4)
        hipLaunchKernelGGL(k_gemv_q6k_mfma<1>, grid, dim3(64 * kQ6MWaves), lds, s, (const uint8_t*)W, x.q, x.d, y, N, K, ncol);
    else
        hipLaunchKernelGGL(k_gemv_q6k_mfma<2>, grid, dim3(64 * kQ6MWaves), lds, s, (const uint8_t*)W, x.q, x.d, y, N, K, ncol);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

// the shapes whose x, d and x scales the kernel stages in one pass
bool gemv_q80_mfma_fits(int K, int ncol) {
    return ncol >= 1 && ncol <= 8 && K >= 64 && K % 64 == 0 && (size_t)ncol * (K / 64) <= (size_t)64 * kQ8MWaves * kQ8MScaleRegs &&
           (size_t)ncol * (K / 16) <= (size_t)64 * kQ8MWaves * kQ8MXRegs && (size_t)K / 4 <= (size_t)64 * kQ8MWaves * kQ8MDRegs;
}

// ncol (1..8) columns of q8 x against a Q8_0_SOA matrix (gemv_q80_mfma_fits, x.d 8-byte aligned),
// bitwise the unit kernel's columns
int gemv_q80_mfma(const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, hipStream_t s) {
    if (!gemv_q80_mfma_fits(K, ncol) || N < 1 || ((uintptr_t)x.d & 7)) return QMM_ERR_SHAPE;
    const size_t lds = gemv_q80_mfma_lds(K, ncol);
    const dim3 grid((unsigned)((N + 15) / 16));
    hipLaunchKernelGGL(k_gemv_q80_mfma, grid, dim3(64 * kQ8MWaves), lds, s, (const uint8_t*)W, x.q, x.d, y, N, K, ncol);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

}  // namespace qmm
