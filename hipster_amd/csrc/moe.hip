// moe.hip -- MoE decode path on gfx950 (wave64): routing, expert gather GEMV (gate|up), silu*up ->
// q8, down projection with the weighted combine, and the prefill combine over sorted rows.
//
// Entry points (C ABI, include/hipster_qmm.h) and the reference functions they replace:
//   qmm_moe_route / qmm_moe_route_n   fn::moe_route        engine/kernels/fn.hip:157-205,301
//   qmm_gemv_moe                      hip::gemv_moe        engine/kernels/gemv.hip:1075-1129,1385-1394
//   qmm_moe_silu_quant                fn::moe_silu_quant   engine/kernels/fn.hip:206-211,305
//   qmm_moe_combine_sorted            fn::moe_combine_sorted engine/kernels/fn.hip:126-132,295-297
//   qmm_moe_decode / _noalloc         (route, gate|up, silu-q8, down: qwen4exp.cpp:345-354 in one call)
//
// Expert gather (gate|up, or any call without slot weights): the reference launches one thread
// group per (token, slot, row block), so an expert picked by several tokens, and the shared expert
// (picked by every token), is streamed once per token.  Here the workgroup of slot te first checks
// on the device whether an earlier slot routes to the same expert; if so it exits, otherwise it
// computes every slot of that expert as columns of one weight read (at most 8 columns per pass).
// Each distinct expert is thus read once per step, with no host sync and no extra launch.  A
// column's arithmetic is the same whatever the number of columns (T-invariant, bitwise).
//
// Down projection with slot weights: y[t][n] = sum_e slotw[t,e] * (W_{ids[t,e]} . x[t*nexp+e]).
// The waves of a workgroup (8 at one token, 4 from two on) split the slots of one token; the per-slot
// row results meet in LDS and one lane per row adds them in slot order (deterministic, no atomics).
#include "q4k_pair.hpp"
#include "qmm_common.hpp"

#include <hip/hip_runtime.h>

#include <mutex>

// Workspace of qmm_moe_decode_noalloc: one copy per GPU, held until the process ends.  Host code
// never passes this name to a kernel or a copy (on the host it is only a stand-in for the symbol):
// moe_scratch() looks up each device's address once and every use goes through that pointer.
constexpr size_t kDecScratchBytes = (size_t)2 << 20;
static __device__ __align__(256) uint8_t scratch[kDecScratchBytes];

namespace qmm {
namespace {

constexpr int kMaxCols = 8;        // columns per pass of the gather GEMV
constexpr int kMaxSlots = 16;      // slots per token

// ------------------------------------------------------------------------------------------
// Routing (fn.hip:157-205).  One wave per token (4 tokens per workgroup), VPL logits per lane (expert
// lane + 64 j).  The arithmetic is the reference's: mx = max of the logits; e = __expf(l - mx); the
// denominator is the xor-butterfly sum of e over each 32 consecutive experts (experts 32g..32g+31 are
// the 32 lanes of half g & 1 of value j = g >> 1), then those group sums added in order; p = e / sum;
// the top-k by p with ties to the lower id; weights p / (the selected p summed in selection order);
// slot k is the shared expert: id -1, weight sigmoid(logit[nexp]).  The top-k is found by ranks, not
// by k sequential argmax rounds (route_token): (p, id) packed as one 64-bit key, a threshold from the
// ranks of the lanes' best keys, then the keys at or above it ranked against each other in LDS.

// one DPP step of a wave max / min (lanes without a source see the neutral value)
template <int CTRL, int ROWS>
__device__ __forceinline__ float max_dpp(float v) {
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), CTRL, ROWS, 0xf, false)));
}
template <int CTRL, int ROWS>
__device__ __forceinline__ int min_dpp(int v) {
    return min(v, __builtin_amdgcn_update_dpp(0x7fffffff, v, CTRL, ROWS, 0xf, false));
}
// DPP row_shr 1/2/4/8 leave each row's result in its lane 15; row_bcast15 / row_bcast31 carry them
// into lane 63, which is read back as a wave-uniform value.
__device__ __forceinline__ float wave_max64(float v) {
    v = max_dpp<0x111, 0xf>(v); v = max_dpp<0x112, 0xf>(v); v = max_dpp<0x114, 0xf>(v); v = max_dpp<0x118, 0xf>(v);
    v = max_dpp<0x142, 0xa>(v); v = max_dpp<0x143, 0xc>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
template <int CTRL, int ROWS>
__device__ __forceinline__ int imax_dpp(int v) {
    return max(v, __builtin_amdgcn_update_dpp((int)0x80000000, v, CTRL, ROWS, 0xf, false));
}
__device__ __forceinline__ int wave_imax64(int v) {
    v = imax_dpp<0x111, 0xf>(v); v = imax_dpp<0x112, 0xf>(v); v = imax_dpp<0x114, 0xf>(v); v = imax_dpp<0x118, 0xf>(v);
    v = imax_dpp<0x142, 0xa>(v); v = imax_dpp<0x143, 0xc>(v);
    return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ int wave_min64(int v) {
    v = min_dpp<0x111, 0xf>(v); v = min_dpp<0x112, 0xf>(v); v = min_dpp<0x114, 0xf>(v); v = min_dpp<0x118, 0xf>(v);
    v = min_dpp<0x142, 0xa>(v); v = min_dpp<0x143, 0xc>(v);
    return __builtin_amdgcn_readlane(v, 63);
}

constexpr int kRouteMaxK = 16, kRouteMaxExp = 1024;
// LDS of one routing wave (64-bit words): the 64 lane heads, the candidates (at most topk lanes x 16
// entries), the topk selections in rank order
constexpr int kRouteLdsWords = 64 + kRouteMaxK * 16 + kRouteMaxK;

// (p bits, id) as one unsigned 64-bit key whose order is the selection order: higher p first (the bits
// of p as a signed int, offset to unsigned: every p >= 0 above a missing expert's -inf), then the
// lower id
__device__ __forceinline__ uint64_t route_key(int pbits, int id) {
    return ((uint64_t)((uint32_t)pbits ^ 0x80000000u) << 32) | (uint32_t)(0xffffffffu - (uint32_t)id);
}

// r[q & 3] += how many of the 16 keys at ks (LDS, 16-byte aligned) exceed mine: eight 16-byte reads in
// flight before the comparisons, so one LDS latency covers 16 keys
__device__ __forceinline__ void route_count16(const uint64_t* ks, uint64_t mine, int (&r)[4]) {
    ulonglong2 h[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) h[q] = *(const ulonglong2*)(ks + 2 * q);
#pragma unroll
    for (int q = 0; q < 8; ++q) r[q & 3] += (h[q].x > mine) + (h[q].y > mine);
}

// one wave routes the token whose logits start at l: ids / weights of its topk + 1 slots to idt / wt;
// lds: kRouteLdsWords words of LDS private to this wave
template <int VPL>
__device__ __forceinline__ void route_token(const float* __restrict__ l, int nexp, int topk, int* idt, float* wt, uint64_t* lds) {
    const int lane = threadIdx.x & 63;
    float v[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {                      // unconditional (clamped) loads: no wait per load
        const float x = l[min(lane + 64 * j, nexp - 1)];
        v[j] = lane + 64 * j < nexp ? x : -INFINITY;
    }
    const float gate = l[nexp];
    float mx = v[0];
#pragma unroll
    for (int j = 1; j < VPL; ++j) mx = fmaxf(mx, v[j]);
    mx = wave_max64(mx);
    float e[VPL], gs[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) e[j] = lane + 64 * j < nexp ? __expf(v[j] - mx) : 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) gs[j] = hw32_sum(e[j]);
    float sum = 0.f;                                     // groups past nexp add +0 (exact)
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gs[j]), 0));
        sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gs[j]), 32));
    }
    // Top-k without sequential rounds.  Every expert's key (route_key of p = e / sum); the lane's best
    // key is its head.  The topk-th best head theta bounds the selection: the topk best keys are all >=
    // theta and lie in the topk lanes whose heads are >= theta.  So: rank the 64 heads against each
    // other, take theta, gather the keys >= theta (at most topk x VPL), rank them against each other;
    // rank r < topk is selection r.  The same selections and order as taking the best key topk times.
    uint64_t key[VPL], head = 0;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        key[j] = route_key(__float_as_int(lane + 64 * j < nexp ? e[j] / sum : -INFINITY), lane + 64 * j);
        head = key[j] > head ? key[j] : head;
    }
    uint64_t* const heads = lds;
    uint64_t* const cand = lds + 64;
    uint64_t* const sel = lds + 64 + kRouteMaxK * 16;
    heads[lane] = head;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    int hr[4] = {0, 0, 0, 0};                            // four independent counts (no add chain)
#pragma unroll
    for (int m = 0; m < 64; m += 16) route_count16(heads + m, head, hr);
    const int hrank = (hr[0] + hr[1]) + (hr[2] + hr[3]);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(hrank == topk - 1);   // exactly one lane
    const int tl = __builtin_ctzll(hit);
    const uint64_t theta = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(head >> 32), tl) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)head, tl);
    int nc = 0;                                          // wave-uniform candidate count
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const bool c = key[j] >= theta;
        const uint64_t b = __builtin_amdgcn_ballot_w64(c);
        if (c) cand[nc + __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0))] = key[j];
        nc += __builtin_popcountll(b);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    for (int c0 = 0; c0 < nc; c0 += 64) {                // candidate c0 + lane: its rank among all nc
        const int ci = c0 + lane;
        const uint64_t mine = cand[min(ci, nc - 1)];
        int rc[4] = {0, 0, 0, 0};
        int m = 0;
        for (; m + 16 <= nc; m += 16) route_count16(cand + m, mine, rc);
        for (; m < nc; ++m) rc[m & 3] += cand[m] > mine;
        const int r = (rc[0] + rc[1]) + (rc[2] + rc[3]);
        if (ci < nc && r < topk) sel[r] = mine;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float psel = 0.f, wsum = 0.f;
    int isel = 0;
    for (int r = 0; r < topk; ++r) {                     // the selected p summed in selection order
        const uint64_t k = sel[r];
        const float pr = __uint_as_float((uint32_t)(k >> 32) ^ 0x80000000u);
        if (lane == r) { psel = pr; isel = (int)(0xffffffffu - (uint32_t)k); }
        wsum += pr;
    }
    if (lane < topk) { idt[lane] = isel; wt[lane] = psel / wsum; }
    if (lane == topk) { idt[topk] = -1; wt[topk] = 1.f / (1.f + __expf(-gate)); }
}

template <int VPL>
__global__ void __launch_bounds__(256) k_moe_route(const float* __restrict__ logits, int* __restrict__ ids,
                                                   float* __restrict__ w, int T, int nexp, int stride, int topk) {
    __shared__ __align__(16) uint64_t lds[4][kRouteLdsWords];   // 16-byte reads of the heads (2688 B per wave)
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;                                  // wave-uniform
    route_token<VPL>(logits + (size_t)t * stride, nexp, topk, ids + (size_t)t * (topk + 1), w + (size_t)t * (topk + 1),
                     lds[threadIdx.x >> 6]);
}

// ------------------------------------------------------------------------------------------
// h = silu(g) * u quantised per 32 (fn.hip:206-211): one 32-lane half-wave per sub-block.
__device__ __forceinline__ float silu_f(float x) { return x / (1.f + __expf(-x)); }

__device__ __forceinline__ void half_wave_quant32(float v, int8_t* __restrict__ q, float* __restrict__ d,
                                                  float* __restrict__ s, size_t sb, int l) {
    float amax = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    const float dd = amax / 127.f, id = amax > 0.f ? 127.f / amax : 0.f;
    const int qi = __float2int_rn(v * id);
    int sum = qi;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 32);
    q[sb * 32 + l] = (int8_t)qi;
    if (l == 0) { d[sb] = dd; s[sb] = dd * (float)sum; }
}

__global__ void __launch_bounds__(256) k_moe_silu_quant(const float* __restrict__ g, const float* __restrict__ u,
                                                        int8_t* __restrict__ q, float* __restrict__ d, float* __restrict__ s,
                                                        size_t nsb) {
    const size_t sb = (size_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int l = threadIdx.x & 31;
    if (sb >= nsb) return;
    const size_t i = sb * 32 + l;
    half_wave_quant32(silu_f(g[i]) * u[i], q, d, s, sb, l);
}

// ------------------------------------------------------------------------------------------
// Expert gather GEMV, Q4_K experts and shared expert.  grid = (row blocks, slots, segments).
// Row block = 4 waves x (64 / LPR) rows.  I = pair iterations per row (ceil(4 K/256 / LPR)).
template <int LPR, int I, int NC, bool EXACT>
__device__ __forceinline__ void moe_cols(const Q4kPairs<I>& A, int t, int j, int ntask, uint8_t* smem, int K, int N, int row,
                                         const int* cols, float* __restrict__ y) {
    XPairSrc<true> xs[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) xs[c] = XPairSrc<true>{smem + (size_t)c * (K + (K >> 2)), nullptr, nullptr, K};
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.f;
    const Q4kPairDecode dc(j);
    q4k_pairs_compute<NC, I, true, EXACT, LPR>(A, dc, t, ntask, 0, xs, acc);
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = group_sum(acc[c], LPR);
    if (t == 0 && row < N) {
#pragma unroll
        for (int c = 0; c < NC; ++c) y[(size_t)cols[c] * N + row] = acc[c];
    }
}

// stage the x rows xrow[c] (c < nc) of q8 x into LDS in the pair layout (column c at c * 5K/4)
__device__ __forceinline__ void stage_gather(uint8_t* lds, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                             const float* __restrict__ xsum, const int* xrow, int nc, int K) {
    const int nu = K >> 4, kq = K >> 6, nsb = K >> 5;
    for (int v = threadIdx.x; v < nc * nu; v += blockDim.x) {
        const int c = v / nu, u = v - c * nu, p = u >> 2, q = u & 3;
        *(uint4*)(lds + (size_t)c * (K + (K >> 2)) + (size_t)(q * kq + p) * 16) = ld16(xq + (size_t)xrow[c] * K + (size_t)u * 16);
    }
    for (int v = threadIdx.x; v < nc * kq; v += blockDim.x) {
        const int c = v / kq, p = v - c * kq;
        const float2 dd = *(const float2*)(xd + (size_t)xrow[c] * nsb + 2 * p), ss = *(const float2*)(xsum + (size_t)xrow[c] * nsb + 2 * p);
        *(float4*)(lds + (size_t)c * (K + (K >> 2)) + (size_t)K + (size_t)p * 16) = make_float4(dd.x, dd.y, ss.x, ss.y);
    }
}

// stage_gather in two halves, for the x rows row0 .. row0 + nc - 1 of a workgroup whose x items
// (nc * (K/16 + K/64) 16-byte pieces) fit NR per thread: load() issues every piece into registers at
// once, store() writes them where stage_gather does.  A caller loads first and stores after its weight
// loads are issued, so the x latency overlaps its ids -> weights chain (loads retire in issue order:
// the stores wait for x only).  No branches: every thread loads two 8-byte halves per item (an item
// past the last is the last again, stored twice with the same bytes), so the compiler's wait counts
// stay exact.
template <int NR>
struct GatherRegs {
    uint2 lo[NR], hi[NR];
    // item v: q piece u of row c (v = c * nu + u) below nq, else the (d, s) pair piece p of row c
    // (v - nq = c * kq + p); off = its LDS offset
    __device__ __forceinline__ static void item(int v, int K, int nc, int& c, int& u, bool& isq) {
        const int nu = K >> 4, kq = K >> 6, nq = nc * nu;
        isq = v < nq;
        const int d = isq ? nu : kq, w = isq ? v : v - nq;
        c = div_small(w, d, __builtin_amdgcn_rcpf((float)d));
        u = w - c * d;
    }
    __device__ __forceinline__ void load(const int8_t* __restrict__ xq, const float* __restrict__ xd, const float* __restrict__ xsum,
                                         int row0, int nc, int K) {
        const int n = nc * ((K >> 4) + (K >> 6)), nsb = K >> 5;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            int c, u;
            bool isq;
            item(min((int)threadIdx.x + (int)blockDim.x * r, n - 1), K, nc, c, u, isq);
            const int8_t* pq = xq + (size_t)(row0 + c) * K + (size_t)u * 16;
            const size_t ps = (size_t)(row0 + c) * nsb + 2 * u;
            lo[r] = *(const uint2*)(isq ? (const void*)pq : (const void*)(xd + ps));
            hi[r] = *(const uint2*)(isq ? (const void*)(pq + 8) : (const void*)(xsum + ps));
        }
    }
    __device__ __forceinline__ void store(uint8_t* lds, int nc, int K) const {
        const int n = nc * ((K >> 4) + (K >> 6)), kq = K >> 6;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            int c, u;
            bool isq;
            item(min((int)threadIdx.x + (int)blockDim.x * r, n - 1), K, nc, c, u, isq);
            const size_t off = (size_t)c * (K + (K >> 2)) + (isq ? (size_t)((u & 3) * kq + (u >> 2)) * 16 : (size_t)K + (size_t)u * 16);
            *(uint4*)(lds + off) = make_uint4(lo[r].x, lo[r].y, hi[r].x, hi[r].y);
        }
    }
};

// the gather of slot te's expert for the columns s_cols[0..ncols) (after the dedup): weights of
// expert id (segment seg), x rows xrow_te ? slot : slot / nexp
template <int LPR, int I>
__device__ __forceinline__ void gather_expert(const qmm_moe_segs& a, int seg, int id, int ncols, const int* s_cols, uint8_t* smem,
                                              const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                              const float* __restrict__ xsum, int N, int K, int nexp, int xrow_te) {
    const int nb = K >> 8, ntask = 4 * nb, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, t = lane & (LPR - 1), j = t & 3;
    constexpr int RPW = 64 / LPR;
    const int row = (blockIdx.x * 4 + wave) * RPW + lane / LPR;
    const uint8_t* wbase = id >= 0 ? (const uint8_t*)a.w[seg] + (size_t)id * a.ebytes : (const uint8_t*)a.shared[seg];
    const uint8_t* rp = wbase + (size_t)min(row, N - 1) * ((size_t)nb * 144);
    float* y = a.y[seg];
    const bool exact = (ntask % LPR) == 0;
    // the expert's rows are loaded once, before the x staging, so both latencies overlap
    Q4kPairs<I> A;
    q4k_load_pairs<I, LPR>(rp, t, j, ntask, 0, A);
    for (int c0 = 0; c0 < ncols; c0 += kMaxCols) {
        const int nc = min(kMaxCols, ncols - c0);
        int xrow[kMaxCols];
#pragma unroll
        for (int c = 0; c < kMaxCols; ++c) {
            const int sl = s_cols[c0 + min(c, nc - 1)];
            xrow[c] = xrow_te ? sl : sl / nexp;
        }
        if (c0 > 0) __syncthreads();   // previous pass done with the LDS copy
        stage_gather(smem, xq, xd, xsum, xrow, nc, K);
        __syncthreads();
        const int* cols = s_cols + c0;
#define QMM_MOE_NC(NCV)                                                                                    \
    case NCV:                                                                                              \
        if (exact) moe_cols<LPR, I, NCV, true>(A, t, j, ntask, smem, K, N, row, cols, y);                  \
        else moe_cols<LPR, I, NCV, false>(A, t, j, ntask, smem, K, N, row, cols, y);                       \
        break;
        switch (nc) {
            QMM_MOE_NC(1) QMM_MOE_NC(2) QMM_MOE_NC(3) QMM_MOE_NC(4)
            QMM_MOE_NC(5) QMM_MOE_NC(6) QMM_MOE_NC(7) QMM_MOE_NC(8)
        }
#undef QMM_MOE_NC
    }
}

template <int LPR, int I>
__global__ void __launch_bounds__(256) k_gemv_moe_q4k(qmm_moe_segs a, const int* __restrict__ ids, int nexp,
                                                      const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                      const float* __restrict__ xsum, int N, int K, int nslot, int xrow_te) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_cols[64 + kMaxCols];
    __shared__ int s_n, s_dup;
    const int te = blockIdx.y, seg = blockIdx.z, tid = threadIdx.x;
    const int id = ids[te];
    if (tid < 64) moe_slot_columns(ids, nslot, te, id, s_cols, &s_n, &s_dup);
    __syncthreads();
    if (s_dup) return;
    gather_expert<LPR, I>(a, seg, id, s_n, s_cols, smem, xq, xd, xsum, N, K, nexp, xrow_te);
}

// ------------------------------------------------------------------------------------------
// The MoE decode step (qmm_moe_decode), T <= 8, two launches: k_moe_route_gu_q8 (routing, the
// gate|up rows and h = silu(g) * u as q8) and k_gemv_moe_down_q4k (the down projection and the
// slot-ordered combine).  The four-launch sequence moe_route, gemv_moe (gate|up), moe_silu_quant,
// gemv_moe (down) gives the same ids, weights, q8 of h and y bit for bit.
constexpr int kDecMaxTok = 8;
constexpr size_t kDecDownLds = 64 * 1024;   // dynamic LDS budget of the decode down projection

// The step's first launch (T <= 8): workgroup (32-row block rb, slot e) routes the T tokens (wave t
// routes token t, route_token: the arithmetic of k_moe_route) while the other waves stage the tokens'
// x; then, if e is the first slot holding its expert (the gather's dedup, moe_slot_columns), it
// computes rows rb*32..rb*32+31 of that expert's gate (the first half of the waves) and up (the second
// half) projections for
// every slot holding it (the columns, in slot order) with the gather's per-row arithmetic (q4k pairs
// over LPR lanes per row: the same floats as k_gemv_moe_q4k), meets them in LDS and writes, one
// half-wave per column, h = silu(g) * u quantised per 32 (half_wave_quant32: the q8 bits of
// k_moe_silu_quant).  The second launch is the plain q8 down projection (k_gemv_moe_down_q4k).
// Waves per workgroup.  At T = 1 (routing inside) LPR: each wave computes 64 / LPR rows in one pass
// (its 64 lanes are that many rows of LPR lanes), the shortest chain after the routing (T = 1 step
// 13.7 -> 13.4 us on one box against 8 waves at LPR 16); from two tokens on 8, each wave 8 rows in
// 8 / (64 / LPR) passes (16 waves measured 0.5-1.5 us slower at T = 4 and 8).  A row's arithmetic is
// the same either way.
template <int LPR, bool ROUTE>
constexpr int gu_waves() { return ROUTE ? LPR : 8; }

template <int NC, int LPR, int I, int NP>
__device__ __forceinline__ void gu_rows(const Q4kPairs<I> (&A)[NP], const uint8_t* smem, const int* cols, int nexp, int H,
                                        int t, int j, int ntask, int rbase, float (*s_g)[kDecMaxTok]) {
    constexpr int RPW = 64 / LPR;
    XPairSrc<true> xs[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) xs[c] = XPairSrc<true>{smem + (size_t)(cols[c] / nexp) * (H + (H >> 2)), nullptr, nullptr, H};
    const Q4kPairDecode dc(j);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        float acc[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[c] = 0.f;
        if ((ntask % LPR) == 0) q4k_pairs_compute<NC, I, true, true, LPR>(A[p], dc, t, ntask, 0, xs, acc);
        else q4k_pairs_compute<NC, I, true, false, LPR>(A[p], dc, t, ntask, 0, xs, acc);
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[c] = group_sum(acc[c], LPR);
        if (t == 0) {
#pragma unroll
            for (int c = 0; c < NC; ++c) s_g[rbase + p * RPW][c] = acc[c];
        }
    }
}

// ROUTE true (T = 1 only): wave 0 routes the token while the others stage x; ROUTE false: the ids come
// from ids_out (k_moe_route ran before), nothing is routed or written there.  XF (ROUTE false, the
// tokens' x fits kGuXItems 16-byte pieces): x and the slot ids are loaded into registers first, then
// the slot's expert rows (its id by a scalar load), and only then are x and the ids stored to LDS and
// the dedup run, so the x latency and the dedup overlap the weight loads (a slot that turns out to be a
// duplicate drops rows that the slot computing its expert loads as well)
constexpr int kGuXItems = 1536;
template <int LPR, int I, int VPL, bool ROUTE, bool XF>
__global__ void __launch_bounds__((64 * gu_waves<LPR, ROUTE>())) k_moe_route_gu_q8(qmm_moe_segs a, const float* __restrict__ logits, int stride,
                                                                  int nexp_total, int topk, int T, int* __restrict__ ids_out,
                                                                  float* __restrict__ w_out, const int8_t* __restrict__ xq,
                                                                  const float* __restrict__ xd, const float* __restrict__ xsum,
                                                                  int F, int H, int8_t* __restrict__ hq, float* __restrict__ hd,
                                                                  float* __restrict__ hs) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_ids[kDecMaxTok * kMaxSlots];
    __shared__ float s_w[kDecMaxTok * kMaxSlots];
    __shared__ int s_cols[64 + kMaxCols];
    __shared__ int s_n, s_dup;
    __shared__ float s_gu[2][32][kDecMaxTok];
    constexpr int GW = gu_waves<LPR, ROUTE>();
    // the wave index uniform (readfirstlane), so that the segment's base pointer is a scalar load that
    // does not wait for the vector loads issued before it
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, nexp = topk + 1, nslot = T * nexp;
    // x of the T tokens in the pair layout of stage_gather, token c at c * 5H/4
    auto stage = [&](int first, int step) {
        const int nu = H >> 4, kq = H >> 6, nsb = H >> 5;
        for (int v = first; v < T * nu; v += step) {
            const int c = v / nu, u = v - c * nu, pp = u >> 2, q = u & 3;
            *(uint4*)(smem + (size_t)c * (H + (H >> 2)) + (size_t)(q * kq + pp) * 16) = ld16(xq + (size_t)c * H + (size_t)u * 16);
        }
        for (int v = first; v < T * kq; v += step) {
            const int c = v / kq, pp = v - c * kq;
            const float2 dd = *(const float2*)(xd + (size_t)c * nsb + 2 * pp), ss = *(const float2*)(xsum + (size_t)c * nsb + 2 * pp);
            *(float4*)(smem + (size_t)c * (H + (H >> 2)) + (size_t)H + (size_t)pp * 16) = make_float4(dd.x, dd.y, ss.x, ss.y);
        }
    };
    static_assert(!(ROUTE && XF), "x ahead of the ids only without routing");
    const int e = blockIdx.y, rb = blockIdx.x;
    // GW / 2 waves per segment (gate, up), RW rows per wave in NP passes of RPW rows
    constexpr int RPW = 64 / LPR, RW = 64 / GW, NP = RW / RPW;
    static_assert(NP >= 1 && NP * RPW == RW, "a wave's rows are whole passes");
    const int seg = wave / (GW / 2), rbase = (wave % (GW / 2)) * RW + lane / LPR;
    const int nb = H >> 8, ntask = 4 * nb, t = lane & (LPR - 1), j = t & 3;
    Q4kPairs<I> A[NP];
    auto load_rows = [&](int id) {                           // this wave's rows of expert id (gate or up)
        const uint8_t* wbase = id >= 0 ? (const uint8_t*)a.w[seg] + (size_t)id * a.ebytes : (const uint8_t*)a.shared[seg];
#pragma unroll
        for (int p = 0; p < NP; ++p)
            q4k_load_pairs<I, LPR>(wbase + (size_t)min(rb * 32 + rbase + p * RPW, F - 1) * ((size_t)nb * 144), t, j, ntask, 0, A[p]);
    };
    if constexpr (ROUTE) {                                   // T = 1 (the launcher routes here only then)
        __shared__ __align__(16) uint64_t s_route[kRouteLdsWords];
        if (wave == 0) route_token<VPL>(logits, nexp_total, topk, s_ids, s_w, s_route);
        else stage(tid - 64, 64 * (GW - 1));
        __syncthreads();
        if (rb == 0 && e == 0 && tid < nslot) {
            ids_out[tid] = s_ids[tid];
            w_out[tid] = s_w[tid];
        }
    } else if constexpr (XF) {
        GatherRegs<(kGuXItems + 64 * GW - 1) / (64 * GW)> g;
        g.load(xq, xd, xsum, 0, T, H);
        const int idv = ids_out[min(tid, nslot - 1)];
        __builtin_amdgcn_sched_barrier(0);
        load_rows(ids_out[e]);                               // e is uniform: a scalar load
        __builtin_amdgcn_sched_barrier(0);
        g.store(smem, T, H);
        if (tid < nslot) s_ids[tid] = idv;
        __syncthreads();
    } else {
        if (tid < nslot) s_ids[tid] = ids_out[tid];
        stage(tid, 64 * GW);
        __syncthreads();
    }
    const int id = s_ids[e];
    int ncols = 1;
    if constexpr (!ROUTE) {
        if (tid < 64) moe_slot_columns(s_ids, nslot, e, id, s_cols, &s_n, &s_dup);
        __syncthreads();
        if (s_dup) return;                                   // an earlier slot computes this expert
        ncols = min(s_n, kMaxCols);                          // at most T <= 8: a token holds an expert once
    }   // routed here (T = 1): the token's slots hold distinct experts, slot e is the one column
    if constexpr (!XF) load_rows(id);
    if constexpr (ROUTE) {
        const int col0[1] = {e};
        gu_rows<1, LPR, I, NP>(A, smem, col0, nexp, H, t, j, ntask, rbase, s_gu[seg]);
        if (tid == 0) s_cols[0] = e;
    } else {
        switch (ncols) {
#define QMM_GU(NCV) case NCV: gu_rows<NCV, LPR, I, NP>(A, smem, s_cols, nexp, H, t, j, ntask, rbase, s_gu[seg]); break;
            QMM_GU(1) QMM_GU(2) QMM_GU(3) QMM_GU(4) QMM_GU(5) QMM_GU(6) QMM_GU(7) QMM_GU(8)
#undef QMM_GU
        }
    }
    __syncthreads();
    if (tid < 32 * ncols) {                                  // one half-wave per column: its slot's q8 block
        const int c = tid >> 5, l = tid & 31;
        half_wave_quant32(silu_f(s_gu[0][l][c]) * s_gu[1][l][c], hq, hd, hs, (size_t)s_cols[c] * (F / 32) + rb, l);
    }
}

// the down projection of one token's slots: wave w of DW takes the slots e = w, w + DW, ... (at most
// kMaxSlots / DW of them); their weight rows are loaded before the caller stages x (stage(), then a
// barrier), per-slot row results go to LDS and lane r of wave 0 sums row r over the slots in order.
// A slot's row is one wave's work whatever the wave count, so the results do not depend on it: 8
// waves at one token (the slots' latency chains side by side: 14.7 against 15.5 us for the T = 1 decode
// step), 4 from two tokens on (more workgroups, fewer idle waves).
template <int LPR, int I, int DW, typename Pre, typename Stage>
__device__ __forceinline__ void down_slots(const qmm_moe_segs& a, const int* __restrict__ ids, int nexp, uint8_t* smem, int N, int K,
                                           Pre pre, Stage stage) {
    constexpr int RPW = 64 / LPR, SPW = kMaxSlots / DW;
    __shared__ float vres[kMaxSlots][RPW];
    __shared__ float sw[kMaxSlots];
    const int tok = blockIdx.y, tid = threadIdx.x;
    pre();                                               // x loads that need no ids, if the caller has them
    __builtin_amdgcn_sched_barrier(0);
    const float swv = a.slotw[tok * nexp + min(tid, nexp - 1)];   // read now, stored after the weight loads
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), t = lane & (LPR - 1), j = t & 3;
    const int nb = K >> 8, ntask = 4 * nb;
    const int rloc = lane / LPR, row = blockIdx.x * RPW + rloc;
    Q4kPairs<I> A[SPW];
    // every wave loads SPW slots' rows, a slot past the last being the last again (not computed): loads
    // on every path keep the wait before the x stores from covering the weights
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
        const int id = ids[tok * nexp + min(wave + DW * i, nexp - 1)];   // wave-uniform: a scalar load
        const uint8_t* wbase = id >= 0 ? (const uint8_t*)a.w[0] + (size_t)id * a.ebytes : (const uint8_t*)a.shared[0];
        q4k_load_pairs<I, LPR>(wbase + (size_t)min(row, N - 1) * ((size_t)nb * 144), t, j, ntask, 0, A[i]);
    }
    __builtin_amdgcn_sched_barrier(0);
    stage();
    if (tid < nexp) sw[tid] = swv;
    __syncthreads();
    const Q4kPairDecode dc(j);
    const bool exact = (ntask % LPR) == 0;
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
        const int e = wave + DW * i;
        if (e < nexp) {
            XPairSrc<true> xs[1] = {XPairSrc<true>{smem + (size_t)e * (K + (K >> 2)), nullptr, nullptr, K}};
            float acc[1] = {0.f};
            if (exact) q4k_pairs_compute<1, I, true, true, LPR>(A[i], dc, t, ntask, 0, xs, acc);
            else q4k_pairs_compute<1, I, true, false, LPR>(A[i], dc, t, ntask, 0, xs, acc);
            acc[0] = group_sum(acc[0], LPR);
            if (t == 0) vres[e][rloc] = acc[0];
        }
    }
    __syncthreads();
    if (tid < RPW && blockIdx.x * RPW + tid < N) {
        float acc = 0.f;
        for (int e = 0; e < nexp; ++e) acc += sw[e] * vres[e][tid];
        a.y[0][(size_t)tok * N + blockIdx.x * RPW + tid] = acc;
    }
}

// ------------------------------------------------------------------------------------------
// Down projection + weighted combine: grid = (row blocks of 64/LPR rows, tokens), down_slots over
// the token's slot rows of q8 x.

// XF: the token's x pieces (nexp * (K/16 + K/64) of 16 bytes) fit the kDownXItems a workgroup holds in
// registers (launch_down checks): they are loaded before the slot ids, their latency off the chain
// ids -> weights
constexpr int kDownXItems = 512;
template <int LPR, int I, int DW, bool XF>
__global__ void __launch_bounds__(64 * DW) k_gemv_moe_down_q4k(qmm_moe_segs a, const int* __restrict__ ids, int nexp,
                                                           const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                           const float* __restrict__ xsum, int N, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tok = blockIdx.y;
    if constexpr (XF) {                                  // the nexp slot rows of this token: tok * nexp + e
        GatherRegs<kDownXItems / (64 * DW)> g;
        down_slots<LPR, I, DW>(a, ids, nexp, smem, N, K, [&] { g.load(xq, xd, xsum, tok * nexp, nexp, K); },
                               [&] { g.store(smem, nexp, K); });
    } else {
        int xrow[kMaxSlots];
#pragma unroll
        for (int e = 0; e < kMaxSlots; ++e) xrow[e] = tok * nexp + min(e, nexp - 1);
        down_slots<LPR, I, DW>(a, ids, nexp, smem, N, K, [] {}, [&] { stage_gather(smem, xq, xd, xsum, xrow, nexp, K); });
    }
}

// ------------------------------------------------------------------------------------------
// prefill combine over expert-sorted rows (fn.hip:126-132): y[t][d] = sum_e w[t*nexp+e] * down[kpos[t*nexp+e]][d]
// one workgroup per token; thread i sums float4 columns i, i+256, ... in slot order
__global__ void __launch_bounds__(256) k_moe_combine_sorted(const float* __restrict__ down, const float* __restrict__ w,
                                                            const int* __restrict__ kpos, float* __restrict__ y, int nexp, int E,
                                                            bool vec4) {
    const int t = blockIdx.x;
    const int* kp = kpos + (size_t)t * nexp;
    const float* wt = w + (size_t)t * nexp;
    if (vec4) {                                          // E % 4 == 0, down and y 16-byte aligned
        const int E4 = E >> 2;
        for (int d4 = threadIdx.x; d4 < E4; d4 += 256) {
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int e = 0; e < nexp; ++e) {
                const float we = wt[e];
                const float4 v = ((const float4*)(down + (size_t)kp[e] * E))[d4];
                acc.x += we * v.x;
                acc.y += we * v.y;
                acc.z += we * v.z;
                acc.w += we * v.w;
            }
            ((float4*)(y + (size_t)t * E))[d4] = acc;
        }
    } else {
        for (int d = threadIdx.x; d < E; d += 256) {
            float acc = 0.f;
            for (int e = 0; e < nexp; ++e) acc += wt[e] * down[(size_t)kp[e] * E + d];
            y[(size_t)t * E + d] = acc;
        }
    }
}

// lanes per row for the expert GEMVs: 8 when a row has at most 8 pairs (K <= 512), else 16
inline int moe_lpr(int K) { return K / 256 * 4 <= 8 ? 8 : 16; }

template <int LPR>
int launch_gather(const qmm_moe_segs& a, int nseg, const int* ids, int nexp, qmm_xq8 x, int N, int K, int T, int xrow_te,
                  hipStream_t s) {
    const int iters = (K / 256 * 4 + LPR - 1) / LPR;
    const dim3 grid((N + 4 * (64 / LPR) - 1) / (4 * (64 / LPR)), T * nexp, nseg);
    const size_t lds = (size_t)kMaxCols * (K + K / 4);
    if (lds > 64 * 1024) return QMM_ERR_SHAPE;
#define QMM_G(IV) case IV: hipLaunchKernelGGL((k_gemv_moe_q4k<LPR, IV>), grid, dim3(256), lds, s, a, ids, nexp, x.q, x.d, x.s, N, K, T * nexp, xrow_te); break;
    switch (iters) {
        QMM_G(1) QMM_G(2) QMM_G(3) QMM_G(4) QMM_G(5) QMM_G(6)
        default: return QMM_ERR_SHAPE;
    }
#undef QMM_G
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

template <int LPR>
int launch_down(const qmm_moe_segs& a, const int* ids, int nexp, qmm_xq8 x, int N, int K, int T, hipStream_t s) {
    const int iters = (K / 256 * 4 + LPR - 1) / LPR;
    const dim3 grid((N + (64 / LPR) - 1) / (64 / LPR), T);
    const size_t lds = (size_t)nexp * (K + K / 4);
    if (lds > kDecDownLds) return QMM_ERR_SHAPE;
    const bool xf = (size_t)nexp * (K / 16 + K / 64) <= (size_t)kDownXItems;
#define QMM_D(IV)                                                                                                      \
    case IV:                                                                                                           \
        if (T == 1) {                                                                                                  \
            if (xf) hipLaunchKernelGGL((k_gemv_moe_down_q4k<LPR, IV, 8, true>), grid, dim3(512), lds, s, a, ids, nexp, x.q, x.d, x.s, N, K);  \
            else hipLaunchKernelGGL((k_gemv_moe_down_q4k<LPR, IV, 8, false>), grid, dim3(512), lds, s, a, ids, nexp, x.q, x.d, x.s, N, K);  \
        } else {                                                                                                       \
            if (xf) hipLaunchKernelGGL((k_gemv_moe_down_q4k<LPR, IV, 4, true>), grid, dim3(256), lds, s, a, ids, nexp, x.q, x.d, x.s, N, K);  \
            else hipLaunchKernelGGL((k_gemv_moe_down_q4k<LPR, IV, 4, false>), grid, dim3(256), lds, s, a, ids, nexp, x.q, x.d, x.s, N, K);  \
        }                                                                                                              \
        break;
    switch (iters) {
        QMM_D(1) QMM_D(2) QMM_D(3) QMM_D(4) QMM_D(5) QMM_D(6)
        default: return QMM_ERR_SHAPE;
    }
#undef QMM_D
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

// the step's first launch (k_moe_route_gu_q8): q8 of h into hq / hd / hs
template <int LPR, int VPL>
int launch_decode_gu_q8(const qmm_moe_segs& a, const float* logits, int stride, int nexp_total, int topk, int T, int* ids, float* w,
                        qmm_xq8 x, int F, int H, qmm_xq8 h, hipStream_t s) {
    const int iters = (H / 256 * 4 + LPR - 1) / LPR;
    const dim3 grid(F / 32, T * (topk + 1));
    const size_t lds = (size_t)T * (H + H / 4);
    const bool xf = (size_t)T * (H / 16 + H / 64) <= (size_t)kGuXItems;
    // without routing the kernel does not use VPL: one instance (VPL 1) serves every expert count
#define QMM_G(IV) case IV:                                                                                                   \
        if (T == 1)                                                                                                          \
            hipLaunchKernelGGL((k_moe_route_gu_q8<LPR, IV, VPL, true, false>), grid, dim3(64 * gu_waves<LPR, true>()), lds, s, a, logits,   \
                               stride, nexp_total, topk, T, ids, w, x.q, x.d, x.s, F, H, h.q, h.d, h.s);                      \
        else if (xf)                                                                                                         \
            hipLaunchKernelGGL((k_moe_route_gu_q8<LPR, IV, 1, false, true>), grid, dim3(64 * gu_waves<LPR, false>()), lds, s, a, logits,     \
                               stride, nexp_total, topk, T, ids, w, x.q, x.d, x.s, F, H, h.q, h.d, h.s);                      \
        else                                                                                                                 \
            hipLaunchKernelGGL((k_moe_route_gu_q8<LPR, IV, 1, false, false>), grid, dim3(64 * gu_waves<LPR, false>()), lds, s, a, logits,    \
                               stride, nexp_total, topk, T, ids, w, x.q, x.d, x.s, F, H, h.q, h.d, h.s);                      \
        break;
    switch (iters) {
        QMM_G(1) QMM_G(2) QMM_G(3) QMM_G(4) QMM_G(5) QMM_G(6)
        default: return QMM_ERR_SHAPE;
    }
#undef QMM_G
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

template <int VPL>
int decode_gu_q8_vpl(const qmm_moe_segs& a, const float* logits, int stride, int nexp_total, int topk, int T, int* ids, float* w,
                     qmm_xq8 x, int F, int H, qmm_xq8 h, hipStream_t s) {
    return moe_lpr(H) == 8 ? launch_decode_gu_q8<8, VPL>(a, logits, stride, nexp_total, topk, T, ids, w, x, F, H, h, s)
                           : launch_decode_gu_q8<16, VPL>(a, logits, stride, nexp_total, topk, T, ids, w, x, F, H, h, s);
}

}  // namespace

// checks shared by qmm_moe_decode and the workspace-free variant; 0 when the call can run
int moe_decode_check(int fmt, const void* Wg, const void* Wu, const void* Wd, const void* Sg, const void* Su, const void* Sd,
                     const float* logits, int stride, int nexp_total, int topk, qmm_xq8 x, int T, int H, int F, const int* ids,
                     const float* w, const float* y) {
    if (fmt != QMM_Q4_K) return QMM_ERR_FORMAT;
    if (!Wg || !Wu || !Wd || !Sg || !Su || !Sd || !logits || !x.q || !x.d || !x.s || !ids || !w || !y) return QMM_ERR_NULL;
    if (T < 0 || T > kDecMaxTok || nexp_total < 1 || nexp_total > kRouteMaxExp || topk < 1 || topk + 1 > kMaxSlots ||
        topk > nexp_total || stride < nexp_total + 1 || H <= 0 || F <= 0 || H % 256 || F % 256 || H > 6144 || F > 6144)
        return QMM_ERR_SHAPE;
    // the down launch holds every slot's q8 h row in LDS (launch_down's budget): refuse here, before
    // the first launch writes ids, w or the workspace
    if ((size_t)(topk + 1) * (F + F / 4) > kDecDownLds) return QMM_ERR_SHAPE;
    return QMM_OK;
}

// the two launches; workspace gu: the q8 of h (T * (topk + 1) * F bytes, then d and s per 32)
int moe_decode_run(const void* Wg, const void* Wu, const void* Wd, size_t ebytes_gu, size_t ebytes_d, const void* Sg, const void* Su,
                   const void* Sd, const float* logits, int stride, int nexp_total, int topk, qmm_xq8 x, int T, int H, int F, int* ids,
                   float* w, float* gu, float* y, hipStream_t s) {
    if (T == 0) return QMM_OK;
    const int nexp = topk + 1;
    const qmm_moe_segs ga = {{Wg, Wu}, {Sg, Su}, {nullptr, nullptr}, ebytes_gu, nullptr};
    // h as q8 at the start of the workspace
    const size_t nh = (size_t)T * nexp * F;
    const qmm_xq8 h = {(int8_t*)gu, gu + nh / 4, gu + nh / 4 + nh / 32};
    if (T > 1) {   // T routing waves in every workgroup cost more than a launch: route once first
        if (int e = qmm_moe_route_n(logits, ids, w, T, nexp_total, stride, topk, s)) return e;
    }
    const int rc = nexp_total <= 128 ? decode_gu_q8_vpl<2>(ga, logits, stride, nexp_total, topk, T, ids, w, x, F, H, h, s)
                 : nexp_total <= 256 ? decode_gu_q8_vpl<4>(ga, logits, stride, nexp_total, topk, T, ids, w, x, F, H, h, s)
                 : nexp_total <= 512 ? decode_gu_q8_vpl<8>(ga, logits, stride, nexp_total, topk, T, ids, w, x, F, H, h, s)
                                     : decode_gu_q8_vpl<16>(ga, logits, stride, nexp_total, topk, T, ids, w, x, F, H, h, s);
    if (rc != QMM_OK) return rc;
    const qmm_moe_segs da = {{Wd, nullptr}, {Sd, nullptr}, {y, nullptr}, ebytes_d, w};
    return moe_lpr(F) == 8 ? launch_down<8>(da, ids, nexp, h, H, F, T, s) : launch_down<16>(da, ids, nexp, h, H, F, T, s);
}

// the device address of `scratch` on the current device, looked up on the first call per device
int moe_scratch(void** out) {
    constexpr int kMaxDev = 64;
    static std::mutex mu;
    static void* ptr[kMaxDev] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return QMM_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return QMM_ERR_LAUNCH;
        ptr[dev] = p;
    }
    *out = ptr[dev];
    return QMM_OK;
}

}  // namespace qmm

using namespace qmm;

extern "C" {

int qmm_moe_route_n(const float* logits, int* ids, float* w, int T, int nexp, int stride, int topk, void* stream) {
    if (!logits || !ids || !w) return QMM_ERR_NULL;
    if (T < 0 || nexp < 1 || nexp > kRouteMaxExp || topk < 1 || topk > kRouteMaxK || topk > nexp || stride < nexp + 1)
        return QMM_ERR_SHAPE;
    if (T == 0) return QMM_OK;
    const dim3 grid((T + 3) / 4);
    hipStream_t s = (hipStream_t)stream;
    if (nexp <= 128) hipLaunchKernelGGL(k_moe_route<2>, grid, dim3(256), 0, s, logits, ids, w, T, nexp, stride, topk);
    else if (nexp <= 256) hipLaunchKernelGGL(k_moe_route<4>, grid, dim3(256), 0, s, logits, ids, w, T, nexp, stride, topk);
    else if (nexp <= 512) hipLaunchKernelGGL(k_moe_route<8>, grid, dim3(256), 0, s, logits, ids, w, T, nexp, stride, topk);
    else hipLaunchKernelGGL(k_moe_route<16>, grid, dim3(256), 0, s, logits, ids, w, T, nexp, stride, topk);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_moe_route(const float* logits, int* ids, float* w, int T, void* stream) {
    return qmm_moe_route_n(logits, ids, w, T, 512, 513, 10, stream);
}

int qmm_moe_silu_quant(const float* gate, const float* up, qmm_xq8 xq, int rows, int n, void* stream) {
    if (!gate || !up || !xq.q || !xq.d || !xq.s) return QMM_ERR_NULL;
    if (rows < 0 || n <= 0 || n % 32 != 0) return QMM_ERR_SHAPE;
    const size_t nsb = (size_t)rows * n / 32;
    if (nsb == 0) return QMM_OK;
    hipLaunchKernelGGL(k_moe_silu_quant, dim3((unsigned)((nsb + 7) / 8)), dim3(256), 0, (hipStream_t)stream, gate, up, xq.q, xq.d,
                       xq.s, nsb);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

int qmm_gemv_moe(int fmt, int shared_fmt, const qmm_moe_segs* a, int nseg, const int* ids, int nexp, qmm_xq8 x, int N, int K,
                 int T, int xrow_te, void* stream) {
    // the reference's combinations (gemv.hip:1386-1392): the shared expert in the routed format or in
    // Q8_0_SOA; routed Q4_K, Q5_K, IQ4_XS, Q8_0_SOA, Q5_1_SOA
    const bool fmt_ok = fmt == QMM_Q4_K || fmt == QMM_Q5_K || fmt == QMM_IQ4_XS || fmt == QMM_Q8_0_SOA || fmt == QMM_Q5_1_SOA;
    if (!fmt_ok || (shared_fmt != fmt && shared_fmt != QMM_Q8_0_SOA)) return QMM_ERR_FORMAT;
    if (!a || !ids || !x.q || !x.d || !x.s) return QMM_ERR_NULL;
    auto kgran = [](int f) { return f == QMM_Q5_1_SOA ? 32 : f == QMM_Q8_0_SOA ? 64 : 256; };   // as qmm_gemv_q8
    if (nseg < 1 || nseg > 2 || N <= 0 || K <= 0 || K % kgran(fmt) != 0 || K % kgran(shared_fmt) != 0 || T < 0 || nexp < 1 ||
        nexp > kMaxSlots)
        return QMM_ERR_SHAPE;
    if (T > 64) return QMM_ERR_SHAPE;   // at most 64 columns (tokens) per expert in the dedup list
    // a caller without a shared expert (the reference's bench_gemv gather) passes NULL shared matrices;
    // in the routed format a negative id then reads expert 0, so no slot reads through NULL
    qmm_moe_segs sg = *a;
    for (int g = 0; g < nseg; ++g) {
        if (!sg.shared[g] && shared_fmt == fmt) sg.shared[g] = sg.w[g];
        if (!sg.w[g] || !sg.shared[g] || !sg.y[g]) return QMM_ERR_NULL;
    }
    if (T == 0) return QMM_OK;
    hipStream_t s = (hipStream_t)stream;
    if (sg.slotw && nseg != 1) return QMM_ERR_ARG;
    if (fmt != QMM_Q4_K || shared_fmt != QMM_Q4_K) return moe_fmt_dispatch(fmt, shared_fmt, &sg, nseg, ids, nexp, x, N, K, T, xrow_te, s);
    if (sg.slotw) {
        return moe_lpr(K) == 8 ? launch_down<8>(sg, ids, nexp, x, N, K, T, s) : launch_down<16>(sg, ids, nexp, x, N, K, T, s);
    }
    return moe_lpr(K) == 8 ? launch_gather<8>(sg, nseg, ids, nexp, x, N, K, T, xrow_te, s)
                           : launch_gather<16>(sg, nseg, ids, nexp, x, N, K, T, xrow_te, s);
}

int qmm_moe_decode(int fmt, const void* Wg, const void* Wu, const void* Wd, size_t ebytes_gu, size_t ebytes_d, const void* Sg,
                   const void* Su, const void* Sd, const float* logits, int stride, int nexp_total, int topk, qmm_xq8 x, int T, int H,
                   int F, int* ids, float* w, float* ws, size_t ws_bytes, float* y, void* stream) {
    if (int e = moe_decode_check(fmt, Wg, Wu, Wd, Sg, Su, Sd, logits, stride, nexp_total, topk, x, T, H, F, ids, w, y)) return e;
    if (!ws) return QMM_ERR_NULL;
    if (ws_bytes < qmm_moe_decode_ws_bytes(T, topk, F)) return QMM_ERR_WORKSPACE;
    return moe_decode_run(Wg, Wu, Wd, ebytes_gu, ebytes_d, Sg, Su, Sd, logits, stride, nexp_total, topk, x, T, H, F, ids, w, ws, y,
                          (hipStream_t)stream);
}

size_t qmm_moe_decode_scratch_max(void) { return kDecScratchBytes; }

int qmm_moe_decode_noalloc(int fmt, const void* Wg, const void* Wu, const void* Wd, size_t ebytes_gu, size_t ebytes_d, const void* Sg,
                           const void* Su, const void* Sd, const float* logits, int stride, int nexp_total, int topk, qmm_xq8 x, int T,
                           int H, int F, int* ids, float* w, float* y, void* stream) {
    if (int e = moe_decode_check(fmt, Wg, Wu, Wd, Sg, Su, Sd, logits, stride, nexp_total, topk, x, T, H, F, ids, w, y)) return e;
    if (qmm_moe_decode_ws_bytes(T, topk, F) > kDecScratchBytes) return QMM_ERR_WORKSPACE;
    if (T == 0) return QMM_OK;
    void* ws = nullptr;
    if (int e = moe_scratch(&ws)) return e;
    // every byte of the workspace that the step reads it has written first in the same call: nothing
    // to clear.  Calls that overlap on one GPU (other streams, other threads) share it and race.
    return moe_decode_run(Wg, Wu, Wd, ebytes_gu, ebytes_d, Sg, Su, Sd, logits, stride, nexp_total, topk, x, T, H, F, ids, w, (float*)ws,
                          y, (hipStream_t)stream);
}

size_t qmm_moe_decode_ws_bytes(int T, int topk, int F) {
    // h = silu(gate) * up as q8: the bytes, then d and s per 32
    const size_t nh = T <= 0 || topk < 1 || F <= 0 ? 0 : (size_t)T * (topk + 1) * F;
    return nh + nh / 32 * 2 * sizeof(float);
}

int qmm_moe_combine_sorted(const float* down, const float* w, const int* kpos, float* y, int T, int nexp, int E, void* stream) {
    if (!down || !w || !kpos || !y) return QMM_ERR_NULL;
    if (T < 0 || nexp < 1 || E <= 0) return QMM_ERR_SHAPE;
    if (T == 0) return QMM_OK;
    const bool vec4 = E % 4 == 0 && ((uintptr_t)down & 15) == 0 && ((uintptr_t)y & 15) == 0;
    hipLaunchKernelGGL(k_moe_combine_sorted, dim3(T), dim3(256), 0, (hipStream_t)stream, down, w, kpos, y, nexp, E, vec4);
    QMM_LAUNCH_CHECK();
    return QMM_OK;
}

}  // extern "C"
