// hipster_qmm_shim.hpp -- header-only C++ shim that restores the reference engine's call surface
// (namespace hip in engine/kernels/gemv.h, gemm.h and the MoE part of fn.h) on top of the C ABI of
// libhipster_qmm.so (include/hipster_qmm.h).  An engine that includes this header instead of those
// three files compiles unchanged against the gfx950 library.
//
// Differences from the reference, all deliberate:
//  - errors (unsupported format, bad shape, launch failure) throw std::runtime_error carrying the
//    library's status string, where the reference calls abort() or misbehaves silently;
//  - gemv_wmma / gemv_wmma_ok map onto the library's T-invariant GEMV (any ncol gives every column
//    the same reduction order), so `mode` is accepted and ignored, except mode 3 (weights in the
//    experimental 16-row interleaved layout), which runs qmm_gemv_q8's reader of that layout per weight;
//  - the experiment knobs g_persist_blocks, g_moe_tpr and g_moe_fake exist and are ignored (launch
//    shapes here depend on the tensor shape only);
//  - moe_gemm keeps its signature and q8 arithmetic (Q4_K tiles on the int8 matrix cores, the other
//    formats on the VALU); the engine's fast prefill path
//    is moe_sort + moe_gemm_gate_up_bf16 + moe_gemm_bf16 (bf16 MFMA);
//  - BlasLt::gemm runs the library's own bf16 MFMA GEMM (no hipBLASLt, no autotune, no workspace);
//  - fn::moe_combine_sorted takes the row width from the hidden size E of the caller's model: the
//    reference fixes E = 2560 at compile time; here it is the template argument (default 2560).
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "hipster_qmm.h"

namespace hip {

namespace detail {
inline void ck(int status, const char* what) {
    if (status != QMM_OK) throw std::runtime_error(std::string(what) + ": " + qmm_status_string(status));
}
}  // namespace detail

// ---- gemv.h -------------------------------------------------------------------------------
inline int g_persist_blocks = 0;   // gemv.h:6 (accepted, not used)
inline int g_moe_tpr = 0;          // gemv.h:53 (accepted, not used)
inline int g_moe_fake = 0;         // gemv.h:54 (accepted, not used)
struct XQ8 { int8_t* q; float* d; float* s; float2* ds = nullptr; };                         // gemv.h:8
struct XQ8K { int8_t* q; float* d; int16_t* bs; };                                            // gemv.h:33
enum class WFmt { Q4_K, Q5_K, IQ4_XS, Q6_K_SOA, Q8_0_SOA, Q5_1_SOA };                           // gemv.h:13
struct GemvSeg { WFmt fmt; const void* w; float* y; int N, K; };                                 // gemv.h:27
struct MoeSegs { const void* w[2]; const void* shared[2]; float* y[2]; size_t ebytes; const float* slotw = nullptr; };  // gemv.h:43
struct MoeTile { int expert, k0, ncols; };                                                      // gemv.h:48

inline qmm_xq8 to_c(const XQ8& x) { return qmm_xq8{x.q, x.d, x.s, (void*)x.ds}; }
inline qmm_xq8k to_c(const XQ8K& x) { return qmm_xq8k{x.q, x.d, x.bs}; }

inline void quantize_x_q8(const float* x, XQ8 out, int ncol, int K, hipStream_t s) {
    detail::ck(qmm_quantize_x_q8(x, to_c(out), ncol, K, (void*)s), "quantize_x_q8");
}
inline size_t wfmt_row_bytes(WFmt f, int K) { return qmm_wfmt_row_bytes((int)f, K); }
inline void repack_row_q6_K(const uint8_t* src, uint8_t* dst, int K) {
    detail::ck(qmm_repack_row_q6_K(src, dst, K), "repack_row_q6_K");
}
inline void repack_row_q8_0(const uint8_t* src, uint8_t* dst, int K) {                       // gemv.h:16
    detail::ck(qmm_repack_row_q8_0(src, dst, K), "repack_row_q8_0");
}
inline void repack_row_q5_1(const uint8_t* src, uint8_t* dst, int K) {                       // gemv.h:17
    detail::ck(qmm_repack_row_q5_1(src, dst, K), "repack_row_q5_1");
}
inline void repack_row_q5_0(const uint8_t* src, uint8_t* dst, int K) {                       // gemv.h:18
    detail::ck(qmm_repack_row_q5_0(src, dst, K), "repack_row_q5_0");
}
inline void repack_interleave8(WFmt f, const uint8_t* src, uint8_t* dst, int N, int K) {           // gemv.h:21
    detail::ck(qmm_repack_interleave8((int)f, src, dst, N, K), "repack_interleave8");
}
inline size_t wmma_il_bytes(WFmt f, int N, int K) { return qmm_wmma_il_bytes((int)f, N, K); }       // gemv.h:37
inline void repack_wmma_il(WFmt f, const uint8_t* src, uint8_t* dst, int N, int K) {               // gemv.h:38
    detail::ck(qmm_repack_wmma_il((int)f, src, dst, N, K), "repack_wmma_il");
}
inline void gemv_q8(WFmt f, const void* W, XQ8 x, float* y, int N, int K, int ncol, int tpr, int rpt, hipStream_t s) {
    detail::ck(qmm_gemv_q8((int)f, W, to_c(x), y, N, K, ncol, tpr, rpt, (void*)s), "gemv_q8");
}
inline void gemv_multi(const GemvSeg* segs, int nseg, XQ8 x, int ncol, hipStream_t s) {
    qmm_gemv_seg c[4];
    if (nseg < 1 || nseg > 4) detail::ck(QMM_ERR_SHAPE, "gemv_multi");
    for (int i = 0; i < nseg; ++i) c[i] = qmm_gemv_seg{(int32_t)segs[i].fmt, segs[i].w, segs[i].y, segs[i].N, segs[i].K};
    detail::ck(qmm_gemv_multi(c, nseg, to_c(x), ncol, (void*)s), "gemv_multi");
}
// gemv.hip:1272-1275: every format but Q5_1_SOA, K % 256 == 0, one K
inline bool gemv_wmma_ok(const GemvSeg* segs, int nseg) {
    if (nseg < 1 || nseg > 4) return false;
    for (int i = 0; i < nseg; ++i)
        if (segs[i].fmt == WFmt::Q5_1_SOA || segs[i].K % 256 != 0 || segs[i].K != segs[0].K) return false;
    return true;
}
inline void gemv_wmma(const GemvSeg* segs, int nseg, XQ8 x, int ncol, int mode, hipStream_t s) {    // gemv.h:36
    if (mode != 3) return gemv_multi(segs, nseg, x, ncol, s);
    if (nseg < 1 || nseg > 4) detail::ck(QMM_ERR_SHAPE, "gemv_wmma");
    for (int i = 0; i < nseg; ++i)   // weights repacked by repack_wmma_il: tpr 3, rpt 4 reads that layout
        detail::ck(qmm_gemv_q8((int)segs[i].fmt, segs[i].w, to_c(x), segs[i].y, segs[i].N, segs[i].K, ncol, 3, 4, (void*)s), "gemv_wmma");
}
inline void quantize_x_q8k(const float* x, XQ8K out, int ncol, int K, hipStream_t s) {                // gemv.h:34
    detail::ck(qmm_quantize_x_q8k(x, to_c(out), ncol, K, (void*)s), "quantize_x_q8k");
}
inline void gemv_wmma_q8k(const GemvSeg* segs, int nseg, XQ8K x, int ncol, int /*ks_mode*/, hipStream_t s) {   // gemv.h:35
    if (nseg < 1) detail::ck(QMM_ERR_SHAPE, "gemv_wmma_q8k");
    for (int i0 = 0; i0 < nseg; i0 += 4) {
        qmm_gemv_seg c[4];
        const int n = nseg - i0 < 4 ? nseg - i0 : 4;
        for (int i = 0; i < n; ++i) c[i] = qmm_gemv_seg{(int32_t)segs[i0 + i].fmt, segs[i0 + i].w, segs[i0 + i].y, segs[i0 + i].N, segs[i0 + i].K};
        detail::ck(qmm_gemv_q8k(c, n, to_c(x), ncol, (void*)s), "gemv_wmma_q8k");
    }
}
// split-K partials part[(c*ksplit + ks)][N] (gemv.h:55)
inline void gemv_splitk(WFmt f, const void* W, XQ8 x, float* part, int N, int K, int ksplit, int ncol, hipStream_t s) {
    detail::ck(qmm_gemv_splitk((int)f, W, to_c(x), part, N, K, ksplit, ncol, (void*)s), "gemv_splitk");
}
// hyper-connection up-projection with the silu + q8 prologue (gemv.h:52)
inline void hc_up_fused(const void* W, const float* part, int ksplit, float* y, int N, int T, hipStream_t s) {
    detail::ck(qmm_hc_up_fused(W, part, ksplit, y, N, T, (void*)s), "hc_up_fused");
}
inline void gemv_moe(WFmt f, WFmt fs, const MoeSegs& a, int nseg, const int* ids, int nexp, XQ8 x, int N, int K, int T,
                     bool xrow_te, hipStream_t s) {
    qmm_moe_segs c;
    for (int g = 0; g < 2; ++g) { c.w[g] = a.w[g]; c.shared[g] = a.shared[g]; c.y[g] = a.y[g]; }
    c.ebytes = a.ebytes;
    c.slotw = a.slotw;
    detail::ck(qmm_gemv_moe((int)f, (int)fs, &c, nseg, ids, nexp, to_c(x), N, K, T, xrow_te ? 1 : 0, (void*)s), "gemv_moe");
}
inline void gemv_q4_K_f32(const void* W, const float* x, float* y, int N, int K, int ncol, int tpr, hipStream_t s) {
    detail::ck(qmm_gemv_q4_K_f32(W, x, y, N, K, ncol, tpr, (void*)s), "gemv_q4_K_f32");
}
// grouped expert GEMM with the reference's signature and q8 activations (gemv.h:49-50): routed tiles
// then shared-expert tiles, counts from the host, y[k][N] f32
inline void moe_gemm(WFmt f, WFmt fs, const void* W, const void* Wsh, size_t ebytes, const MoeTile* tiles, int ntiles,
                     const MoeTile* stiles, int nstiles, int ct, const int* rowtab, XQ8 x, float* y, int N, int K, hipStream_t s) {
    static_assert(sizeof(MoeTile) == sizeof(qmm_moe_tile), "MoeTile layout");
    detail::ck(qmm_moe_gemm_q8((int)f, (int)fs, W, Wsh, ebytes, reinterpret_cast<const qmm_moe_tile*>(tiles), ntiles,
                               reinterpret_cast<const qmm_moe_tile*>(stiles), nstiles, ct, rowtab, to_c(x), y, N, K, (void*)s),
               "moe_gemm");
}

// ---- gemm.h -------------------------------------------------------------------------------
inline void dequant_bf16(WFmt f, const void* W, uint16_t* out, int N, int K, hipStream_t s) {
    detail::ck(qmm_dequant_bf16((int)f, W, out, N, K, (void*)s), "dequant_bf16");
}
inline void f32_to_bf16(const float* x, uint16_t* out, size_t n, hipStream_t s) {
    detail::ck(qmm_f32_to_bf16(x, out, n, (void*)s), "f32_to_bf16");
}
inline void bf16_to_f32(const uint16_t* x, float* out, size_t n, hipStream_t s) {
    detail::ck(qmm_bf16_to_f32(x, out, n, (void*)s), "bf16_to_f32");
}
inline void bf16_to_f32_seg(const uint16_t* x, int Nt, int off, int N, float* out, int M, hipStream_t s) {
    detail::ck(qmm_bf16_to_f32_seg(x, Nt, off, N, out, M, (void*)s), "bf16_to_f32_seg");
}
inline void bf16_to_f32_seg2(const uint16_t* x, const uint16_t* x2, int Nt, int off, int N, float* out, int M, hipStream_t s) {
    detail::ck(qmm_bf16_to_f32_seg2(x, x2, Nt, off, N, out, M, (void*)s), "bf16_to_f32_seg2");
}
class BlasLt {
public:
    // D[M][N] bf16 = A[M][K] bf16 . W[N][K]^T bf16, f32 accumulate (gemm.h:27)
    void gemm(const uint16_t* A, const uint16_t* W, uint16_t* D, int M, int N, int K, hipStream_t s) {
        detail::ck(qmm_gemm_bf16(A, W, D, M, N, K, (void*)s), "BlasLt::gemm");
    }
    // the same with row strides lda / ldw in elements: split-K over column halves (gemm.h:29)
    void gemm_ld(const uint16_t* A, int lda, const uint16_t* W, int ldw, uint16_t* D, int M, int N, int K, hipStream_t s) {
        detail::ck(qmm_gemm_bf16_ld(A, lda, W, ldw, D, M, N, K, (void*)s), "BlasLt::gemm_ld");
    }
    // D[M][N] f32 = A[M][K] f32 . W[N][K]^T f32: the prefill router (gemm.h:31)
    void gemm_f32(const float* A, const float* W, float* D, int M, int N, int K, hipStream_t s) {
        detail::ck(qmm_gemm_f32(A, W, D, M, N, K, (void*)s), "BlasLt::gemm_f32");
    }
};

// ---- additions with no reference counterpart (the calls the engine's prefill moves to) ----------
// D[M][N] f32 = A[M][K] bf16 . dequant(W)[N][K]^T in one launch: replaces dequant_bf16 + BlasLt::gemm
// + bf16_to_f32_seg of Qwen4Exp::lin_gemm / Qwen35::lin_multi without the bf16 weight scratch.
inline void gemm_wq(WFmt f, const void* W, const uint16_t* A, float* D, int M, int N, int K, hipStream_t s) {
    detail::ck(qmm_gemm_wq((int)f, W, A, D, M, N, K, (void*)s), "gemm_wq");
}
// quantize_x_q8 + gemv_q8 in one launch for Q4_K (x f32 [ncol][K], ncol <= 4, K <= 6144); the same y
// bit for bit, one launch fewer per decode matvec
inline void gemv_q8_f32x(WFmt f, const void* W, const float* x, float* y, int N, int K, int ncol, hipStream_t s) {
    detail::ck(qmm_gemv_q8_f32x((int)f, W, x, y, N, K, ncol, (void*)s), "gemv_q8_f32x");
}
// device sort of the routed slots (replaces the host block of qwen4exp.cpp:628-645; no host sync)
inline void moe_sort(const int* ids, int T, int nslot, int nexperts, int maxc, int* kpos, int* rowtok, MoeTile* tiles,
                     int* counts, hipStream_t s) {
    static_assert(sizeof(MoeTile) == sizeof(qmm_moe_tile), "MoeTile layout");
    detail::ck(qmm_moe_sort(ids, T, nslot, nexperts, maxc, kpos, rowtok, reinterpret_cast<qmm_moe_tile*>(tiles), counts,
                            (void*)s),
               "moe_sort");
}
// grouped expert GEMM over sorted bf16 rows; the tile count is read from counts on the device
inline void moe_gemm_bf16(WFmt f, WFmt fs, const void* W, const void* Wsh, size_t ebytes, const MoeTile* tiles,
                          const int* counts, int max_tiles, const int* rowtab, const uint16_t* A, float* D, int N, int K,
                          hipStream_t s) {
    detail::ck(qmm_moe_gemm_bf16((int)f, (int)fs, W, Wsh, ebytes, reinterpret_cast<const qmm_moe_tile*>(tiles), counts,
                                 max_tiles, rowtab, A, D, N, K, (void*)s),
               "moe_gemm_bf16");
}
// gate and up grouped GEMMs and silu in one launch: h = bf16(silu(A . Wg^T) * (A . Wu^T)), sorted rows
inline void moe_gemm_gate_up_bf16(WFmt f, WFmt fs, const void* Wg, const void* Wgsh, const void* Wu, const void* Wush,
                                  size_t ebytes, const MoeTile* tiles, const int* counts, int max_tiles, const int* rowtab,
                                  const uint16_t* A, uint16_t* H, int N, int K, hipStream_t s) {
    detail::ck(qmm_moe_gemm_gate_up_bf16((int)f, (int)fs, Wg, Wgsh, Wu, Wush, ebytes,
                                         reinterpret_cast<const qmm_moe_tile*>(tiles), counts, max_tiles, rowtab, A, H, N, K,
                                         (void*)s),
               "moe_gemm_gate_up_bf16");
}
inline void moe_silu_bf16(const float* gate, const float* up, uint16_t* h, size_t n, hipStream_t s) {
    detail::ck(qmm_moe_silu_bf16(gate, up, h, n, (void*)s), "moe_silu_bf16");
}

// ---- ops.h (the q8 / bf16 producers of the matmul inputs) -----------------------------------
inline void add_rmsnorm_quant(float* x, const float* y, const float* w, float* xn, XQ8 xq, int T, int n, float eps,
                              hipStream_t s) {                                                      // ops.h:14
    detail::ck(qmm_add_rmsnorm_quant(x, y, w, xn, to_c(xq), T, n, eps, (void*)s), "add_rmsnorm_quant");
}
inline void add_rmsnorm_bf16(float* x, const float* y, const float* w, uint16_t* xb, int T, int n, float eps,
                             hipStream_t s) {                                                       // ops.h:18
    detail::ck(qmm_add_rmsnorm_bf16(x, y, w, xb, T, n, eps, (void*)s), "add_rmsnorm_bf16");
}
inline void silu_mul_quant(const float* gate, const float* up, XQ8 xq, int n, hipStream_t s) {      // ops.h:24
    detail::ck(qmm_silu_mul_quant(gate, up, to_c(xq), n, (void*)s), "silu_mul_quant");
}
inline void silu_mul_bf16(const float* gate, const float* up, uint16_t* out, size_t n, hipStream_t s) {  // ops.h:20
    detail::ck(qmm_silu_mul_bf16(gate, up, out, n, (void*)s), "silu_mul_bf16");
}

namespace fn {
// ---- fn.h (MoE part) ----------------------------------------------------------------------
inline void moe_route(const float* logits, int* ids, float* w, int T, hipStream_t s) {
    detail::ck(qmm_moe_route(logits, ids, w, T, (void*)s), "moe_route");
}
inline void moe_gemv(WFmt fmt, WFmt shared_fmt, const MoeSegs& a, int nseg, const int* ids, int nexp, XQ8 xq, int N, int K, int T,
                     hipStream_t s) {
    // the reference's forwarder: the down projection (slot weights set) reads per-(t, e) rows
    hip::gemv_moe(fmt, shared_fmt, a, nseg, ids, nexp, xq, N, K, T, a.slotw != nullptr, s);
}
inline void f32_gemv(const float* W, const float* x, float* y, int N, int K, int T, hipStream_t s) {   // fn.h:37
    detail::ck(qmm_f32_gemv(W, x, y, N, K, T, (void*)s), "f32_gemv");
}
inline void moe_silu_quant(const float* gate, const float* up, XQ8 xq, int rows, int n, hipStream_t s) {
    detail::ck(qmm_moe_silu_quant(gate, up, to_c(xq), rows, n, (void*)s), "moe_silu_quant");
}
template <int E = 2560>
inline void moe_combine_sorted(const float* down, const float* w, const int* kpos, float* y, int T, int nexp, hipStream_t s) {
    detail::ck(qmm_moe_combine_sorted(down, w, kpos, y, T, nexp, E, (void*)s), "moe_combine_sorted");
}
}  // namespace fn

}  // namespace hip
