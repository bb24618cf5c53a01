/*
 * hipster_qmm.h -- C ABI of the MI355X (gfx950) quantized-matmul library.
 *
 * This is the drop-in boundary for the dzannotti/hipster engine's quantized matmul path.  Every
 * entry point is the `extern "C"` twin of a reference function (cited per declaration as
 * file:line in the reference repo); a header-only C++ shim (include/hipster_qmm_shim.hpp) restores
 * the reference's `namespace hip` names and signatures on top of it, so the engine's callers compile
 * unchanged.
 *
 * Conventions (same as the reference unless stated):
 *  - All buffers are device pointers owned by the caller.  The library never allocates on these
 *    calls; work runs asynchronously on `stream` (a hipStream_t passed as void*, NULL = default).
 *  - Outputs are column-per-token: y[c*N + row].
 *  - Every call returns a status (QMM_OK = 0).  Where the reference aborts on an unsupported
 *    format or silently misbehaves on a bad shape, these return an error code before launching.
 *  - Numerics: no float atomics; every output element is reduced in a fixed order that does not
 *    depend on the number of columns/tokens in the call (T-invariance, bitwise).
 */
#ifndef HIPSTER_QMM_H
#define HIPSTER_QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
enum {
    QMM_OK = 0,
    QMM_ERR_FORMAT = -1,    /* weight format not supported by this entry point */
    QMM_ERR_SHAPE = -2,     /* N/K/ncol/T out of range (e.g. K % 256 != 0) */
    QMM_ERR_NULL = -3,      /* a required pointer is NULL */
    QMM_ERR_LAUNCH = -4,    /* the HIP runtime rejected the launch */
    QMM_ERR_WORKSPACE = -5, /* workspace missing or too small */
    QMM_ERR_ARG = -6,       /* other invalid argument (mode, tpr, alignment, ...) */
    QMM_ERR_LAYOUT = -7,    /* a weight layout this library does not read (kept for the ABI: every layout
                               of the reference's call surface is read now) */
    QMM_ERR_IO = -8,        /* a GGUF file is missing, truncated, not GGUF v3 or has a tensor past its end */
    QMM_ERR_NOT_FOUND = -9, /* no tensor / key of that name in the GGUF */
    QMM_ERR_UNSUPPORTED = -10 /* an entry point of the reference's call surface that lies off the quantized
                               matmul path (declared so that the reference's callers compile) */
};

/* ---- weight formats: values of the reference's `enum class WFmt` (engine/kernels/gemv.h:13),
 * plus QMM_Q6_K, the GGUF-native 210-byte Q6_K block read without a repack (this build). ---- */
enum {
    QMM_Q4_K = 0,      /* GGUF block_q4_K, 144 B / 256 weights (engine/src/quant.h:22).  Every entry point;
                          K granule 256 */
    QMM_Q5_K = 1,      /* GGUF block_q5_K, 176 B / 256 weights (quant.h:23).  GEMVs (q8, multi, splitk, q8k),
                          gemv_moe, dequant_bf16, gemm_wq, moe_gemm_bf16, moe_gemm_q8; K granule 256 */
    QMM_IQ4_XS = 2,    /* GGUF block_iq4_xs, 136 B / 256 weights (quant.h:30).  The same entry points as
                          QMM_Q5_K; K granule 256 */
    QMM_Q6_K_SOA = 3,  /* Q6_K rows repacked [ql K/2][qh K/4][sc K/16][d K/128] (gemv.h:15).  GEMVs (q8,
                          multi; splitk and q8k with K % 512), dequant_bf16, gemm_wq (K % 512); K granule 256 */
    QMM_Q8_0_SOA = 4,  /* Q8_0 rows repacked [qs K][d K/32 x f16] (gemv.h:16).  GEMVs (q8, multi, splitk; q8k
                          with K % 256), hc_up_fused, gemv_moe (routed or shared), dequant_bf16, gemm_wq
                          (K % 128), moe_gemm_bf16, moe_gemm_q8; K granule 64 */
    QMM_Q5_1_SOA = 5,  /* Q5_1 / Q5_0 rows repacked [qs K/2][qh K/8][d K/32][m K/32] (gemv.h:17-18).  GEMVs (q8,
                          multi, splitk), gemv_moe, dequant_bf16, gemm_wq (K % 128), moe_gemm_bf16, moe_gemm_q8;
                          K granule 32 */
    QMM_Q6_K = 6       /* GGUF block_q6_K, 210 B / 256 weights (quant.h:24).  GEMVs (q8, multi) and
                          dequant_bf16; K granule 256 */
};

/* ---- POD structs, byte-compatible with the reference's (gemv.h:8,27,43,48) ---- */
/* x quantised per 32: q [ncol][K] int8, d [ncol][K/32] (scale), s [ncol][K/32] (d*sum q);
 * ds is an optional packed (d, s) float2 copy (reference: XQ8, gemv.h:8). */
typedef struct { int8_t* q; float* d; float* s; void* ds; } qmm_xq8;
/* one weight of a merged launch (reference: GemvSeg, gemv.h:27) */
typedef struct { int32_t fmt; const void* w; float* y; int32_t N, K; } qmm_gemv_seg;
/* MoE expert weights of one launch (reference: MoeSegs, gemv.h:43) */
typedef struct { const void* w[2]; const void* shared[2]; float* y[2]; size_t ebytes; const float* slotw; } qmm_moe_segs;
/* a tile of <= 16*ct expert-sorted columns (reference: MoeTile, gemv.h:48) */
typedef struct { int32_t expert, k0, ncols; } qmm_moe_tile;
/* x quantised per 256 ("Q8_K"): q [ncol][K] int8, d [K/256][16] f32, bs [K/256][16][8] int16 sums of the q
 * of each 32 (reference: XQ8K, gemv.h:33) */
typedef struct { int8_t* q; float* d; int16_t* bs; } qmm_xq8k;

/* ---- GGUF (the on-disk format of the weights; reference: engine/src/gguf.h, gguf.cpp) ---- */
/* ggml tensor types (the reference's GType numbering, gguf.h:12-17) */
enum {
    QMM_GGML_F32 = 0, QMM_GGML_F16 = 1, QMM_GGML_Q4_0 = 2, QMM_GGML_Q4_1 = 3, QMM_GGML_Q5_0 = 6, QMM_GGML_Q5_1 = 7,
    QMM_GGML_Q8_0 = 8, QMM_GGML_Q8_1 = 9, QMM_GGML_Q2_K = 10, QMM_GGML_Q3_K = 11, QMM_GGML_Q4_K = 12, QMM_GGML_Q5_K = 13,
    QMM_GGML_Q6_K = 14, QMM_GGML_Q8_K = 15, QMM_GGML_IQ4_NL = 20, QMM_GGML_IQ3_S = 21, QMM_GGML_IQ4_XS = 23,
    QMM_GGML_I8 = 24, QMM_GGML_I32 = 26, QMM_GGML_BF16 = 30
};
/* kinds of KV values (the reference's GValue kinds, gguf.h:37-41: every integer width collapses to one
 * signed and one unsigned kind, f32/f64 to FLOAT) */
enum { QMM_GGUF_KV_UINT = 0, QMM_GGUF_KV_INT = 1, QMM_GGUF_KV_FLOAT = 2, QMM_GGUF_KV_BOOL = 3, QMM_GGUF_KV_STRING = 4,
       QMM_GGUF_KV_ARRAY = 5 };
/* an opened model (one file, or every shard of a split) */
typedef struct qmm_gguf qmm_gguf;
/* one tensor (reference: GTensor, gguf.h:26-35): ne[0] is the contiguous (K) dimension; data points into
 * the read-only mapping of shard `shard`, at file offset file_off; name valid until qmm_gguf_close */
typedef struct {
    const char* name; int32_t type; uint32_t n_dims; uint64_t ne[4]; size_t nbytes; const uint8_t* data;
    int32_t shard; uint64_t file_off;
} qmm_gguf_tensor;
/* (elements, bytes) per block of a ggml type (reference: gtype_block, gguf.h:20, gguf.cpp:26-42) */
int qmm_gtype_block(int type, uint32_t* block_elems, uint32_t* block_bytes);
/* open a GGUF v3 file and map it read-only; a path <base>-0000i-of-0000N.gguf opens all N shards and joins
 * their tensor tables (reference: GGUF::GGUF / open_one, gguf.cpp:71-129); KV keys of later shards replace
 * earlier ones except split.*; data starts at the next multiple of general.alignment (default 32) */
int qmm_gguf_open(const char* path, qmm_gguf** out);
void qmm_gguf_close(qmm_gguf* g);
int64_t qmm_gguf_n_tensors(const qmm_gguf* g);
size_t qmm_gguf_mapped_bytes(const qmm_gguf* g);
int qmm_gguf_tensor_at(const qmm_gguf* g, int64_t i, qmm_gguf_tensor* out);
/* tensor by name (reference: GGUF::find / get, gguf.cpp:131-137); QMM_ERR_NOT_FOUND when absent */
int qmm_gguf_find(const qmm_gguf* g, const char* name, qmm_gguf_tensor* out);
/* KV lookups (reference: kv, kv_u32, kv_f32, kv_str, gguf.cpp:138-143); the string stays valid until close */
int qmm_gguf_kv_kind(const qmm_gguf* g, const char* key, int* kind);
int qmm_gguf_kv_u32(const qmm_gguf* g, const char* key, uint32_t* out);
int qmm_gguf_kv_f32(const qmm_gguf* g, const char* key, float* out);
int qmm_gguf_kv_str(const qmm_gguf* g, const char* key, const char** out);
int qmm_gguf_kv_array_len(const qmm_gguf* g, const char* key, uint64_t* out);
/* copy a tensor's bytes into a host buffer with pread, then drop them from the page cache (reference:
 * GGUF::read_tensor, gguf.cpp:148-156) */
int qmm_gguf_read_tensor(const qmm_gguf* g, const char* name, void* dst, size_t dst_bytes);
/* the layout the kernels read for a GGUF weight type, and its row bytes (reference: to_lin,
 * qwen4exp.cpp:34-65): Q4_K, Q5_K, IQ4_XS as stored; Q6_K -> QMM_Q6_K_SOA; Q8_0 -> QMM_Q8_0_SOA;
 * Q5_1 and Q5_0 -> QMM_Q5_1_SOA; F32, F16, BF16 -> QMM_Q8_0_SOA (requantised); others QMM_ERR_FORMAT */
int qmm_weight_format(int gtype, int K, int* wfmt, size_t* row_bytes);
/* N rows of K weights of GGUF type gtype -> that layout in dst (N * row_bytes bytes): a copy, the row
 * repacks above, or for F32/F16/BF16 the reference's quantize_row_q8_0_soa (quant.h:174-183: d =
 * f16(amax/127) with quant.h's own f32->f16 rounding, q = rint(x/d)); rows split over nthreads host threads */
int qmm_prepare_weight(int gtype, const uint8_t* src, int N, int K, uint8_t* dst, int nthreads);

/* ---- library / host helpers ---- */
const char* qmm_version(void);
const char* qmm_status_string(int status);
/* bytes of one row of K weights (reference: wfmt_row_bytes, gemv.hip:1337-1340); 0 if the format
 * is unknown or K is not a multiple of its block (256, or 32 for QMM_Q8_0_SOA / QMM_Q5_1_SOA) */
size_t qmm_wfmt_row_bytes(int fmt, int K);
/* one GGUF Q6_K row -> the SoA layout of QMM_Q6_K_SOA (reference: repack_row_q6_K, gemv.hip:1341-1350) */
int qmm_repack_row_q6_K(const uint8_t* src, uint8_t* dst, int K);
/* one GGUF Q8_0 row (34 B / 32) -> QMM_Q8_0_SOA, same size (reference: repack_row_q8_0, gemv.h:16,
 * gemv.hip:1351-1354); K % 32 == 0 */
int qmm_repack_row_q8_0(const uint8_t* src, uint8_t* dst, int K);
/* one GGUF Q5_1 row (24 B / 32) -> QMM_Q5_1_SOA, same size (reference: repack_row_q5_1, gemv.h:17,
 * gemv.hip:1458-1465); K % 32 == 0 */
int qmm_repack_row_q5_1(const uint8_t* src, uint8_t* dst, int K);
/* one GGUF Q5_0 row (22 B / 32) -> QMM_Q5_1_SOA (K*24/32 bytes) with m = f16(-16 d), exact
 * (reference: repack_row_q5_0, gemv.h:18, gemv.hip:1448-1457); K % 32 == 0 */
int qmm_repack_row_q5_0(const uint8_t* src, uint8_t* dst, int K);
/* the reference's experimental 8-row block interleave (reference: repack_interleave8, gemv.h:21,
 * gemv.hip:1442-1447): block b of row r moves to ((r/8)*8*nb + b*8 + r%8) blocks; fmt Q4_K, Q5_K or
 * IQ4_XS, N % 8 == 0, K % 256 == 0.  Host only; qmm_gemv_q8 with rpt 5 reads this layout. */
int qmm_repack_interleave8(int fmt, const uint8_t* src, uint8_t* dst, int N, int K);
/* bytes of the reference's 16-row chunk-major layout (reference: wmma_il_bytes, gemv.h:37,
 * gemv.hip:1280): ceil(N/16) * (K/256) * 16 * block bytes (Q4_K 144, Q5_K 176, IQ4_XS 136, Q6_K_SOA 210,
 * Q8_0_SOA 272); 0 for other formats or K % 256 != 0 */
size_t qmm_wmma_il_bytes(int fmt, int N, int K);
/* that layout (reference: repack_wmma_il, gemv.h:38, gemv.hip:1281-1303), byte for byte; host only
 * (qmm_gemv_q8 with rpt 4, tpr 3 reads it) */
int qmm_repack_wmma_il(int fmt, const uint8_t* src, uint8_t* dst, int N, int K);

/* ---- activation quantiser (reference: quantize_x_q8, gemv.h:10, gemv.hip:36-51,1333-1336) ----
 * per 32 values: d = amax/127, q = round-half-even(x*127/amax), s = d*sum(q); x f32 [ncol][K]. */
int qmm_quantize_x_q8(const float* x, qmm_xq8 out, int ncol, int K, void* stream);

/* ---- decode GEMV, int8 activations (reference: gemv_q8, gemv.h:25, gemv.hip:1466-1485) ----
 * y[c][n] = sum_k W[n][k] * x[c][k] for c < ncol (1..8).  fmt: every format of the call surface
 * (Q4_K, Q5_K, IQ4_XS, Q6_K, Q6_K_SOA, Q8_0_SOA, Q5_1_SOA); K % 256 == 0, or K % 64 for Q8_0_SOA and
 * K % 32 for Q5_1_SOA (32-weight blocks).  tpr/rpt are the reference's tuning knobs; this build picks its own launch shape (Q4_K,
 * Q6_K_SOA and Q8_0_SOA run on the int8 matrix cores from a few columns on, the knobs below; every
 * kernel adds a column's values in the same order, so its bits do not depend on ncol) and accepts any values,
 * as the reference does, with the reference's three routes kept: rpt 4 = qmm_gemv_multi (ncol <= 16);
 * rpt 5 = W in qmm_repack_interleave8's layout (Q4_K, Q5_K, IQ4_XS; N % 8 == 0); rpt 4 with tpr 3 = W
 * in qmm_repack_wmma_il's layout (Q4_K, Q5_K, IQ4_XS, Q6_K_SOA, Q8_0_SOA; K % 256 == 0; ncol <= 16).
 * The interleaved layouts give every row the arithmetic of its format's plain q8 GEMV (1e-5). */
int qmm_gemv_q8(int fmt, const void* W, qmm_xq8 x, float* y, int N, int K, int ncol, int tpr, int rpt, void* stream);
/* several weights sharing x (reference: gemv_multi, gemv.h:28, gemv.hip:1355-1369); up to 4
 * segments, all with the same K, any ncol.  Each run of consecutive segments of one format is one launch
 * per column pass (the grouping of the reference's gemv_wmma, gemv.hip:1313-1317): Q4_K per 16 columns
 * on the int8 matrix cores from 4 columns on (the knob below), else per 8 columns on the dot4 kernel;
 * Q5_K, IQ4_XS, Q8_0_SOA and Q5_1_SOA per 8 columns; Q6_K (both layouts) one launch per segment.
 * Results are bitwise those of qmm_gemv_q8 on each segment, and a Q4_K column's bits do not depend on
 * ncol (the matrix-core kernel adds the same values in the same order as the one-column kernel). */
int qmm_gemv_multi(const qmm_gemv_seg* segs, int nseg, qmm_xq8 x, int ncol, void* stream);
/* Tuning knob (no reference counterpart, like the reference's bench knobs): Q4_K GEMV calls with at
 * least n columns use the matrix-core kernel (default 4; n > 16 keeps every call on the dot4
 * kernels).  Returns the previous value.  Results are the same bits either way. */
int qmm_set_gemv_mfma_min_ncol(int n);
/* Tuning knob (no reference counterpart): Q6_K_SOA GEMV calls of n..8 columns (K % 512 == 0,
 * ncol * K <= 262144, x.d 16-byte aligned) use the int8 matrix-core kernel (default 3; n > 8 keeps
 * every call on the dot4 kernels).  Returns the previous value.  Results are the same bits either way. */
int qmm_set_gemv_q6k_mfma_min_ncol(int n);
/* Tuning knob (no reference counterpart): Q8_0_SOA GEMV calls of n..8 columns (ncol * K <= 40960,
 * K <= 8192, x.d 8-byte aligned) use the int8 matrix-core kernel (default 4; n > 8 keeps every call on the dot4
 * kernels).  Returns the previous value.  Results are the same bits either way. */
int qmm_set_gemv_q80_mfma_min_ncol(int n);
/* Tuning knob (no reference counterpart): the Q5_K / IQ4_XS / Q8_0_SOA / Q5_1_SOA GEMV stages x once
 * per workgroup in LDS where that measured faster (on = 1, the default; needs K % 128 == 0 and the
 * columns' x within 64 KiB) or always reads it from global memory (0).  Returns the previous value.
 * Results are the same bits either way. */
int qmm_set_gemv_fmt_xlds(int on);
/* split-K GEMV for skinny weights (reference: gemv_splitk, gemv.h:55, gemv.hip:1397-1441):
 * part[(c*ksplit + ks)*N + n] = W[n][K range ks] . x[c][K range ks], the K range of split ks being the
 * 256-weight blocks [ks*nb/ksplit, (ks+1)*nb/ksplit), nb = ceil(K/256), as the reference's; the consumer
 * sums the partials in a fixed order.  fmt: Q4_K, Q5_K, IQ4_XS, Q6_K_SOA (K % 512), Q8_0_SOA (K % 64),
 * Q5_1_SOA (K % 32); 1 <= ksplit <= nb; any ncol (8 per launch). */
int qmm_gemv_splitk(int fmt, const void* W, qmm_xq8 x, float* part, int N, int K, int ksplit, int ncol, void* stream);
/* the Flash-Next hyper-connection up-projection (reference: hc_up_fused, gemv.h:52, gemv.hip:976-1005).
 * Off the quantized matmul path (a model-specific prologue of one engine): declared so that the
 * reference's callers compile against the shim, and returns QMM_ERR_UNSUPPORTED without launching. */
int qmm_hc_up_fused(const void* W, const float* part, int ksplit, float* y, int N, int T, void* stream);
/* x -> Q8_K (reference: quantize_x_q8k, gemv.h:34, gemv.hip:686-705): per 256, d = amax/127,
 * q = round-half-even(x*127/amax) (0 when amax == 0), bs = sum of each 32 q; ncol <= 16, K % 256 == 0 */
int qmm_quantize_x_q8k(const float* x, qmm_xq8k out, int ncol, int K, void* stream);
/* GEMV on Q8_K activations (reference: gemv_wmma_q8k, gemv.h:35, gemv.hip:706-794,1259-1271): y[c][n] for each
 * segment, c < ncol <= 16; fmt Q4_K, Q5_K, IQ4_XS, Q6_K_SOA (K % 512), Q8_0_SOA; K % 256 == 0, equal K. */
int qmm_gemv_q8k(const qmm_gemv_seg* segs, int nseg, qmm_xq8k x, int ncol, void* stream);
/* qmm_quantize_x_q8 followed by qmm_gemv_q8, in one launch and bit for bit the same y: x is f32
 * [ncol][K], quantised to q8 per 32 inside the GEMV (no q8 buffer).  No reference counterpart (the
 * reference quantises in the producing kernel, e.g. add_rmsnorm_quant, ops.hip:79-98).
 * fmt Q4_K, ncol <= 4, K <= 6144, K % 256 == 0. */
int qmm_gemv_q8_f32x(int fmt, const void* W, const float* x, float* y, int N, int K, int ncol, void* stream);
/* f32-activation Q4_K GEMV: acc += (d*sc)*sum(x*q) - (dmin*m)*sum(x) per sub-block
 * (reference: gemv_q4_K_f32, gemv.h:57, gemv.hip:1177-1216,1486-1489); ncol 1..8; tpr accepted and
 * not used (any value, as the reference's). */
int qmm_gemv_q4_K_f32(const void* W, const float* x, float* y, int N, int K, int ncol, int tpr, void* stream);

/* ---- MoE decode ---- */
/* routing (reference: fn::moe_route, fn.h:43, fn.hip:157-205,301): logits [T][513] f32 -> softmax over
 * 512 experts (p = exp(l - max) / sum, the sum in the reference's order) -> top-10 by p (ties to the
 * lower id) -> weights renormalised over the 10 in selection order; slot 10 is the shared expert
 * (id -1, weight sigmoid(logits[t][512])).  ids [T][11] int32, w [T][11] f32. */
int qmm_moe_route(const float* logits, int* ids, float* w, int T, void* stream);
/* the same for nexp <= 1024 experts, row stride >= nexp+1 (logit nexp = shared gate), topk <= 16:
 * ids/w [T][topk+1].  No reference counterpart (the reference fixes 512/513/10 at compile time). */
int qmm_moe_route_n(const float* logits, int* ids, float* w, int T, int nexp, int stride, int topk, void* stream);
/* router matmul (reference: fn::f32_gemv, fn.h:37, fn.hip:251-277): y[t][n] = W[n] . x[t], W [N][K] f32,
 * x [T][K] f32, y [T][N] f32, K % 4 == 0, W and x 16-byte aligned.  The reference's arithmetic and
 * order (32 lanes per row over float4 steps 4l + 128k, its fma contraction, the xor-butterfly sum):
 * the same bits. */
int qmm_f32_gemv(const float* W, const float* x, float* y, int N, int K, int T, void* stream);
/* D[m][n] = A[m] . W[n] in f32 (reference: hip::BlasLt::gemm_f32, gemm.h:31, gemm.hip:162-186, which
 * runs hipBLASLt; the prefill router, qwen4exp.cpp:626): A [M][K], W [N][K], D [M][N] f32, K % 4 == 0,
 * A and W 16-byte aligned.  f32 matrix-core accumulation: within f32 rounding of the exact dot (the
 * reference's summation order is hipBLASLt's, unspecified). */
int qmm_gemm_f32(const float* A, const float* W, float* D, int M, int N, int K, void* stream);
/* qmm_f32_gemv of the router (nexp+1 rows: the experts and the shared gate) into logits [T][nexp+1],
 * then qmm_moe_route_n on them: the two calls of qwen4exp.cpp:346-347 in one (two launches, no host
 * work between).  No reference counterpart as one function. */
int qmm_moe_router(const float* Wr, const float* x, float* logits, int* ids, float* w, int T, int nexp, int K, int topk,
                   void* stream);
/* expert GEMV (reference: gemv_moe, gemv.h:44, gemv.hip:1075-1129,1385-1394).  Slot te = t*nexp+e
 * uses expert ids[te] (ids < 0: the shared matrices a->shared[g]); x row = te if xrow_te else t.
 * Without a->slotw: y[g][te][N] = W[g][ids[te]] . x[row] for g < nseg (gate|up share the launch);
 * each distinct expert is read once for all the slots routed to it.  With a->slotw (nseg = 1):
 * y[t][N] = sum_e slotw[te] * (W[ids[te]] . x[te]) summed in slot order (down + combine).
 * Formats as the reference's (gemv.hip:1386-1392): routed fmt Q4_K, Q5_K, IQ4_XS, Q8_0_SOA or Q5_1_SOA,
 * shared_fmt = fmt or Q8_0_SOA; K as for qmm_gemv_q8 (so the engine's K = 640 down projection runs
 * in the 32-weight formats); all-Q4_K also needs K <= 6144.  nexp <= 16; T <= 64.  a->shared[g] may be
 * NULL when shared_fmt = fmt (a caller without a shared expert): negative ids then read expert 0.  Every slot's rows
 * are bitwise the plain GEMV of its expert, except Q4_K routed experts beside a Q8_0_SOA shared expert
 * (a different, equally exact, Q4_K decode). */
int qmm_gemv_moe(int fmt, int shared_fmt, const qmm_moe_segs* a, int nseg, const int* ids, int nexp, qmm_xq8 x,
                 int N, int K, int T, int xrow_te, void* stream);
/* The whole MoE decode step in one call (no reference counterpart as one function: the reference runs
 * fn::moe_route, gemv_moe gate|up, fn::moe_silu_quant and gemv_moe down, qwen4exp.cpp:345-354).  At
 * two launches: the first routes logits [T][stride] (nexp_total experts, the shared gate at column
 * nexp_total, top-k), computes each distinct expert's gate and up rows once for the slots holding it and
 * writes h = silu(gate) * up as q8; the second is the down projection with the slot-ordered combine.
 * Outputs: ids / w [T][topk+1] as qmm_moe_route_n writes them, y [T][H] = the slot-ordered combine.  The
 * caller's workspace ws (qmm_moe_decode_ws_bytes(T, topk, F) bytes) holds the q8 of h (T*(topk+1)*F
 * bytes, then d and s per 32).  Bitwise
 * the four calls qmm_moe_route_n, qmm_gemv_moe (gate|up), qmm_moe_silu_quant, qmm_gemv_moe (down).
 * fmt Q4_K for routed and shared experts (gate, up [F][H] at Wg / Wu + e * ebytes_gu; down [H][F] at
 * Wd + e * ebytes_d; shared Sg, Su, Sd); x q8 [T][H]; T <= 8, topk + 1 <= 16, H and F multiples of 256,
 * at most 6144, and (topk + 1) * F * 5/4 <= 65536 (the down projection keeps every slot's q8 h row in
 * LDS: F <= 4608 at topk 10, F <= 3072 at topk 15).  A shape outside these limits is refused with
 * QMM_ERR_SHAPE before anything is launched or written. */
int qmm_moe_decode(int fmt, const void* Wg, const void* Wu, const void* Wd, size_t ebytes_gu, size_t ebytes_d, const void* Sg,
                   const void* Su, const void* Sd, const float* logits, int stride, int nexp_total, int topk, qmm_xq8 x, int T, int H,
                   int F, int* ids, float* w, float* ws, size_t ws_bytes, float* y, void* stream);
size_t qmm_moe_decode_ws_bytes(int T, int topk, int F);
/* qmm_moe_decode without a workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  The workspace is a static device array of qmm_moe_decode_scratch_max() bytes (2 MiB) per
 * GPU, held until the process ends; QMM_ERR_WORKSPACE when qmm_moe_decode_ws_bytes(T, topk, F) exceeds
 * it.  Allocates nothing.  Calls that overlap on one GPU (other streams or threads) share the array and
 * race: serialise them.  Same arguments, limits and bits as qmm_moe_decode. */
int qmm_moe_decode_noalloc(int fmt, const void* Wg, const void* Wu, const void* Wd, size_t ebytes_gu, size_t ebytes_d,
                           const void* Sg, const void* Su, const void* Sd, const float* logits, int stride, int nexp_total,
                           int topk, qmm_xq8 x, int T, int H, int F, int* ids, float* w, float* y, void* stream);
size_t qmm_moe_decode_scratch_max(void);
/* h = silu(gate) * up quantised per 32 into xq, rows x n (reference: fn::moe_silu_quant, fn.h:48,
 * fn.hip:206-211,305) */
int qmm_moe_silu_quant(const float* gate, const float* up, qmm_xq8 xq, int rows, int n, void* stream);
/* prefill combine (reference: fn::moe_combine_sorted, fn.h:38, fn.hip:126-132,295-297):
 * y[t][d] = sum_e w[t*nexp+e] * down[kpos[t*nexp+e]][d], slot order; the row width E is an argument
 * here (the reference fixes E = 2560 at compile time). */
int qmm_moe_combine_sorted(const float* down, const float* w, const int* kpos, float* y, int T, int nexp, int E,
                           void* stream);

/* ---- prefill GEMM ---- */
/* whole weight -> bf16 [N][K], bit-exact: quant.h arithmetic ((d*sc)*q - dmin*m, no contraction) then
 * round-to-nearest-even (reference: dequant_bf16, gemm.h:12, gemm.hip:16-76,96-107).  fmt: every
 * format of the call surface; K % 256 == 0 (K % 64 for Q8_0_SOA, K % 32 for Q5_1_SOA). */
int qmm_dequant_bf16(int fmt, const void* W, uint16_t* out, int N, int K, void* stream);
/* D[M][N] f32 = A[M][K] bf16 . W[N][K]^T with W dequantised to bf16 inside the kernel exactly as
 * qmm_dequant_bf16 (bf16 MFMA, f32 accumulate).  Replaces the reference's dequant_bf16 + BlasLt::gemm
 * pair (engine/src/qwen35.cpp:204-239, engine/src/qwen4exp.cpp:513-527) with one launch and no
 * scratch.  fmt: Q4_K, Q5_K, IQ4_XS (K % 256), Q6_K_SOA (K % 512), Q8_0_SOA, Q5_1_SOA (K % 128);
 * GGUF-native Q6_K rows take qmm_dequant_bf16 + qmm_gemm_bf16 (the engine repacks Q6_K to the SoA
 * layout at load). */
int qmm_gemm_wq(int fmt, const void* W, const uint16_t* A, float* D, int M, int N, int K, void* stream);
/* D[M][N] bf16 = A[M][K] bf16 . W[N][K]^T bf16, f32 accumulate, RNE to bf16 (reference: BlasLt::gemm,
 * gemm.h:27, gemm.hip:125-160; here an own MFMA kernel, no hipBLASLt: the fused GEMM's kernel with bf16
 * rows as its weight source when K % 128 == 0).  K % 64 == 0. */
int qmm_gemm_bf16(const uint16_t* A, const uint16_t* W, uint16_t* D, int M, int N, int K, void* stream);
/* the same with row strides (elements) for A and W (reference: BlasLt::gemm_ld, gemm.h:29,
 * gemm.hip:125-160; the split-K halves of qwen35.cpp:230-231): A[m][k] at A[m*lda + k], W[n][k] at
 * W[n*ldw + k]; D [M][N] dense.  lda, ldw >= K and multiples of 8, A and W 16-byte aligned. */
int qmm_gemm_bf16_ld(const uint16_t* A, int lda, const uint16_t* W, int ldw, uint16_t* D, int M, int N, int K, void* stream);
/* bf16 helpers (reference: gemm.h:14-20, gemm.hip:77-95) */
int qmm_f32_to_bf16(const float* x, uint16_t* out, size_t n, void* stream);
int qmm_bf16_to_f32(const uint16_t* x, float* out, size_t n, void* stream);
/* rows m < M of a [M][Nt] bf16 matrix, columns off..off+N -> f32 [M][N] (plus x2 when not NULL) */
int qmm_bf16_to_f32_seg(const uint16_t* x, int Nt, int off, int N, float* out, int M, void* stream);
int qmm_bf16_to_f32_seg2(const uint16_t* x, const uint16_t* x2, int Nt, int off, int N, float* out, int M, void* stream);

/* ---- MoE prefill ---- */
#define QMM_MOE_MAX_TILE_ROWS 128   /* rows per tile of the grouped GEMMs: qmm_moe_sort's maxc limit */
/* Device-side replacement of the host sort of engine/src/qwen4exp.cpp:628-645: slots te = t*nslot + e
 * of ids [T][nslot] (id -1 = shared expert, else 0..nexperts-1) ordered by (id, te), stable.
 * kpos[te] = sorted position, rowtok[k] = token of sorted position k, tiles = tiles of <= maxc
 * consecutive positions of one expert, routed experts first (ascending id) then the shared expert
 * (expert -1); counts[0] = routed tiles, counts[1] = shared tiles (both written on the device: no
 * host sync).  tiles needs room for ceil(T*nslot/maxc) + nexperts + 1 entries.  nexperts <= 1024;
 * 1 <= maxc <= QMM_MOE_MAX_TILE_ROWS.  Ids outside [-1, nexperts-1] are clamped into that range on
 * the device (no host check: the ids live on the device). */
int qmm_moe_sort(const int* ids, int T, int nslot, int nexperts, int maxc, int* kpos, int* rowtok, qmm_moe_tile* tiles,
                 int* counts, void* stream);
/* Grouped expert GEMM over sorted rows (reference: moe_gemm, gemv.h:49-50, gemv.hip:909-969,1377-1381,
 * with bf16 activations and the bf16 MFMA path): for tile i < counts[0] + counts[1] (read on the device)
 * and r < ncols: D[k0 + r][n] = A[rowtab ? rowtab[k0 + r] : k0 + r] . W_e[n] (f32), W_e the expert
 * matrix at W + expert * ebytes, or Wsh for expert -1, dequantised exactly to bf16.  fmt / shared_fmt:
 * Q4_K, Q5_K, IQ4_XS, Q8_0_SOA, Q5_1_SOA, independently (the reference's moe_gemm formats,
 * gemv.hip:962-968, and IQ4_XS); K as for qmm_gemv_q8.  Tiles of at most 128 rows (qmm_moe_sort with
 * maxc <= 128); max_tiles bounds the grid (the capacity of tiles). */
int qmm_moe_gemm_bf16(int fmt, int shared_fmt, const void* W, const void* Wsh, size_t ebytes, const qmm_moe_tile* tiles,
                      const int* counts, int max_tiles, const int* rowtab, const uint16_t* A, float* D, int N, int K,
                      void* stream);
/* The gate and up grouped GEMMs and the silu of the reference's prefill MoE (moe_gemm twice and
 * fn::moe_silu_quant, engine/src/qwen4exp.cpp:646-648) in one launch: for the tiles as above,
 * H[k0 + r][n] = bf16(silu(g) * u), g = A[row] . Wg_e[n], u = A[row] . Wu_e[n] (f32, each bitwise equal
 * to qmm_moe_gemm_bf16's output; silu(x) = x / (1 + exp(-x)) as in qmm_moe_silu_bf16).  N = ffn rows. */
int qmm_moe_gemm_gate_up_bf16(int fmt, int shared_fmt, const void* Wg, const void* Wgsh, const void* Wu, const void* Wush,
                              size_t ebytes, const qmm_moe_tile* tiles, const int* counts, int max_tiles, const int* rowtab,
                              const uint16_t* A, uint16_t* H, int N, int K, void* stream);
/* Grouped expert GEMM with the reference's own signature and q8 activations (reference: moe_gemm,
 * gemv.h:49-50, gemv.hip:909-969,1377-1381; called at qwen4exp.cpp:647-650): routed tiles tiles[0..ntiles)
 * in format fmt (W + expert*ebytes) and shared-expert tiles stiles[0..nstiles) in shared_fmt (Wsh), tile
 * counts from the host; for every tile column r < ncols, y[(k0 + r)*N + n] = W_e[n] . x[row] with row =
 * rowtab[k0 + r] (or k0 + r when rowtab is NULL): the reference's q8 arithmetic per row (integer dot per
 * sub-block, f32 fix-up), not bf16.  ct (the reference's 16-column tiles per block, >= 1) is accepted and
 * not needed: tiles of any width work.  fmt / shared_fmt: Q4_K, Q5_K, IQ4_XS, Q8_0_SOA, Q5_1_SOA. */
int qmm_moe_gemm_q8(int fmt, int shared_fmt, const void* W, const void* Wsh, size_t ebytes, const qmm_moe_tile* tiles, int ntiles,
                    const qmm_moe_tile* stiles, int nstiles, int ct, const int* rowtab, qmm_xq8 x, float* y, int N, int K,
                    void* stream);
/* h = bf16(silu(gate) * up), n elements (the bf16-path counterpart of fn::moe_silu_quant, fn.hip:206-211) */
int qmm_moe_silu_bf16(const float* gate, const float* up, uint16_t* h, size_t n, void* stream);

/* ---- activation producers (the kernels whose outputs the matmuls read) ---- */
/* per row t < T: if y != NULL, x += y (written back); xn = x * rs * w with rs = 1/sqrt(mean(x^2) + eps);
 * xq = q8(xn) per 32 (ds filled when given).  n % 32 == 0, n <= 16384 (reference: add_rmsnorm_quant,
 * ops.h:14, ops.hip:62-98,760-762; the reference processes only the first 6144 values of a row).
 * The sum of squares is the reference's (same per-thread fma order, same pairwise tree); rs is
 * correctly rounded where the reference uses the hardware rsqrt (within about 1 ulp). */
int qmm_add_rmsnorm_quant(float* x, const float* y, const float* w, float* xn, qmm_xq8 xq, int T, int n, float eps,
                          void* stream);
/* as qmm_add_rmsnorm_quant with xb = bf16(x * rs * w) (RNE) as the only output besides x; any n <= 16384
 * (reference: add_rmsnorm_bf16, ops.h:18, ops.hip:111-120,763) */
int qmm_add_rmsnorm_bf16(float* x, const float* y, const float* w, uint16_t* xb, int T, int n, float eps, void* stream);
/* xq = q8(silu(gate) * up) per 32, silu(v) = v / (1 + exp(-v)); n % 32 == 0 (reference: silu_mul_quant,
 * ops.h:24, ops.hip:146-151,770-772) */
int qmm_silu_mul_quant(const float* gate, const float* up, qmm_xq8 xq, int n, void* stream);
/* out = bf16(silu(gate) * up), n elements (reference: silu_mul_bf16, ops.h:20, ops.hip:131,765) */
int qmm_silu_mul_bf16(const float* gate, const float* up, uint16_t* out, size_t n, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* HIPSTER_QMM_H */
