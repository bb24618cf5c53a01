/*
 * qmm_oracle.h -- CPU restatement of the dzannotti/hipster quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (hipster_amd/, include/) links, loads or
 * calls this code.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * and only as the checker (or as the timed CPU baseline), never as the thing measured or shipped.
 *
 * Every function cites the reference file:line it restates (paths relative to the reference repo).
 * How each function is pinned (golden fixtures from the reference's own quant.h, closed forms,
 * brute force) is listed in tests/test_oracle.py; a function with no such check says so here.
 *
 * Weight format ids follow the reference's WFmt enum (engine/kernels/gemv.h:13):
 *   QO_Q4_K = 0 (GGUF block, 144 B / 256 weights), QO_Q5_K = 1 (176 B / 256), QO_IQ4_XS = 2
 *   (136 B / 256), QO_Q6_K_SOA = 3 (row-SoA repack of Q6_K), QO_Q8_0_SOA = 4 (row-SoA repack of
 *   Q8_0: [qs K][d K/32 x f16]), QO_Q5_1_SOA = 5 (row-SoA repack of Q5_1 or Q5_0:
 *   [qs K/2][qh K/8][d K/32 x f16][m K/32 x f16]),
 * plus ids of this build for the GGUF-native rows the repacks start from: QO_Q6_K = 6 (210 B
 * Q6_K block), QO_Q8_0 = 8 (34 B / 32), QO_Q5_1 = 9 (24 B / 32), QO_Q5_0 = 10 (22 B / 32).
 */
#ifndef QMM_ORACLE_H
#define QMM_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { QO_Q4_K = 0, QO_Q5_K = 1, QO_IQ4_XS = 2, QO_Q6_K_SOA = 3, QO_Q8_0_SOA = 4, QO_Q5_1_SOA = 5,
       QO_Q6_K = 6, QO_Q8_0 = 8, QO_Q5_1 = 9, QO_Q5_0 = 10 };

/* ---- scalar number formats ---- */
float qo_f16_to_f32(uint16_t h);   /* engine/src/quant.h:11-17 (exact, subnormals included) */
uint16_t qo_f32_to_bf16(float f);  /* engine/kernels/gemm.hip:12 (round-to-nearest-even, no NaN case) */
uint16_t qo_f32_to_f16(float f);   /* round to nearest even, as (_Float16)x (gemv.hip:1453); no NaN case */
float qo_bf16_to_f32(uint16_t b);  /* engine/kernels/fn.hip:23 */

/* ---- weight blocks ---- */
void qo_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m); /* quant.h:37-40 */
void qo_dequant_q4_K_block(const uint8_t* blk, float* y);              /* quant.h:43-53 */
void qo_dequant_q6_K_block(const uint8_t* blk, float* y);              /* quant.h:65-80 */
void qo_repack_row_q6_K(const uint8_t* src, uint8_t* dst, int K);      /* gemv.hip:1341-1350 */
void qo_dequant_q5_K_block(const uint8_t* blk, float* y);              /* quant.h:54-64 */
extern const int8_t qo_iq4nl_levels[16];                               /* quant.h:35 */
void qo_dequant_iq4_xs_block(const uint8_t* blk, float* y);            /* quant.h:93-100 */
void qo_dequant_q8_0_block(const uint8_t* blk, float* y);              /* quant.h:81 */
void qo_dequant_q5_1_block(const uint8_t* blk, float* y);              /* quant.h:82-88 */
void qo_dequant_q5_0_block(const uint8_t* blk, float* y);              /* GGUF Q5_0 definition (see .c) */
void qo_repack_row_q8_0(const uint8_t* src, uint8_t* dst, int K);      /* gemv.hip:1351-1354 */
void qo_repack_row_q5_1(const uint8_t* src, uint8_t* dst, int K);      /* gemv.hip:1458-1465 */
void qo_repack_row_q5_0(const uint8_t* src, uint8_t* dst, int K);      /* gemv.hip:1448-1457 */
size_t qo_row_bytes(int wfmt, int K);                                  /* gemv.hip:1337-1340 */
int qo_k_granule(int wfmt);                                            /* 256, or 32 for the 32-weight block formats */
/* one row of K weights in format wfmt -> f32; returns 0, or -1 for an unknown format */
int qo_dequant_row(int wfmt, const uint8_t* row, float* y, int K);     /* quant.h:185-201 */
/* whole matrix [N][K] -> f32 or bf16 (gemm.hip:16-76 semantics: f32 dequant, then RNE to bf16) */
int qo_dequant_matrix(int wfmt, const uint8_t* W, int N, int K, float* out, int nthreads);
int qo_dequant_matrix_bf16(int wfmt, const uint8_t* W, int N, int K, uint16_t* out, int nthreads);

/* ---- activations ---- */
/* per 32: d = amax/127, q = rne(x*127/amax), s = d*sum(q)  (engine/bench/bench_gemv.cpp:17-25) */
void qo_quantize_x_q8(const float* x, int K, int8_t* q, float* d, float* s);
void qo_quantize_x_q8k(const float* x, int K, int ncol, int8_t* q, float* d, int16_t* bs);   /* gemv.hip:686-705 */
/* xr[k] = q[k] * d[k/32]  (bench_gemv.cpp:89, the "same-math" x the q8 kernels are gated against) */
void qo_q8_to_f32(const int8_t* q, const float* d, int K, float* xr);
/* silu(g)*u per element, then the q8 quantiser over rows of n (fn.hip:206-211) */
void qo_silu_mul(const float* g, const float* u, size_t n, float* h);

/* ops.hip:64-78: the pairwise tree of block_sum1024 over 1024 per-thread partials */
float qo_block_sum1024(const float* part);
/* ops.hip:79-98: per row t < T: x += y (y may be NULL), xn = (x*sc)*w with sc = 1/sqrt(ss/n + eps)
 * (correctly rounded; the reference's rsqrtf is within about 1 ulp), q8 of xn; n % 32 == 0 */
int qo_add_rmsnorm_quant(float* x, const float* y, const float* w, float* xn, int8_t* q, float* d, float* s, int T, int n,
                         float eps);
/* ops.hip:111-120: as above, xb = bf16((x*sc)*w) */
int qo_add_rmsnorm_bf16(float* x, const float* y, const float* w, uint16_t* xb, int T, int n, float eps);

/* ---- GEMV references ---- */
/* y[c][n] = sum_k w[n][k] * x[c][k] in double, mag[c][n] = sum_k |w*x| (bench_gemv.cpp:95-104) */
int qo_gemv_ref(int wfmt, const uint8_t* W, int N, int K, const float* x, int ncol,
                double* y, double* mag, int nthreads);
/* same for an explicit row list (sampled rows): y[c][i] for row rows[i] */
int qo_gemv_ref_rows(int wfmt, const uint8_t* W, int N, int K, const float* x, int ncol,
                     const int* rows, int nrows, double* y, double* mag);
/* CPU baseline: per row dequant then fp32 dot (what the reference's host path does), threaded */
int qo_gemv_f32(int wfmt, const uint8_t* W, int N, int K, const float* x, int ncol, float* y, int nthreads);

/* ---- MoE routing / sort / combine ---- */
/* softmax over nexp logits (row stride `stride`; the denominator summed per 32 experts with the
 * xor-butterfly tree, then across groups in order), top-k by the rounded probability with ties ->
 * lower id, weights renormalised over the k in selection order; slot k is the shared expert: id -1,
 * w = sigmoid(logits[nexp]) (engine/kernels/fn.hip:157-205).  ids/w are [T][k+1]. */
void qo_moe_route(const float* logits, int T, int nexp, int stride, int topk, int* ids, float* w);
/* y[t][n] = W[n] . x[t] with the reference's f32_gemv arithmetic (fn.hip:251-277): 32 lanes per row
 * over float4 steps 4l + 128k, t = fma(a.w,b.w, fma(a.z,b.z, fma(a.x,b.x, a.y*b.y))), acc += t,
 * xor-butterfly sum.  K % 4 == 0. */
int qo_f32_gemv(const float* W, const float* x, float* y, int N, int K, int T);
/* slots te = t*NE+e sorted by (expert id, te) with the shared slots (id < 0) kept in their own
 * list; tiles of <= maxc consecutive sorted positions per expert (engine/src/qwen4exp.cpp:628-641).
 * kpos[te] = sorted position, rowtok[k] = token of sorted position k, tiles as {expert,k0,ncols}.
 * The comparator orders by expert id, so the shared slots (id -1) take positions 0..T-1 and the
 * routed experts follow in ascending id.  Returns the number of routed tiles; *nstiles gets the
 * number of shared tiles, which are stored after the routed ones in `tiles` (3 ints each). */
int qo_moe_sort(const int* eid, int T, int NE, int maxc, int* kpos, int* rowtok, int* tiles, int* nstiles);

/* Decode MoE (T tokens, NE = topk+1 slots, q8 activations throughout, reference semantics of
 * gemv.hip:1075-1114 + fn.hip:206-211): gate/up per slot on q8(x[t]); h = silu(g)*u; q8(h);
 * down per slot; y[t][n] = sum_e w[t][e] * down_e[n] in slot order (double accumulate).
 * Weights: routed experts at Wg/Wu/Wd + id*ebytes, shared at Sg/Su/Sd.  Also returns the
 * per-slot gate/up outputs g,u [T*NE][F] and the down outputs dn [T*NE][H] for staged checks. */
int qo_moe_decode(int wfmt, const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd,
                  size_t ebytes_gu, size_t ebytes_d, const uint8_t* Sg, const uint8_t* Su,
                  const uint8_t* Sd, const float* x, const int* ids, const float* w, int T, int NE,
                  int H, int F, float* g, float* u, float* dn, float* y);
/* Down stage alone for given q8 h rows (staged check of the down + combine kernel). */
int qo_moe_down_q8(int wfmt, const uint8_t* Wd, size_t ebytes_d, const uint8_t* Sd,
                   const int8_t* hq, const float* hd, const int* ids, const float* w, int T,
                   int NE, int H, int F, float* dn, float* y);

/* Prefill MoE, bf16 path for the listed tokens: x bf16 [T][H]; per slot of token t:
 * g,u = bf16(W) . x (double acc), h = bf16(silu(g)*u), down = bf16(Wd) . h,
 * y[t] = sum_e w[t][e]*down_e in slot order.  Writes y for tokens toks[i] into y[i][H]. */
int qo_moe_prefill_tokens(int wfmt, const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Wd,
                          size_t ebytes_gu, size_t ebytes_d, const uint8_t* Sg, const uint8_t* Su,
                          const uint8_t* Sd, const uint16_t* xb, const int* ids, const float* w,
                          int NE, int H, int F, const int* toks, int ntok, float* y, int nthreads);

/* Dense prefill GEMM reference on sampled (m, n) pairs: D[m][n] = sum_k bf16(W[n][k]) * A[m][k]
 * (A bf16), double accumulate (gemm.hip:16-76 dequant + a bf16 GEMM with f32 compute). */
int qo_gemm_wq_ref(int wfmt, const uint8_t* W, const uint16_t* A, int M, int N, int K,
                   const int* ms, const int* ns, int npairs, double* out);

#ifdef __cplusplus
}
#endif
#endif
