/*
 * oracle.h -- CPU restatement of aikit's W8A8 linear path (TEST INFRASTRUCTURE).
 *
 * This library is the parity checker for the HIP path, never the product: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * Every function names the reference file:line it restates (module
 * github.com/townsendmerino/aikit, default amd64 build: no GOEXPERIMENT=simd,
 * no FMA contraction, SSE f32 arithmetic).
 */
#ifndef AIKIT_ORACLE_H
#define AIKIT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* linalg/quant.go:43-71 quantizeRowInt8Core. zero_scale is what an all-zero row
 * reports: 0 for activations (quantizeRowInt8, :171-173), 1 for weights
 * (QuantizeRowInt8, :83-85). Returns the row scale. */
float orc_quantize_row(const float *row, int8_t *q, int64_t n, float zero_scale);

/* linalg/quant.go:24-35 QuantizeRowsInt8 (weights; all-zero row -> scale 1). */
void orc_quantize_rows_weights(const float *w, int64_t rows, int64_t cols,
                               int8_t *q, float *scales);

/* linalg/quant.go:206-213 QuantizeActivationsInto (all-zero row -> scale 0). */
void orc_quantize_activations(const float *a, int64_t M, int64_t K, int8_t *aq,
                              float *scales);

/* linalg/quant.go:150-156 dotI8Scalar: int32 sum with Go's wrapping semantics. */
int32_t orc_dot_i8(const int8_t *a, const int8_t *b, int64_t n);

/* The int32 accumulators of linalg/quant.go:295 (dotI8 per (i,j)), [M,N]. */
void orc_acc_i32(const int8_t *aq, const int8_t *bq, int32_t *acc, int64_t M,
                 int64_t K, int64_t N);

/* linalg/quant.go:248-298 w8a8Span over columns [j0,j1). */
void orc_w8a8_span(const int8_t *aq, const float *ascales, const int8_t *bq,
                   const float *bscales, float *dst, int64_t M, int64_t K,
                   int64_t N, int64_t j0, int64_t j1);

/* linalg/quant.go:192-198 MatmulBTW8A8Into (quantize + w8a8Span, serial). */
void orc_matmul_bt_w8a8(const float *a, const int8_t *bq, const float *bscales,
                        float *dst, int64_t M, int64_t K, int64_t N);

/* encoder/linalg.go:130-140 addBias (no-op when bias is NULL). */
void orc_add_bias(float *dst, const float *bias, int64_t M, int64_t N);

/* linalg/exp.go:81-117 expF32Core, :62-75 ExpF32, :207-244 ErfF32,
 * :260-263 GELUF32, :319-337 TanhF32. */
float orc_exp_f32_core(float x);
float orc_exp_f32(float x);
float orc_erf_f32(float x);
float orc_gelu_f32(float x);
float orc_tanh_f32(float x);

/* linalg/exp_scalar.go:51-55 geluIntoRaw, in place over n elements. */
void orc_gelu_into(float *x, int64_t n);
/* linalg/exp_scalar.go:61-65 tanhIntoRaw, in place. */
void orc_tanh_into(float *x, int64_t n);
/* Elementwise ErfF32 / ExpF32 over n elements, in place (accuracy sweeps). */
void orc_erf_into(float *x, int64_t n);
void orc_exp_into(float *x, int64_t n);

/* One W8A8 linear as a BERT layer composes it (encoder/bert.go:359-361 with the
 * W8A8 primitive substituted for s.mm): MatmulBTW8A8Into, then addBias, then
 * (act == 1) gelu. act: 0 none, 1 exact-erf GELU. */
void orc_w8a8_linear(const float *a, int64_t M, int64_t K, const int8_t *bq,
                     const float *bscales, int64_t N, const float *bias, int act,
                     float *dst);

/* encoder/layernorm.go:18-38 layerNorm (f64 mean/variance), in place. */
void orc_layer_norm(float *x, const float *w, const float *b, int64_t L,
                    int64_t D, double eps);

/* linalg/exp_scalar.go:84-89 softmaxRowScaledIntoRaw + :9-35 softmaxRowIntoRaw,
 * in place on one row. */
void orc_softmax_row_scaled(float *row, int64_t n, float scale);

/* gpu/enccuda/backend_test.go:32-44 refMatmulBT: float64 dst[M,N] = a[M,K] . b[N,K]^T,
 * each dot accumulated in double in k order. */
void orc_matmul_bt_f64(const float *a, const float *b, int64_t M, int64_t K, int64_t N, double *dst);

/* encoder/attention.go:81-130 attentionCore for one sequence with mOut == L:
 * per-head softmax(Q Kᵀ * 1/sqrt(headDim)) V into ctx[L,D]. The f32 dots use
 * a plain sequential f32 sum (the reference's AVX2 dotF32 reduction order is not
 * restated: attention is outside the W8A8 path and both arms of every parity
 * test share this code). */
void orc_attention(const float *Q, const float *K, const float *V, float *ctx,
                   int64_t L, int64_t D, int64_t heads);

/* encoder/pooling.go:84-105 poolOne(mean): f64 accumulation over L rows. */
void orc_dequant_rows_i8(const int8_t *q, const float *scales, int64_t rows, int64_t cols, float *dst);
void orc_matmul_bt_q8_f64(const float *a, const int8_t *q, const float *scales, int64_t M, int64_t K, int64_t N,
                          double *dst);
void orc_pool_mean(const float *seq, int64_t L, int64_t D, float *out);

/* embed/pool.go:22-38 L2Normalize (f64 norm, eps 1e-12), in place. */
void orc_l2_normalize(float *v, int64_t n);

/* ---- cpu_baseline.c: the reference's AVX2 W8A8 CPU path (reported baseline) ---- */

/* linalg/quant_i8_amd64.go:10-21 dotI8 (AVX2 bulk + scalar tail). */
int32_t cpub_dot_i8(const int8_t *a, const int8_t *b, int64_t n);

/* linalg/quant.go:192-234 with linalg/linalg.go:208-230's column fan-out over
 * `workers` threads. aq (>= M*K) and as (>= M) are caller scratch. */
void cpub_matmul_bt_w8a8(const float *a, const int8_t *bq, const float *bs,
                         float *dst, int64_t M, int64_t K, int64_t N, int workers,
                         int8_t *aq, float *as);

/* cpub_matmul_bt_w8a8 + addBias + (act == 1) GELU chunked over workers. */
void cpub_w8a8_linear(const float *a, int64_t M, int64_t K, const int8_t *bq,
                      const float *bs, int64_t N, const float *bias, int act,
                      float *dst, int workers, int8_t *aq, float *as);

/* orc_attention's arithmetic with the heads spread over `workers` threads and loops the
 * compiler vectorises; bit-identical to orc_attention (the encode's CPU baseline). */
void cpub_attention(const float *Q, const float *K, const float *V, float *ctx, int64_t L, int64_t D,
                    int64_t heads, int workers);

#ifdef __cplusplus
}
#endif

#endif
