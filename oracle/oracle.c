/*
 * oracle.c -- CPU restatement of aikit's W8A8 linear path (TEST INFRASTRUCTURE).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this
 * library, and only as the checker. It restates the Go reference
 * (github.com/townsendmerino/aikit) operation by operation. It must be compiled
 * with -ffp-contract=off and without -ffast-math: the Go amd64 compiler never
 * fuses a*b+c, evaluates float32 expressions in IEEE single precision with
 * round-to-nearest-even, and rounds untyped constants to float32 exactly once
 * (the f-suffixed literals below are the same correctly rounded float32 values).
 *
 * Pinning (how each function is checked against something other than itself):
 * see tests/test_oracle.py -- closed forms, the reference's own test vectors
 * (encoder/quant_test.go:165-201, gpu/cuda_vit_test.go:154-310,
 * linalg/quant_test.go:234-262), brute force and long-double erf/exp.
 */
#include "oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Go's int8(x) for a float64 x that the clamp left in [-127,127] is exact; a NaN
 * (from an Inf or NaN input) converts through CVTTSD2SQ to 0x8000000000000000 on
 * amd64, whose low byte is 0. */
static int8_t go_f64_to_i8(double x) {
    if (x != x) return 0;
    return (int8_t)(int)x;
}

/* linalg/quant.go:43-71 quantizeRowInt8Core. */
float orc_quantize_row(const float *row, int8_t *q, int64_t n, float zero_scale) {
    float max_abs = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float v = row[i];
        if (v < 0) v = -v;
        if (v > max_abs) max_abs = v; /* NaN never compares greater: ignored */
    }
    if (max_abs == 0) {
        memset(q, 0, (size_t)n);
        return zero_scale;
    }
    float s = max_abs / 127.0f;
    float inv = 1.0f / s;
    for (int64_t i = 0; i < n; i++) {
        /* math.Round(float64(v*inv)): the product is an f32 multiply, rounding is
         * half away from zero (C round()). */
        double x = round((double)(row[i] * inv));
        if (x > 127) x = 127;
        else if (x < -127) x = -127;
        q[i] = go_f64_to_i8(x);
    }
    return s;
}

/* linalg/quant.go:24-35 QuantizeRowsInt8 -> QuantizeRowInt8 (:83-85, zero -> 1). */
void orc_quantize_rows_weights(const float *w, int64_t rows, int64_t cols,
                               int8_t *q, float *scales) {
    for (int64_t i = 0; i < rows; i++)
        scales[i] = orc_quantize_row(w + i * cols, q + i * cols, cols, 1.0f);
}

/* linalg/quant.go:206-213 QuantizeActivationsInto -> quantizeRowInt8 (:171-173,
 * zero -> 0, the sentinel w8a8Span tests). */
void orc_quantize_activations(const float *a, int64_t M, int64_t K, int8_t *aq,
                              float *scales) {
    for (int64_t i = 0; i < M; i++)
        scales[i] = orc_quantize_row(a + i * K, aq + i * K, K, 0.0f);
}

/* linalg/quant.go:150-156 dotI8Scalar. Go's int32 arithmetic wraps; unsigned
 * arithmetic gives the same bits without C's signed-overflow UB. */
int32_t orc_dot_i8(const int8_t *a, const int8_t *b, int64_t n) {
    uint32_t s = 0;
    for (int64_t k = 0; k < n; k++) s += (uint32_t)((int32_t)a[k] * (int32_t)b[k]);
    return (int32_t)s;
}

void orc_acc_i32(const int8_t *aq, const int8_t *bq, int32_t *acc, int64_t M,
                 int64_t K, int64_t N) {
    for (int64_t i = 0; i < M; i++)
        for (int64_t j = 0; j < N; j++)
            acc[i * N + j] = orc_dot_i8(aq + i * K, bq + j * K, K);
}

/* linalg/quant.go:248-298 w8a8Span: column-outer; an all-zero activation row
 * (scale 0) writes +0 without a dot (:291-293); otherwise
 * float32(acc)*aScales[i]*bScale, left to right (:295). */
void orc_w8a8_span(const int8_t *aq, const float *ascales, const int8_t *bq,
                   const float *bscales, float *dst, int64_t M, int64_t K,
                   int64_t N, int64_t j0, int64_t j1) {
    for (int64_t j = j0; j < j1; j++) {
        const int8_t *bj = bq + j * K;
        float bscale = bscales[j];
        for (int64_t i = 0; i < M; i++) {
            if (ascales[i] == 0) {
                dst[i * N + j] = 0;
                continue;
            }
            dst[i * N + j] = (float)orc_dot_i8(aq + i * K, bj, K) * ascales[i] * bscale;
        }
    }
}

/* linalg/quant.go:192-198 MatmulBTW8A8Into, then :220-234 MatmulBTW8A8Pre. The
 * column fan-out (:230-232) is numerically inert, so the serial span stands for
 * it. */
void orc_matmul_bt_w8a8(const float *a, const int8_t *bq, const float *bscales,
                        float *dst, int64_t M, int64_t K, int64_t N) {
    int8_t *aq = (int8_t *)malloc((size_t)(M * K > 0 ? M * K : 1));
    float *as = (float *)malloc((size_t)(M > 0 ? M : 1) * sizeof(float));
    orc_quantize_activations(a, M, K, aq, as);
    orc_w8a8_span(aq, as, bq, bscales, dst, M, K, N, 0, N);
    free(aq);
    free(as);
}

/* encoder/linalg.go:130-140 addBias: a separate f32 add after the matmul. */
void orc_add_bias(float *dst, const float *bias, int64_t M, int64_t N) {
    if (!bias) return;
    for (int64_t i = 0; i < M; i++)
        for (int64_t n = 0; n < N; n++) dst[i * N + n] += bias[n];
}

static float f32_from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* Go's int32(kf) on amd64 is CVTTSS2SL: truncation, and 0x80000000 for NaN or
 * out-of-range values. */
static int32_t go_f32_to_i32(float f) {
    if (!(f >= -2147483648.0f && f < 2147483648.0f)) return INT32_MIN;
    return (int32_t)f;
}

/* linalg/exp.go:81-117 expF32Core. */
float orc_exp_f32_core(float x) {
    float z = x * 1.4426950408889634f;
    float t = z + 12582912.0f;
    float kf = t - 12582912.0f;
    int32_t k = go_f32_to_i32(kf);
    float r = x - kf * 0.693145751953125f - kf * 1.428606820309417e-06f;
    float p = 1.9875691500e-4f;
    p = p * r + 1.3981999507e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    p = p * r * r + r + 1.0f;
    int64_t e = (int64_t)k + 127; /* Go int32 add; k >= INT32_MIN so no wrap in range used */
    if (e <= 0) return 0.0f;
    if (e >= 255) return p * f32_from_bits((uint32_t)(e - 1) << 23) * 2.0f;
    return p * f32_from_bits((uint32_t)e << 23);
}

/* linalg/exp.go:62-75 ExpF32. */
float orc_exp_f32(float x) {
    if (x != x) return x;
    if (x > 88.72283f) return INFINITY;
    if (x < -87.33654f) return 0.0f;
    return orc_exp_f32_core(x);
}

/* linalg/exp.go:207-244 ErfF32: 11-term Maclaurin series below 1, A&S 7.1.26
 * with expF32Core on [1,4], saturated above 4. */
float orc_erf_f32(float x) {
    float sign = 1.0f;
    if (x < 0) {
        sign = -1.0f;
        x = -x;
    }
    if (x > 4) return sign;
    if (x < 1) {
        float z = x * x;
        float p = 1.3122532963802806e-08f;
        p = p * z - 1.4503852223150468e-07f;
        p = p * z + 1.4589169000933706e-06f;
        p = p * z - 1.3227513227513228e-05f;
        p = p * z + 1.0683760683760684e-04f;
        p = p * z - 7.5757575757575758e-04f;
        p = p * z + 4.6296296296296294e-03f;
        p = p * z - 2.3809523809523808e-02f;
        p = p * z + 1.0000000000000001e-01f;
        p = p * z - 3.3333333333333331e-01f;
        p = p * z + 1.0f;
        return sign * 1.1283791670955126f * x * p;
    }
    float t = 1.0f / (1.0f + 0.3275911f * x);
    float p = 1.061405429f;
    p = p * t - 1.453152027f;
    p = p * t + 1.421413741f;
    p = p * t - 0.284496736f;
    p = p * t + 0.254829592f;
    return sign * (1.0f - p * t * orc_exp_f32_core(-x * x));
}

/* linalg/exp.go:260-263 GELUF32 = 0.5*x*(1+ErfF32(x*invSqrt2)). */
float orc_gelu_f32(float x) {
    return 0.5f * x * (1.0f + orc_erf_f32(x * 0.7071067811865476f));
}

/* linalg/exp.go:319-337 TanhF32. */
float orc_tanh_f32(float x) {
    float sign = 1.0f;
    if (x < 0) {
        sign = -1.0f;
        x = -x;
    }
    if (x > 9) return sign;
    if (x < 0.625f) {
        float z = x * x;
        float p = -5.70498872745e-3f;
        p = p * z + 2.06390887954e-2f;
        p = p * z - 5.37397155531e-2f;
        p = p * z + 1.33314422036e-1f;
        p = p * z - 3.33332819422e-1f;
        return sign * (p * z * x + x);
    }
    return sign * (1.0f - 2.0f / (orc_exp_f32(2.0f * x) + 1.0f));
}

void orc_gelu_into(float *x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = orc_gelu_f32(x[i]);
}

void orc_tanh_into(float *x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = orc_tanh_f32(x[i]);
}

void orc_w8a8_linear(const float *a, int64_t M, int64_t K, const int8_t *bq,
                     const float *bscales, int64_t N, const float *bias, int act,
                     float *dst) {
    orc_matmul_bt_w8a8(a, bq, bscales, dst, M, K, N);
    orc_add_bias(dst, bias, M, N);
    if (act == 1) orc_gelu_into(dst, M * N);
}

/* encoder/layernorm.go:18-38 layerNorm. */
void orc_layer_norm(float *x, const float *w, const float *b, int64_t L,
                    int64_t D, double eps) {
    for (int64_t i = 0; i < L; i++) {
        float *row = x + i * D;
        double mean = 0;
        for (int64_t j = 0; j < D; j++) mean += (double)row[j];
        mean /= (double)D;
        double variance = 0;
        for (int64_t j = 0; j < D; j++) {
            double d = (double)row[j] - mean;
            variance += d * d;
        }
        variance /= (double)D;
        double inv_std = 1.0 / sqrt(variance + eps);
        for (int64_t j = 0; j < D; j++)
            row[j] = (float)((((double)row[j] - mean) * inv_std) * (double)w[j] +
                             (double)b[j]);
    }
}

/* linalg/exp_scalar.go:84-89 (scale pass) then :9-35 softmaxRowIntoRaw. */
void orc_softmax_row_scaled(float *row, int64_t n, float scale) {
    if (n == 0) return;
    for (int64_t i = 0; i < n; i++) row[i] = row[i] * scale;
    float max_v = row[0];
    for (int64_t i = 1; i < n; i++)
        if (row[i] > max_v) max_v = row[i];
    double sum = 0;
    for (int64_t i = 0; i < n; i++) {
        float e = orc_exp_f32_core(row[i] - max_v);
        row[i] = e;
        sum += (double)e;
    }
    if (sum == 0) {
        float u = 1.0f / (float)n;
        for (int64_t i = 0; i < n; i++) row[i] = u;
        return;
    }
    float inv = (float)(1.0 / sum);
    for (int64_t i = 0; i < n; i++) row[i] *= inv;
}

void orc_attention(const float *Q, const float *K, const float *V, float *ctx,
                   int64_t L, int64_t D, int64_t heads) {
    int64_t hd = D / heads;
    float scale = (float)(1.0 / sqrt((double)hd));
    float *scores = (float *)malloc((size_t)(L > 0 ? L : 1) * sizeof(float));
    for (int64_t h = 0; h < heads; h++) {
        for (int64_t i = 0; i < L; i++) {
            const float *q = Q + i * D + h * hd;
            for (int64_t j = 0; j < L; j++) {
                const float *k = K + j * D + h * hd;
                float s = 0;
                for (int64_t d = 0; d < hd; d++) s += q[d] * k[d];
                scores[j] = s;
            }
            orc_softmax_row_scaled(scores, L, scale);
            float *c = ctx + i * D + h * hd;
            for (int64_t d = 0; d < hd; d++) {
                float s = 0;
                for (int64_t j = 0; j < L; j++) s += scores[j] * V[j * D + h * hd + d];
                c[d] = s;
            }
        }
    }
    free(scores);
}

/* gpu/enccuda/backend_test.go:32-44 refMatmulBT: the float64 ground truth of
 * MatmulBT, dst[m][n] = sum_k (double)a[m][k] * (double)b[n][k], accumulated in k
 * order. The gate every f32 MatmulBT backend is held to (backend_test.go:47-86). */
void orc_matmul_bt_f64(const float *a, const float *b, int64_t M, int64_t K, int64_t N, double *dst) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            double acc = 0;
            for (int64_t k = 0; k < K; k++) acc += (double)a[m * K + k] * (double)b[n * K + k];
            dst[m * N + n] = acc;
        }
}

/* linalg/dequant_i8.go:20-43 DequantizeRowsInt8Into (scalar form dequantRowInt8Scalar,
 * :38-43): dst[r*cols + k] = float32(q[r*cols + k]) * scales[r], one f32 multiply of an
 * exact integer. The weight the CPU's weight-only path widens before its f32 MatmulBT
 * (encoder/linalg_q8.go:80-84). */
void orc_dequant_rows_i8(const int8_t *q, const float *scales, int64_t rows, int64_t cols, float *dst) {
    for (int64_t r = 0; r < rows; r++)
        for (int64_t k = 0; k < cols; k++) dst[r * cols + k] = (float)q[r * cols + k] * scales[r];
}

/* gpu/enccuda/backend_test.go:208-224 cpuQ8Ref: the float64 ground truth of the
 * weight-only product, dst[m][n] = sum_k (double)a[m][k] * ((double)q[n][k] * (double)
 * scales[n]), accumulated in k order. The gate of enccuda's MatmulBTQ8 is <= 2e-4 of
 * max(|ref|, 1) against it (backend_test.go:243-289). */
void orc_matmul_bt_q8_f64(const float *a, const int8_t *q, const float *scales, int64_t M, int64_t K, int64_t N,
                          double *dst) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            const double sc = (double)scales[n];
            double acc = 0;
            for (int64_t k = 0; k < K; k++) acc += (double)a[m * K + k] * ((double)q[n * K + k] * sc);
            dst[m * N + n] = acc;
        }
}

/* encoder/pooling.go:84-105 poolOne(mean). */
void orc_pool_mean(const float *seq, int64_t L, int64_t D, float *out) {
    if (L == 0) {
        for (int64_t j = 0; j < D; j++) out[j] = 0;
        return;
    }
    double *acc = (double *)calloc((size_t)(D > 0 ? D : 1), sizeof(double));
    for (int64_t i = 0; i < L; i++)
        for (int64_t j = 0; j < D; j++) acc[j] += (double)seq[i * D + j];
    double inv = 1.0 / (double)L;
    for (int64_t j = 0; j < D; j++) out[j] = (float)(acc[j] * inv);
    free(acc);
}

/* embed/pool.go:22-38 L2Normalize, l2NormEps = 1e-12 (embed/pool.go:7). */
void orc_l2_normalize(float *v, int64_t n) {
    double sq = 0;
    for (int64_t i = 0; i < n; i++) sq += (double)v[i] * (double)v[i];
    double norm = sqrt(sq);
    if (norm < 1e-12) {
        for (int64_t i = 0; i < n; i++) v[i] = 0;
        return;
    }
    for (int64_t i = 0; i < n; i++) v[i] = (float)((double)v[i] / norm);
}

void orc_erf_into(float *x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = orc_erf_f32(x[i]);
}

void orc_exp_into(float *x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = orc_exp_f32(x[i]);
}
