/*
 * cpu_baseline.c -- C restatement of aikit's Go SIMD W8A8 CPU path, timed beside
 * the GPU as the reported CPU baseline (TEST/BENCH INFRASTRUCTURE; see oracle.h).
 *
 * What it restates, and deliberately no more:
 *   - per-row activation quantization, serial over rows
 *     (linalg/quant.go:192-198 -> :206-213 -> :43-71);
 *   - w8a8Span's column-outer loop and rescale (linalg/quant.go:248-298);
 *   - dotI8 = dotI8AVX2 over the 16-multiple bulk + scalar tail
 *     (linalg/quant_i8_amd64.go:10-21): VPMOVSXBW / VPMADDWD / VPADDD with four
 *     independent accumulators, 64 bytes per step, then 16-byte steps, then a
 *     horizontal reduce (linalg/dot_amd64.s:323-387). No VNNI / AMX: the reference
 *     does not use them;
 *   - the column fan-out: serial below 1<<24 MACs or N < 2
 *     (linalg/quant.go:228-234, linalg/linalg.go:58), otherwise one thread per
 *     worker over ceil(N/workers) columns rounded up to a multiple of 8
 *     (linalg/linalg.go:208-230);
 *   - addBias serial (encoder/linalg.go:130-140) and GELU chunked by 4096 across
 *     the workers (encoder/bert.go:397-413 -> encoder/parallel.go:217-230).
 * Integer codes and int32 accumulators are bit-identical to the scalar oracle.
 */
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>

#include "oracle.h"

/* linalg/dot_amd64.s:323-387 dotI8AVX2 (n a multiple of 16). */
static int32_t dot_i8_avx2(const int8_t *a, const int8_t *b, int64_t n) {
    __m256i acc0 = _mm256_setzero_si256(), acc1 = _mm256_setzero_si256();
    __m256i acc2 = _mm256_setzero_si256(), acc3 = _mm256_setzero_si256();
    while (n >= 64) {
        acc0 = _mm256_add_epi32(acc0, _mm256_madd_epi16(
            _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(a + 0))),
            _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(b + 0)))));
        acc1 = _mm256_add_epi32(acc1, _mm256_madd_epi16(
            _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(a + 16))),
            _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(b + 16)))));
        acc2 = _mm256_add_epi32(acc2, _mm256_madd_epi16(
            _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(a + 32))),
            _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(b + 32)))));
        acc3 = _mm256_add_epi32(acc3, _mm256_madd_epi16(
            _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(a + 48))),
            _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(b + 48)))));
        a += 64;
        b += 64;
        n -= 64;
    }
    acc0 = _mm256_add_epi32(acc0, acc1);
    acc2 = _mm256_add_epi32(acc2, acc3);
    acc0 = _mm256_add_epi32(acc0, acc2);
    while (n >= 16) {
        acc0 = _mm256_add_epi32(acc0, _mm256_madd_epi16(
            _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)a)),
            _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)b))));
        a += 16;
        b += 16;
        n -= 16;
    }
    __m128i x = _mm_add_epi32(_mm256_castsi256_si128(acc0),
                              _mm256_extracti128_si256(acc0, 1));
    x = _mm_hadd_epi32(x, x);
    x = _mm_hadd_epi32(x, x);
    return _mm_cvtsi128_si32(x);
}

/* linalg/quant_i8_amd64.go:10-21 dotI8. */
int32_t cpub_dot_i8(const int8_t *a, const int8_t *b, int64_t n) {
    if (n < 16) return orc_dot_i8(a, b, n);
    int64_t n16 = n & ~(int64_t)15;
    uint32_t s = (uint32_t)dot_i8_avx2(a, b, n16);
    for (int64_t k = n16; k < n; k++) s += (uint32_t)((int32_t)a[k] * (int32_t)b[k]);
    return (int32_t)s;
}

/* linalg/quant.go:248-298 w8a8Span with the AVX2 dot. */
static void span(const int8_t *aq, const float *as, const int8_t *bq,
                 const float *bs, float *dst, int64_t M, int64_t K, int64_t N,
                 int64_t j0, int64_t j1) {
    for (int64_t j = j0; j < j1; j++) {
        const int8_t *bj = bq + j * K;
        float bscale = bs[j];
        for (int64_t i = 0; i < M; i++) {
            if (as[i] == 0) {
                dst[i * N + j] = 0;
                continue;
            }
            dst[i * N + j] = (float)cpub_dot_i8(aq + i * K, bj, K) * as[i] * bscale;
        }
    }
}

typedef struct {
    const int8_t *aq;
    const float *as;
    const int8_t *bq;
    const float *bs;
    float *dst;
    int64_t M, K, N, j0, j1;
} span_job;

static void *span_thread(void *p) {
    span_job *j = (span_job *)p;
    span(j->aq, j->as, j->bq, j->bs, j->dst, j->M, j->K, j->N, j->j0, j->j1);
    return NULL;
}

typedef struct {
    float *x;
    int64_t lo, hi;
} gelu_job;

static void *gelu_thread(void *p) {
    gelu_job *g = (gelu_job *)p;
    orc_gelu_into(g->x + g->lo, g->hi - g->lo);
    return NULL;
}

/* linalg/quant.go:192-234 MatmulBTW8A8Into + MatmulBTW8A8Pre with the
 * linalg/linalg.go:208-230 column fan-out. aq/as are caller scratch (>= M*K, M). */
void cpub_matmul_bt_w8a8(const float *a, const int8_t *bq, const float *bs,
                         float *dst, int64_t M, int64_t K, int64_t N, int workers,
                         int8_t *aq, float *as) {
    orc_quantize_activations(a, M, K, aq, as);
    if (M * N * K < ((int64_t)1 << 24) || N < 2 || workers <= 1) {
        span(aq, as, bq, bs, dst, M, K, N, 0, N);
        return;
    }
    int64_t w = workers > N ? N : workers;
    int64_t chunk = (N + w - 1) / w;
    if (chunk % 8) chunk += 8 - chunk % 8;
    int64_t nj = (N + chunk - 1) / chunk;
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nj);
    span_job *jobs = (span_job *)malloc(sizeof(span_job) * (size_t)nj);
    for (int64_t t = 0; t < nj; t++) {
        int64_t j0 = t * chunk, j1 = j0 + chunk < N ? j0 + chunk : N;
        jobs[t] = (span_job){aq, as, bq, bs, dst, M, K, N, j0, j1};
        pthread_create(&th[t], NULL, span_thread, &jobs[t]);
    }
    for (int64_t t = 0; t < nj; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}

/* One BERT linear: matmul, addBias (serial), GELU chunked by 4096 over workers. */
void cpub_w8a8_linear(const float *a, int64_t M, int64_t K, const int8_t *bq,
                      const float *bs, int64_t N, const float *bias, int act,
                      float *dst, int workers, int8_t *aq, float *as) {
    cpub_matmul_bt_w8a8(a, bq, bs, dst, M, K, N, workers, aq, as);
    orc_add_bias(dst, bias, M, N);
    if (act != 1) return;
    int64_t n = M * N, chunk = 4096, chunks = (n + chunk - 1) / chunk;
    int64_t w = workers < chunks ? workers : chunks;
    if (w <= 1) {
        orc_gelu_into(dst, n);
        return;
    }
    int64_t per = (chunks + w - 1) / w;
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)w);
    gelu_job *jobs = (gelu_job *)malloc(sizeof(gelu_job) * (size_t)w);
    int64_t used = 0;
    for (int64_t t = 0; t < w; t++) {
        int64_t lo = t * per * chunk, hi = (t + 1) * per * chunk;
        if (hi > n) hi = n;
        if (lo >= hi) break;
        jobs[t] = (gelu_job){dst, lo, hi};
        pthread_create(&th[t], NULL, gelu_thread, &jobs[t]);
        used++;
    }
    for (int64_t t = 0; t < used; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}

/* Scaled dot-product attention for the CPU baseline of the whole encode: orc_attention's
 * arithmetic (encoder/attention.go:81-121: per head, scores = Q_h K_h^T, softmaxRowScaled,
 * context = scores V_h), with the heads spread over worker threads (the reference runs its
 * per-head matmuls through the column fan-out, encoder/scratch.go:186-192 ->
 * linalg/linalg.go:208-230). Each score and each context element is summed in the same
 * order, from 0, as orc_attention sums it, with the loops arranged so the compiler can
 * vectorise across keys and across head columns: the result is bit-identical to
 * orc_attention. */
typedef struct {
    const float *Q, *K, *V;
    float *ctx;
    int64_t L, D, hd, h0, h1;
} attn_job;

static void *attn_thread(void *p) {
    attn_job *j = (attn_job *)p;
    const int64_t L = j->L, D = j->D, hd = j->hd;
    const float scale = (float)(1.0 / sqrt((double)hd));
    float *kT = (float *)malloc((size_t)(hd * L + L + hd + 1) * sizeof(float));
    float *sc = kT + hd * L, *c = sc + L;
    for (int64_t h = j->h0; h < j->h1; h++) {
        for (int64_t jj = 0; jj < L; jj++)
            for (int64_t d = 0; d < hd; d++) kT[d * L + jj] = j->K[jj * D + h * hd + d];
        for (int64_t i = 0; i < L; i++) {
            const float *q = j->Q + i * D + h * hd;
            for (int64_t jj = 0; jj < L; jj++) sc[jj] = 0;
            for (int64_t d = 0; d < hd; d++) {
                const float qd = q[d], *kr = kT + d * L;
                for (int64_t jj = 0; jj < L; jj++) sc[jj] += qd * kr[jj];
            }
            orc_softmax_row_scaled(sc, L, scale);
            for (int64_t d = 0; d < hd; d++) c[d] = 0;
            for (int64_t jj = 0; jj < L; jj++) {
                const float pj = sc[jj], *vr = j->V + jj * D + h * hd;
                for (int64_t d = 0; d < hd; d++) c[d] += pj * vr[d];
            }
            float *o = j->ctx + i * D + h * hd;
            for (int64_t d = 0; d < hd; d++) o[d] = c[d];
        }
    }
    free(kT);
    return NULL;
}

void cpub_attention(const float *Q, const float *K, const float *V, float *ctx, int64_t L, int64_t D,
                    int64_t heads, int workers) {
    if (heads <= 0 || L <= 0) return;
    int64_t w = workers < 1 ? 1 : (workers > heads ? heads : workers);
    int64_t per = (heads + w - 1) / w;
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)w);
    attn_job *jobs = (attn_job *)malloc(sizeof(attn_job) * (size_t)w);
    int64_t used = 0;
    for (int64_t t = 0; t < w; t++) {
        int64_t h0 = t * per, h1 = h0 + per < heads ? h0 + per : heads;
        if (h0 >= h1) break;
        jobs[t] = (attn_job){Q, K, V, ctx, L, D, D / heads, h0, h1};
        pthread_create(&th[t], NULL, attn_thread, &jobs[t]);
        used++;
    }
    for (int64_t t = 0; t < used; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}
