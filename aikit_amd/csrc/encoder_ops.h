// encoder_ops.h -- the f32 row operations between a BERT layer's linears, on the device:
// the scaled softmax of attention scores, the residual add + LayerNorm, and mean pooling
// with L2 normalisation. With the W8A8 linears and the f32 MatmulBT they let a whole
// encoder layer stay resident on the device.
//
// Each restates the reference operation for operation (f32 where it is f32, float64
// where it accumulates in float64, no contraction). Softmax and LayerNorm add their
// float64 partial sums over a wavefront as a tree rather than left to right, so their
// float64 sums can differ from the reference in the last bits, and an output in rare
// cases by one f32 ulp. Pooling keeps the reference's summation order and is exact.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "gelu_f32.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace enchip {

// The sum over the wavefront, in every lane: pairs at lane distance 1, 2, 4, 8, 16, 32
// (the lane_dpp / lane_swap moves). Each step adds two values in either order, which
// rounds the same (addition commutes), so every lane holds the same bits.
__device__ __forceinline__ double wave_sum_f64(double s) {
    auto dpp = [](double v, auto ctrl) {
        const uint64_t u = (uint64_t)__double_as_longlong(v);
        const uint32_t lo = lane_dpp<decltype(ctrl)::value>((uint32_t)u);
        const uint32_t hi = lane_dpp<decltype(ctrl)::value>((uint32_t)(u >> 32));
        return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
    };
    s += dpp(s, std::integral_constant<int, 0xB1>{});
    s += dpp(s, std::integral_constant<int, 0x4E>{});
    s += dpp(s, std::integral_constant<int, 0x141>{});
    s += dpp(s, std::integral_constant<int, 0x140>{});
    auto swap_sum = [](double v, bool wide) {
        const uint64_t u = (uint64_t)__double_as_longlong(v);
        uint32_t la, lb, ha, hb;
        if (wide) {
            lane_swap32((uint32_t)u, la, lb);
            lane_swap32((uint32_t)(u >> 32), ha, hb);
        } else {
            lane_swap16((uint32_t)u, la, lb);
            lane_swap16((uint32_t)(u >> 32), ha, hb);
        }
        return __longlong_as_double((long long)(((uint64_t)ha << 32) | la)) +
               __longlong_as_double((long long)(((uint64_t)hb << 32) | lb));
    };
    s = swap_sum(s, false);
    return swap_sum(s, true);
}

// linalg.SoftmaxRowScaledInto (linalg/exp.go:174-182 -> exp_scalar.go:84-89, 9-35), in
// place on each of `rows` rows of `cols` floats (pitch ld); one wavefront per row, the
// row held in registers (cols <= 64*CPL):
//   v = x * scale (f32); maxV = the first v, raised by every later v > maxV (so a NaN
//   first element makes maxV NaN, later NaNs are skipped); e = expF32Core(v - maxV);
//   sum = sum of (double)e; sum == 0 -> every value 1/float32(cols); else
//   x = e * float32(1 / sum).
template <int CPL>
__global__ __launch_bounds__(256) void softmax_rows_scaled(float *__restrict__ x, int64_t ld, int64_t rows, int cols,
                                                           float scale) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    float *p = x + row * ld;
    float v[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        v[j] = c < cols ? p[c] * scale : -INFINITY;
    }
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < CPL; ++j) m = v[j] > m ? v[j] : m;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    const float first = __shfl(v[0], 0, 64);
    if (first != first) m = first;  // the reference starts from element 0
    double sum = 0.0;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        const float e = c < cols ? exp_f32_core_nonpos(v[j] - m) : 0.0f;
        v[j] = e;
        sum += (double)e;
    }
    sum = wave_sum_f64(sum);
    if (sum == 0.0) {
        const float u = 1.0f / (float)cols;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = lane + 64 * j;
            if (c < cols) p[c] = u;
        }
        return;
    }
    const float inv = (float)(1.0 / sum);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        if (c < cols) p[c] = v[j] * inv;
    }
}

// h = layerNorm(h + y) per row (encoder/bert.go:352-353,363-367: the f32 residual add
// `h[i] += y[i]`, then encoder/layernorm.go:18-38), y optional; one wavefront per row,
// D <= 64*CPL:
//   mean = sum((double)v) / D; variance = sum(((double)v - mean)^2) / D;
//   invStd = 1 / sqrt(variance + eps); h = float32((((double)v - mean) * invStd) * w + b).
// VEC: D, ldh, ldy multiples of 4 and 16-byte aligned rows: each lane takes 4 consecutive
// columns per 16-byte load (CPL/4 of them), the residual input read nontemporally (it is
// read once); otherwise one column per lane per step.
template <int CPL, bool VEC>
__global__ __launch_bounds__(256) void residual_layer_norm(float *__restrict__ h, int64_t ldh,
                                                           const float *__restrict__ y, int64_t ldy, int64_t rows,
                                                           int D, const float *__restrict__ w,
                                                           const float *__restrict__ b, double eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    float *p = h + row * ldh;
    const float *q = y != nullptr ? y + row * ldy : nullptr;
    float v[CPL];
    double s = 0.0;
    // column of element j of this lane
    auto col = [&](int j) { return VEC ? 256 * (j >> 2) + 4 * lane + (j & 3) : lane + 64 * j; };
    constexpr int CH = VEC && CPL >= 4 ? CPL / 4 : 1;
    f32x4 wv[CH], bv[CH];  // VEC: the LayerNorm's weight and bias, loaded with the row
    if constexpr (VEC) {
        // every load unconditional on a clamped column (a lane past D re-reads the row's
        // last float4 and ignores it; VEC implies D % 4 == 0), so all are in flight at once
        f32x4 a[CH], r[CH];
#pragma unroll
        for (int j4 = 0; j4 < CH; ++j4) {
            const int cc = min(256 * j4 + 4 * lane, D - 4);
            a[j4] = *reinterpret_cast<const f32x4 *>(p + cc);
            wv[j4] = *reinterpret_cast<const f32x4 *>(w + cc);
            bv[j4] = *reinterpret_cast<const f32x4 *>(b + cc);
        }
        if (q != nullptr) {
#pragma unroll
            for (int j4 = 0; j4 < CH; ++j4)
                r[j4] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(q + min(256 * j4 + 4 * lane, D - 4)));
        }
#pragma unroll
        for (int j4 = 0; j4 < CH; ++j4) {
            const bool in = 256 * j4 + 4 * lane < D;
            v[4 * j4 + 0] = in ? (q != nullptr ? a[j4].x + r[j4].x : a[j4].x) : 0.0f;
            v[4 * j4 + 1] = in ? (q != nullptr ? a[j4].y + r[j4].y : a[j4].y) : 0.0f;
            v[4 * j4 + 2] = in ? (q != nullptr ? a[j4].z + r[j4].z : a[j4].z) : 0.0f;
            v[4 * j4 + 3] = in ? (q != nullptr ? a[j4].w + r[j4].w : a[j4].w) : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            if (col(j) < D) s += (double)v[j];
    } else {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = col(j);
            v[j] = 0.0f;
            if (c < D) {
                v[j] = q != nullptr ? p[c] + q[c] : p[c];
                s += (double)v[j];
            }
        }
    }
    const double mean = wave_sum_f64(s) / (double)D;
    double sq = 0.0;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        if (col(j) < D) {
            const double d = (double)v[j] - mean;
            sq += d * d;
        }
    }
    const double variance = wave_sum_f64(sq) / (double)D;
    const double inv_std = 1.0 / sqrt(variance + eps);
    if constexpr (VEC) {
#pragma unroll
        for (int j4 = 0; j4 < CPL / 4; ++j4) {
            const int c = 256 * j4 + 4 * lane;
            if (c >= D) continue;
            f32x4 o;
            o.x = (float)((((double)v[4 * j4 + 0] - mean) * inv_std) * (double)wv[j4].x + (double)bv[j4].x);
            o.y = (float)((((double)v[4 * j4 + 1] - mean) * inv_std) * (double)wv[j4].y + (double)bv[j4].y);
            o.z = (float)((((double)v[4 * j4 + 2] - mean) * inv_std) * (double)wv[j4].z + (double)bv[j4].z);
            o.w = (float)((((double)v[4 * j4 + 3] - mean) * inv_std) * (double)wv[j4].w + (double)bv[j4].w);
            *reinterpret_cast<f32x4 *>(p + c) = o;
        }
    } else {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = col(j);
            if (c < D) p[c] = (float)((((double)v[j] - mean) * inv_std) * (double)w[c] + (double)b[c]);
        }
    }
}

// residual_layer_norm<CPL, true> fused with the next linear's per-token quantization
// (linalg/quant.go:43-71 on the LayerNorm's output, as quant_rows_frag does it): each
// row of h is normalised exactly as residual_layer_norm computes it and stored, and its
// f32 values are quantized into the fragment-major code layout (frag_off; ldq a multiple
// of 64, D <= ldq <= 64*CPL, columns [D, ldq) zero) with their scale. The codes and
// scale are those quant_rows_frag gives on the stored row, and the stored row that
// residual_layer_norm gives, so the pair reads the normalised rows from HBM zero times
// instead of once. 8 rows per 512-thread block, one wavefront per row; the codes are
// gathered in LDS in line order and written as whole 128-byte lines.
template <int CPL>
__global__ __launch_bounds__(512) void residual_layer_norm_quant(float *__restrict__ h, int64_t ldh,
                                                                 const float *__restrict__ y, int64_t ldy,
                                                                 int64_t rows, int D, const float *__restrict__ w,
                                                                 const float *__restrict__ b, double eps,
                                                                 int8_t *__restrict__ q, int64_t ldq,
                                                                 float *__restrict__ scale) {
    static_assert(CPL % 4 == 0, "16-byte columns");
    constexpr int CH = CPL / 4;   // float4 per lane
    constexpr int CP = 144;       // LDS bytes per 16-code chunk: 8 rows x 16 B + 16 B against bank conflicts
    __shared__ __attribute__((aligned(16))) int8_t lds[16 * CH * CP];
    const int lane = threadIdx.x & 63, rr = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * 8, row = r0 + rr;
    const int ldq4 = (int)(ldq >> 2), D4 = D >> 2;
    auto word = [&](int k4) -> int * { return reinterpret_cast<int *>(lds + (k4 >> 2) * CP + rr * 16 + (k4 & 3) * 4); };
    if (row < rows) {
        float *p = h + row * ldh;
        const float *qy = y != nullptr ? y + row * ldy : nullptr;
        // Every load unconditional on a clamped column (a lane past D re-reads the row's
        // last float4 and ignores it; D % 4 == 0 and D >= 4, host check), the LayerNorm's
        // weight and bias included, so all are in flight at once: one round trip per row.
        f32x4 a[CH], r[CH], wv[CH], bv[CH];
#pragma unroll
        for (int j4 = 0; j4 < CH; ++j4) {
            const int cc = min(256 * j4 + 4 * lane, D - 4);
            a[j4] = *reinterpret_cast<const f32x4 *>(p + cc);
            wv[j4] = *reinterpret_cast<const f32x4 *>(w + cc);
            bv[j4] = *reinterpret_cast<const f32x4 *>(b + cc);
        }
        if (qy != nullptr) {
#pragma unroll
            for (int j4 = 0; j4 < CH; ++j4)
                r[j4] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(qy + min(256 * j4 + 4 * lane, D - 4)));
        }
        float v[CPL];
        double s = 0.0;
#pragma unroll
        for (int j4 = 0; j4 < CH; ++j4) {
            const bool in = 256 * j4 + 4 * lane < D;
            v[4 * j4 + 0] = in ? (qy != nullptr ? a[j4].x + r[j4].x : a[j4].x) : 0.0f;
            v[4 * j4 + 1] = in ? (qy != nullptr ? a[j4].y + r[j4].y : a[j4].y) : 0.0f;
            v[4 * j4 + 2] = in ? (qy != nullptr ? a[j4].z + r[j4].z : a[j4].z) : 0.0f;
            v[4 * j4 + 3] = in ? (qy != nullptr ? a[j4].w + r[j4].w : a[j4].w) : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            if (256 * (j >> 2) + 4 * lane + (j & 3) < D) s += (double)v[j];
        const double mean = wave_sum_f64(s) / (double)D;
        double sq = 0.0;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            if (256 * (j >> 2) + 4 * lane + (j & 3) < D) {
                const double d = (double)v[j] - mean;
                sq += d * d;
            }
        }
        const double variance = wave_sum_f64(sq) / (double)D;
        const double inv_std = 1.0 / sqrt(variance + eps);
        float4 o[CH];
#pragma unroll
        for (int j4 = 0; j4 < CH; ++j4) {
            const int c = 256 * j4 + 4 * lane;
            o[j4] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (c >= D) continue;
            o[j4].x = (float)((((double)v[4 * j4 + 0] - mean) * inv_std) * (double)wv[j4].x + (double)bv[j4].x);
            o[j4].y = (float)((((double)v[4 * j4 + 1] - mean) * inv_std) * (double)wv[j4].y + (double)bv[j4].y);
            o[j4].z = (float)((((double)v[4 * j4 + 2] - mean) * inv_std) * (double)wv[j4].z + (double)bv[j4].z);
            o[j4].w = (float)((((double)v[4 * j4 + 3] - mean) * inv_std) * (double)wv[j4].w + (double)bv[j4].w);
            const f32x4 ov = {o[j4].x, o[j4].y, o[j4].z, o[j4].w};
            *reinterpret_cast<f32x4 *>(p + c) = ov;
        }
        // the quantizer on the stored values (columns past D hold 0: no effect on the max)
        const float m = row_absmax<CH>(o);
        // every one of the 64*CH words is written (ldq4 <= 64*CH): past D the values are 0,
        // so their codes are 0, and no per-word branch is needed
        if (m == 0.0f) {
#pragma unroll
            for (int j4 = 0; j4 < CH; ++j4) *word(lane + 64 * j4) = 0;
            if (lane == 0) scale[row] = 0.0f;
        } else {
            const float sc = m / 127.0f;
            const float inv = 1.0f / sc;
#pragma unroll
            for (int j4 = 0; j4 < CH; ++j4) *word(lane + 64 * j4) = pack_codes(o[j4], inv);
            if (lane == 0) scale[row] = sc;
        }
    }
    __syncthreads();
    // piece p = (chunk p / 8, row p % 8): 8 consecutive threads write one whole line
    const int64_t nk32 = ldq >> 5;
    for (int pc = threadIdx.x; pc < 2 * ldq4; pc += 512) {
        const int c = pc >> 3, r2 = pc & 7;
        if (r0 + r2 < rows)
            *reinterpret_cast<int4 *>(q + frag_off(r0 + r2, 16 * (int64_t)c, nk32)) =
                *reinterpret_cast<const int4 *>(lds + c * CP + r2 * 16);
    }
}

// linalg.ExpF32 (linalg/exp.go:62-75): NaN passes through, overflow to +Inf above
// 88.72283, underflow to 0 below -87.33654, expF32Core otherwise.
__device__ __forceinline__ float exp_f32(float x) {
    if (x != x) return x;
    if (x > 88.72283f) return INFINITY;
    if (x < -87.33654f) return 0.0f;
    return exp_f32_core(x);
}

// linalg.TanhF32 (linalg/exp.go:319-337): Cephes' odd polynomial below |x| = 0.625,
// 1 - 2/(ExpF32(2|x|) + 1) above, sign restored; +-1 above |x| = 9.
__device__ __forceinline__ float tanh_f32(float x) {
    float sign = 1.0f;
    if (x < 0) {
        sign = -1.0f;
        x = -x;
    }
    if (x > 9) return sign;
    if (x < 0.625f) {
        const float z = x * x;
        float p = -5.70498872745e-3f;
        p = p * z + 2.06390887954e-2f;
        p = p * z - 5.37397155531e-2f;
        p = p * z + 1.33314422036e-1f;
        p = p * z - 3.33332819422e-1f;
        return sign * (p * z * x + x);
    }
    return sign * (1.0f - 2.0f / (exp_f32(2.0f * x) + 1.0f));
}

// x = act(x + bias) on rows x cols (pitch ld), bias optional: the cross-encoder head's
// addBias + TanhInto (encoder/crossencoder.go:229-236), TANH = 1, or addBias alone.
template <bool TANH>
__global__ __launch_bounds__(256) void bias_act_rows(float *__restrict__ x, int64_t ld, int64_t rows, int cols,
                                                     const float *__restrict__ bias) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * cols) return;
    const int64_t r = i / cols, c = i % cols;
    float v = x[r * ld + c];
    if (bias != nullptr) v = v + bias[c];
    x[r * ld + c] = TANH ? tanh_f32(v) : v;
}

// BERT's embedding rows (encoder/bert.go:299-322): for token i of each sequence,
//   h[i] = word[clampTokenID(id)] + pos[i + pos_off]   (f32 adds, column by column)
//   h[i] += type[seg]   when the model has token types (type_vocab > 0); seg = segs[i], or
//                       0 without segments, and 0 when out of [0, type_vocab)
// clampTokenID (encoder/forward.go:15-20) maps an id outside [0, vocab) to 0. One
// wavefront per row, 4 rows per block; VEC: 16-byte columns (D, ldh multiples of 4 and
// every table 16-byte aligned). The caller checked L + pos_off <= the position table's
// rows.
template <bool VEC>
__global__ __launch_bounds__(256) void embed_rows(const int32_t *__restrict__ ids, const int32_t *__restrict__ segs,
                                                  int64_t rows, int L, const float *__restrict__ word, int64_t vocab,
                                                  const float *__restrict__ pos, int pos_off,
                                                  const float *__restrict__ type, int64_t type_vocab, int D,
                                                  float *__restrict__ h, int64_t ldh) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int i = (int)(r % L);
    const int32_t id = ids[r];
    const float *wr = word + (id < 0 || id >= vocab ? 0 : (int64_t)id) * D;
    const float *pr = pos + (int64_t)(i + pos_off) * D;
    const float *tr = nullptr;
    if (type_vocab > 0) {
        int32_t seg = segs != nullptr ? segs[r] : 0;
        if (seg < 0 || seg >= type_vocab) seg = 0;
        tr = type + (int64_t)seg * D;
    }
    float *out = h + r * ldh;
    if (VEC) {
        for (int c = 4 * lane; c < D; c += 256) {
            const f32x4 a = *reinterpret_cast<const f32x4 *>(wr + c), b = *reinterpret_cast<const f32x4 *>(pr + c);
            f32x4 v = {a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w};
            if (tr != nullptr) {
                const f32x4 t = *reinterpret_cast<const f32x4 *>(tr + c);
                v.x += t.x;
                v.y += t.y;
                v.z += t.z;
                v.w += t.w;
            }
            *reinterpret_cast<f32x4 *>(out + c) = v;
        }
    } else {
        for (int c = lane; c < D; c += 64) {
            float v = wr[c] + pr[c];
            if (tr != nullptr) v += tr[c];
            out[c] = v;
        }
    }
}

// Mean pooling then L2 normalisation of each of nseq sequences of L rows
// (encoder/pooling.go:84-105 poolOne(mean), embed/pool.go:22-38 L2Normalize) in the
// reference's summation order, so the result is exact:
//   pool_mean_cols: one thread per (sequence, column); the column's float64 sum runs over
//     the rows in order; out = float32(sum * (1/L)). Grid (ceil(D/256), nseq).
//   l2_normalize_rows: one block per sequence (D <= 4096); the row is staged in LDS, one
//     thread adds the squares over the columns in order, then out = float32(out / norm),
//     or 0 when norm < 1e-12.
__global__ __launch_bounds__(256) void pool_mean_cols(const float *__restrict__ h, int64_t ldh, int L, int D,
                                                      float *__restrict__ out, int64_t ldo) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= D) return;
    const float *col = h + (int64_t)blockIdx.y * L * ldh + j;
    double acc = 0.0;
    int i = 0;
    for (; i + 8 <= L; i += 8) {  // 8 loads in flight, then the adds in row order
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = col[(int64_t)(i + u) * ldh];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += (double)x[u];
    }
    for (; i < L; ++i) acc += (double)col[(int64_t)i * ldh];
    out[blockIdx.y * ldo + j] = L > 0 ? (float)(acc * (1.0 / (double)L)) : 0.0f;
}

__global__ __launch_bounds__(256) void l2_normalize_rows(float *__restrict__ out, int64_t ldo, int D) {
    __shared__ float row[4096];
    __shared__ double norm_s;
    float *o = out + blockIdx.x * ldo;
    for (int j = threadIdx.x; j < D; j += 256) row[j] = o[j];
    __syncthreads();
    if (threadIdx.x == 0) {
        double sq = 0.0;
        for (int j = 0; j < D; ++j) sq += (double)row[j] * (double)row[j];
        norm_s = sqrt(sq);
    }
    __syncthreads();
    const double norm = norm_s;
    for (int j = threadIdx.x; j < D; j += 256) o[j] = norm < 1e-12 ? 0.0f : (float)((double)o[j] / norm);
}

}  // namespace enchip
