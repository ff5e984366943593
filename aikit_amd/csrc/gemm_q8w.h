// gemm_q8w.h -- weight-only int8 product with f32 activations,
//   C[m, n] = wscale[n] * sum_k A[m, k] * q[n, k],
// the device side of encoder.Q8Backend.MatmulBTQ8 (encoder/backend_use.go:59-83), whose CPU
// path widens the weight to f32 (f32(q) * wscale, linalg.DequantizeRowsInt8Into) and runs
// the f32 MatmulBT (encoder/linalg_q8.go:80-84). The activations are never quantized.
//
// Arithmetic. Each f32 activation is split exactly into three bf16 parts by truncation:
// b1 = the top 16 bits of a, b2 = the top 16 bits of a - b1, b3 = a - b1 - b2. a - b1 has at
// most 16 significant bits and a - b1 - b2 at most 8, so both subtractions are exact and b3
// is a bf16 value: a = b1 + b2 + b3 with no rounding, over f32's whole range (a part below
// 2^-126 may be flushed, an absolute error under 2^-126). A weight code q (any int8, -128
// included) is a bf16 value exactly. So every v_mfma_f32_32x32x16_bf16 product b_i q is exact
// and the sum over k (three MFMAs per 16-deep block) is accumulated in f32 in an order of its
// own; the channel scale multiplies the sum once at the end. The CPU rounds each widened weight and
// sums in f32 in its own order; the contract both meet is the reference's gate against a
// float64 dot product, worst |C - ref| <= 2e-4 max(|ref|, 1)
// (gpu/enccuda/backend_test.go:234-289). An infinite activation keeps b2 = b3 = 0, so its
// products are +-inf (or NaN against q = 0) as the reference's are; NaN stays NaN.
//
// Layout. The weight is the registered fragment-major int8 image (kernels.h frag_off:
// 1 KiB per 32 channels x 32 k, lane l holding channel l % 32, k 16 (l / 32) .. +15) and is
// read straight into registers, 16 bytes per lane per block. The MFMA's lane half h
// supplies depth 8h .. 8h + 7 of each 16-deep step, so step j of a 32-deep chunk takes
// bytes 8j .. 8j + 7 of the lane's 16, i.e. k = 16h + 8j + (0..7): the A operand is fed in
// the same k order, so the permutation cancels in the sum. A is row-major f32; each
// workgroup loads a BM x 32 chunk once, splits it and stores the three bf16 planes in LDS
// as MFMA operand fragments ((row block, part, step) -> 64 lanes x 16 bytes, lane-contiguous
// so every ds_read_b128 is free of bank conflicts), double-buffered with one barrier per
// chunk; the next chunk's A and weight loads are in flight during the current chunk's
// MFMAs.
//
// Tiles. 4 wavefronts in 2 x 2, each (32 TM) x (32 TN) of 32 x 32 accumulators: BM = 64 TM,
// BN = 64 TN. Rows past M re-read row M - 1 and are not stored; k past K is zero in A (the
// weight image is zero there too); channels past N read the image's zero padding and are
// not stored.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "attention_f32.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace enchip {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Bytes of one A stage in LDS: BM / 32 row blocks x 3 parts x 2 steps x 1 KiB.
__host__ __device__ constexpr int q8w_stage_bytes(int bm) { return (bm / 32) * 6 * 1024; }

// The exact split a = b1 + b2 + b3 of one f32 into the upper halves of t1, t2, t3 (the
// bf16 bit patterns are t >> 16).
__device__ __forceinline__ void q8w_split3(float a, uint32_t &t1, uint32_t &t2, uint32_t &t3) {
    const uint32_t u = __float_as_uint(a);
    t1 = u;
    float r1 = a - __uint_as_float(u & 0xFFFF0000u);
    r1 = __builtin_isinf(a) ? 0.0f : r1;  // inf - inf would be NaN
    t2 = __float_as_uint(r1);
    t3 = __float_as_uint(r1 - __uint_as_float(t2 & 0xFFFF0000u));
}

// bf16x2 word of the upper halves of lo (element 0) and hi (element 1).
__device__ __forceinline__ uint32_t q8w_pack(uint32_t lo, uint32_t hi) {
    return __builtin_amdgcn_perm(hi, lo, 0x07060302u);
}

// 4 int8 codes (bytes of w, element 0 lowest) -> 2 bf16x2 words, exactly.
__device__ __forceinline__ void q8w_widen4(uint32_t w, uint32_t &lo, uint32_t &hi) {
    const float f0 = (float)(int8_t)(w & 0xFFu), f1 = (float)(int8_t)((w >> 8) & 0xFFu);
    const float f2 = (float)(int8_t)((w >> 16) & 0xFFu), f3 = (float)(int8_t)(w >> 24);
    lo = q8w_pack(__float_as_uint(f0), __float_as_uint(f1));
    hi = q8w_pack(__float_as_uint(f2), __float_as_uint(f3));
}

// Grid: tilesM * tilesN workgroups of 256 threads (XCD-aware order), static LDS of two A
// stages. W: the fragment-major image of an Np x Kp weight (Kp a multiple of 64, Np of
// BN); ws[N]. VEC: lda % 4 == 0, K % 4 == 0 and A 16-byte aligned (16-byte loads).
template <int TM, int TN, bool VEC>
__global__ __launch_bounds__(256, 2) void gemm_q8w(const float *__restrict__ A, int64_t lda,
                                                   const int8_t *__restrict__ W, const float *__restrict__ ws,
                                                   float *__restrict__ C, int64_t ldc, int M, int N, int K, int Kp,
                                                   int tilesN) {
    constexpr int BM = 64 * TM;
    constexpr int STAGE = q8w_stage_bytes(BM);
    constexpr int EPT = BM / 8;        // A elements per thread per chunk: 8 or 16 consecutive k
    constexpr int TPR = 32 / EPT;      // threads per row
    __shared__ __attribute__((aligned(16))) char lds[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int logical = xcd_logical_tile(blockIdx.x, gridDim.x);
    const int m0 = (logical / tilesN) * BM, n0 = (logical % tilesN) * (64 * TN);
    const int wm = wave >> 1, wn = wave & 1;
    const int nk = Kp / 32;

    // ---- A loader: row lrow of the tile, k koff .. koff + EPT - 1 of each chunk
    const int lrow = tid / TPR, koff = EPT * (tid % TPR);
    const float *arow = A + (int64_t)min(m0 + lrow, M - 1) * lda;
    float av[EPT];
    auto load_a = [&](int kc) {
        const int k0 = 32 * kc + koff;
        if (32 * kc + 32 <= K) {  // uniform: the whole chunk is inside the row
            if (VEC) {
#pragma unroll
                for (int i = 0; i < EPT / 4; ++i) {
                    const f32x4 t = *reinterpret_cast<const f32x4 *>(arow + k0 + 4 * i);
                    av[4 * i] = t.x;
                    av[4 * i + 1] = t.y;
                    av[4 * i + 2] = t.z;
                    av[4 * i + 3] = t.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < EPT; ++i) av[i] = arow[k0 + i];
            }
        } else {
            // the last partial chunk (or past K): clamped reads, zero past K
#pragma unroll
            for (int i = 0; i < EPT; ++i) {
                const float x = arow[min(k0 + i, K - 1)];
                av[i] = k0 + i < K ? x : 0.0f;
            }
        }
    };
    // split into the stage's three planes: 8-element groups at k8 = koff + 8g go to lane
    // (lrow % 32) + 32 (k8 / 16), step (k8 / 8) % 2 of row block lrow / 32
    auto store_a = [&](int s) {
        char *base = lds + s * STAGE + (lrow >> 5) * 6144;
#pragma unroll
        for (int g = 0; g < EPT / 8; ++g) {
            const int k8 = koff + 8 * g, ln = (lrow & 31) + 32 * (k8 >> 4), j = (k8 >> 3) & 1;
            uint32_t t1[8], t2[8], t3[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) q8w_split3(av[8 * g + e], t1[e], t2[e], t3[e]);
            const u32x4 w1 = {q8w_pack(t1[0], t1[1]), q8w_pack(t1[2], t1[3]), q8w_pack(t1[4], t1[5]),
                              q8w_pack(t1[6], t1[7])};
            const u32x4 w2 = {q8w_pack(t2[0], t2[1]), q8w_pack(t2[2], t2[3]), q8w_pack(t2[4], t2[5]),
                              q8w_pack(t2[6], t2[7])};
            const u32x4 w3 = {q8w_pack(t3[0], t3[1]), q8w_pack(t3[2], t3[3]), q8w_pack(t3[4], t3[5]),
                              q8w_pack(t3[6], t3[7])};
            *reinterpret_cast<u32x4 *>(base + (0 * 2 + j) * 1024 + ln * 16) = w1;
            *reinterpret_cast<u32x4 *>(base + (1 * 2 + j) * 1024 + ln * 16) = w2;
            *reinterpret_cast<u32x4 *>(base + (2 * 2 + j) * 1024 + ln * 16) = w3;
        }
    };

    // ---- weight fragments: this wave's TN channel blocks, 16 bytes per lane per chunk
    const int8_t *wb[TN];
#pragma unroll
    for (int t = 0; t < TN; ++t)
        wb[t] = W + ((int64_t)((n0 >> 5) + TN * wn + t) * nk) * 1024 + lane * 16;
    u32x4 wr[TN];
    auto load_w = [&](int kc) {
#pragma unroll
        for (int t = 0; t < TN; ++t) wr[t] = *reinterpret_cast<const u32x4 *>(wb[t] + (int64_t)kc * 1024);
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][t][e] = 0.0f;

    load_a(0);
    load_w(0);
    store_a(0);
    lds_barrier();
    for (int kc = 0; kc < nk; ++kc) {
        // widen this chunk's weight codes, then put the next chunk's loads in flight
        bf16x8 wq[TN][2];
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            const uint32_t d[4] = {wr[t].x, wr[t].y, wr[t].z, wr[t].w};
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                uint32_t x[4];
                q8w_widen4(d[2 * j], x[0], x[1]);
                q8w_widen4(d[2 * j + 1], x[2], x[3]);
                wq[t][j] = __builtin_bit_cast(bf16x8, (u32x4){x[0], x[1], x[2], x[3]});
            }
        }
        if (kc + 1 < nk) {
            load_a(kc + 1);
            load_w(kc + 1);
        }
        const char *st = lds + (kc & 1) * STAGE;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const char *fb = st + (TM * wm + i) * 6144 + j * 1024 + lane * 16;
                const bf16x8 p1 = *reinterpret_cast<const bf16x8 *>(fb);
                const bf16x8 p2 = *reinterpret_cast<const bf16x8 *>(fb + 2048);
                const bf16x8 p3 = *reinterpret_cast<const bf16x8 *>(fb + 4096);
#pragma unroll
                for (int t = 0; t < TN; ++t) {
                    acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(p3, wq[t][j], acc[i][t], 0, 0, 0);
                    acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(p2, wq[t][j], acc[i][t], 0, 0, 0);
                    acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(p1, wq[t][j], acc[i][t], 0, 0, 0);
                }
            }
        if (kc + 1 < nk) store_a((kc + 1) & 1);  // that stage was last read before the previous barrier
        lds_barrier();
    }

    // ---- C = acc * wscale[n]: lane holds channel n0 + 32 (TN wn + t) + lane % 32, rows acc_row
#pragma unroll
    for (int t = 0; t < TN; ++t) {
        const int n = n0 + 32 * (TN * wn + t) + (lane & 31);
        const float s = ws[min(n, N - 1)];
        if (n >= N) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int mb = m0 + 32 * (TM * wm + i);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = mb + acc_row(r, lane);
                if (m < M) C[(int64_t)m * ldc + n] = acc[i][t][r] * s;
            }
        }
    }
}

// Small-M form: one workgroup per 32-row x (32 TN)-channel tile, its 4 wavefronts
// splitting K (wavefront w takes the 32-deep chunks w, w + 4, w + 8, ...). Each lane loads
// its own MFMA operand values straight from HBM -- lane (row m, half h) the 16 activations
// a[m, 32 kc + 16 h ..], split in registers, and its 16 weight bytes -- so there is no LDS
// and no barrier in the main loop, and a ring of Q8W_RING chunks per wavefront keeps that
// many loads in flight. The four partial sums meet in LDS and are added in a fixed order
// (wavefront 0 + 1 + 2 + 3), so the result does not depend on timing. Same arithmetic,
// edges and preconditions as gemm_q8w.
constexpr int Q8W_RING = 4;

template <int TN, bool VEC>
__global__ __launch_bounds__(256) void gemm_q8w_small(const float *__restrict__ A, int64_t lda,
                                                      const int8_t *__restrict__ W, const float *__restrict__ ws,
                                                      float *__restrict__ C, int64_t ldc, int M, int N, int K, int Kp,
                                                      int tilesN) {
    __shared__ float red[4][TN][16][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5;
    const int logical = xcd_logical_tile(blockIdx.x, gridDim.x);
    const int m0 = (logical / tilesN) * 32, n0 = (logical % tilesN) * (32 * TN);
    const int nk = Kp / 32;
    const float *arow = A + (int64_t)min(m0 + (lane & 31), M - 1) * lda + 16 * h;
    const int8_t *wb[TN];
#pragma unroll
    for (int t = 0; t < TN; ++t) wb[t] = W + ((int64_t)((n0 >> 5) + t) * nk) * 1024 + lane * 16;

    float av[Q8W_RING][16];
    u32x4 wr[Q8W_RING][TN];
    // chunk kc into ring slot d (kc < nk, uniform per wavefront)
    auto load = [&](int d, int kc) {
        const int k0 = 32 * kc + 16 * h;
        if (32 * kc + 32 <= K) {
            if (VEC) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const f32x4 x = *reinterpret_cast<const f32x4 *>(arow + 32 * kc + 4 * i);
                    av[d][4 * i] = x.x;
                    av[d][4 * i + 1] = x.y;
                    av[d][4 * i + 2] = x.z;
                    av[d][4 * i + 3] = x.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) av[d][i] = arow[32 * kc + i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float x = arow[min(32 * kc + i, K - 1 - 16 * h)];
                av[d][i] = k0 + i < K ? x : 0.0f;
            }
        }
#pragma unroll
        for (int t = 0; t < TN; ++t) wr[d][t] = *reinterpret_cast<const u32x4 *>(wb[t] + (int64_t)kc * 1024);
    };

    f32x16 acc[TN];
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[t][e] = 0.0f;

#pragma unroll
    for (int d = 0; d < Q8W_RING; ++d)
        if (wave + 4 * d < nk) load(d, wave + 4 * d);
    for (int kb = wave; kb < nk; kb += 4 * Q8W_RING) {
#pragma unroll
        for (int d = 0; d < Q8W_RING; ++d) {
            const int kc = kb + 4 * d;
            if (kc >= nk) break;  // uniform per wavefront
            // this chunk's operands out of the slot, then the slot's next chunk in flight
            bf16x8 ap[3][2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                uint32_t t1[8], t2[8], t3[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) q8w_split3(av[d][8 * j + e], t1[e], t2[e], t3[e]);
                ap[0][j] = __builtin_bit_cast(bf16x8, (u32x4){q8w_pack(t1[0], t1[1]), q8w_pack(t1[2], t1[3]),
                                                              q8w_pack(t1[4], t1[5]), q8w_pack(t1[6], t1[7])});
                ap[1][j] = __builtin_bit_cast(bf16x8, (u32x4){q8w_pack(t2[0], t2[1]), q8w_pack(t2[2], t2[3]),
                                                              q8w_pack(t2[4], t2[5]), q8w_pack(t2[6], t2[7])});
                ap[2][j] = __builtin_bit_cast(bf16x8, (u32x4){q8w_pack(t3[0], t3[1]), q8w_pack(t3[2], t3[3]),
                                                              q8w_pack(t3[4], t3[5]), q8w_pack(t3[6], t3[7])});
            }
            bf16x8 wq[TN][2];
#pragma unroll
            for (int t = 0; t < TN; ++t) {
                const uint32_t dw[4] = {wr[d][t].x, wr[d][t].y, wr[d][t].z, wr[d][t].w};
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    uint32_t x[4];
                    q8w_widen4(dw[2 * j], x[0], x[1]);
                    q8w_widen4(dw[2 * j + 1], x[2], x[3]);
                    wq[t][j] = __builtin_bit_cast(bf16x8, (u32x4){x[0], x[1], x[2], x[3]});
                }
            }
            if (kc + 4 * Q8W_RING < nk) load(d, kc + 4 * Q8W_RING);
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int t = 0; t < TN; ++t) {
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[2][j], wq[t][j], acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[1][j], wq[t][j], acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[0][j], wq[t][j], acc[t], 0, 0, 0);
                }
        }
    }

    // ---- the four partial sums, added in wavefront order; wavefront w finishes the
    // accumulator registers 4w .. 4w + 3 (rows acc_row(r, lane)) of every channel block
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wave][t][r][lane] = acc[t][r];
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TN; ++t) {
        const int n = n0 + 32 * t + (lane & 31);
        const float s = ws[min(n, N - 1)];
        if (n >= N) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 4 * wave + i;
            const float v = ((red[0][t][r][lane] + red[1][t][r][lane]) + red[2][t][r][lane]) + red[3][t][r][lane];
            const int m = m0 + acc_row(r, lane);
            if (m < M) C[(int64_t)m * ldc + n] = v * s;
        }
    }
}

}  // namespace enchip
