// gemm_f32.h -- f32 C = A . B^T on the gfx950 f32 MFMA: the device side of
// encoder.Backend.MatmulBT (encoder/backend.go:19-28), used by attention for
// QK^T = qH . kH^T and scores . V = scores . (vHT)^T (encoder/attention.go:108,111).
//
// Batched and strided over two levels: problem (y, z) of a launch reads
// A + y*sa + z*sa2, B + y*sb + z*sb2 and writes C + y*sc + z*sc2, so one launch covers
// every (head, sequence) of a layer, each head read in place from the interleaved
// [L, D] activations (lda = D or 3D) with no extraction copy.
// B is [N, K] rows (MatmulBT's b, BKN = false) or [K, N] rows (BKN = true: V itself
// for scores . V, element (n, k) at B[k*ldb + n], so no transpose copy either).
//
// Each wavefront computes a 64 x 64 tile of C as 2 x 2 accumulators of
// v_mfma_f32_32x32x2_f32. In MFMA step s of a 16-deep K block, lane l supplies
// row / column l % 32 at k = k0 + 8*(l/32) + s for both operands, so every lane reads
// 8 consecutive k of its row per block (two 16-byte loads when the rows are 16-byte
// aligned, VEC). The sum is the exact dot product's terms, each product rounded once
// and added in f32 in a different order than the CPU's; the contract is the
// reference's gate against a float64 dot product (gpu/enccuda/backend_test.go:47-86).
// Two forms with the same k order (so the same bits): gemm_f32_bt_lds stages 16-deep K
// chunks of the block's operands through LDS with coalesced 16-byte loads (the one used
// whenever alignment allows), gemm_f32_bt loads each lane's operands straight into
// registers (any pitch or alignment; latency-bound, about 1.4x slower). Elements past K
// count as zero; rows past M and columns past N are clamped on load and never stored.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace enchip {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int F32_KB = 16;  // K block per pipeline stage

// 8 consecutive k (k0 .. k0+7) of one row, raw: addresses past K are clamped into the
// row (kmask zeroes those values where they are used). VEC: the row start and k0 are
// 16-byte aligned and K % 4 == 0, so each float4 is either all in range or all past K.
template <bool VEC>
__device__ __forceinline__ void load8_row(const float *__restrict__ row, int k0, int K, float (&v)[8]) {
    if (VEC) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const f32x4 t = *reinterpret_cast<const f32x4 *>(row + min(k0 + 4 * j, K - 4));
            v[4 * j + 0] = t.x;
            v[4 * j + 1] = t.y;
            v[4 * j + 2] = t.z;
            v[4 * j + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = row[min(k0 + j, K - 1)];
    }
}

// 8 consecutive k of column n of a [K, N] matrix (pitch ldb), raw as load8_row.
__device__ __forceinline__ void load8_col(const float *__restrict__ col, int64_t ldb, int k0, int K, float (&v)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = col[(int64_t)min(k0 + j, K - 1) * ldb];
}

// Zero the values of k >= K (k0 .. k0+7 held in v).
__device__ __forceinline__ void kmask(float (&v)[8], int k0, int K) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = k0 + j < K ? v[j] : 0.0f;
}

// Batch strides of one level (in floats).
struct F32Strides {
    int64_t a, b, c;
};

// WM x WN wavefronts per block (block tile 64*WM x 64*WN); grid (tilesM*tilesN, inner
// batch, outer batch). KM: K is not a multiple of 16, so the last block's k >= K are zeroed.
template <int WM, int WN, bool BKN, bool VEC, bool KM>
__global__ __launch_bounds__(64 * WM * WN) void gemm_f32_bt(
    const float *__restrict__ A, int64_t lda, const float *__restrict__ B, int64_t ldb, float *__restrict__ C,
    int64_t ldc, F32Strides s1, F32Strides s2, int M, int N, int K, int tilesN) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t y = blockIdx.y, z = blockIdx.z;
    A += y * s1.a + z * s2.a;
    B += y * s1.b + z * s2.b;
    C += y * s1.c + z * s2.c;
    const int tm = blockIdx.x / tilesN, tn = blockIdx.x % tilesN;
    const int m0 = tm * 64 * WM + (wave / WN) * 64, n0 = tn * 64 * WN + (wave % WN) * 64;
    if (m0 >= M || n0 >= N) return;  // no barriers: a wavefront with no rows or columns just leaves
    const int r = lane & 31, kh = 8 * (lane >> 5);

    const float *pa[2], *pb[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        pa[t] = A + (int64_t)min(m0 + 32 * t + r, M - 1) * lda;
        const int n = min(n0 + 32 * t + r, N - 1);
        pb[t] = BKN ? B + n : B + (int64_t)n * ldb;
    }
    auto load = [&](int k0, float (&a)[2][8], float (&b)[2][8]) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            load8_row<VEC>(pa[t], k0 + kh, K, a[t]);
            if (BKN) load8_col(pb[t], ldb, k0 + kh, K, b[t]);
            else load8_row<VEC>(pb[t], k0 + kh, K, b[t]);
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // The next K block's loads are issued before the current block's 32 MFMAs (2048
    // cycles). Loads past K stay in bounds (clamped addresses); KM zeroes their values
    // before use (the last block is then partial). An explicit two-set ping-pong with
    // scheduling barriers measured 10-45% slower on MI355X.
    float a[2][8], b[2][8], na[2][8], nb[2][8];
    load(0, a, b);
    for (int k0 = 0; k0 < K; k0 += F32_KB) {
        load(k0 + F32_KB, na, nb);
        if (KM) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                kmask(a[t], k0 + kh, K);
                kmask(b[t], k0 + kh, K);
            }
        }
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                a[t][s] = na[t][s];
                b[t][s] = nb[t][s];
            }
    }

    // accumulator element e of lane l: row 8*(e/4) + 4*(l/32) + e%4, column l%32
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + 32 * j + r;
            if (col >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row < M) C[(int64_t)row * ldc + col] = acc[i][j][e];
            }
        }
}

// LDS-staged form (the one used whenever the operands allow 16-byte loads: K, pitches
// and strides multiples of 4, 16-byte aligned bases, and N % 4 == 0 for BKN). The block's
// (64*WM) x (64*WN) tile takes K in 16-deep chunks through a double LDS buffer: every
// thread loads whole 16-byte pieces of operand rows (coalesced, 4 lanes per 64-byte row
// chunk), the next chunk's loads are in flight during the current chunk's 32 MFMAs per
// wavefront, and one barrier per chunk hands the buffers over. The MFMA operands come
// from LDS in the same k order as gemm_f32_bt (lane half h takes k = 8h + s), so the two
// forms give the same bits. A rows and B columns past M / N are clamped on load, k >= K
// is zeroed when stored to LDS. Measured on MI355X at one config-4 layer's attention
// (768 problems per launch): QK^T 515 -> 360 us, scores . V 392 -> 280 us.
template <int WM, int WN, bool BKN>
__global__ __launch_bounds__(256) void gemm_f32_bt_lds(
    const float *__restrict__ A, int64_t lda, const float *__restrict__ B, int64_t ldb, float *__restrict__ C,
    int64_t ldc, F32Strides s1, F32Strides s2, int M, int N, int K, int tilesN) {
    constexpr int BM = 64 * WM, BN = 64 * WN, BK = F32_KB, KL = BK / 2;
    constexpr int AP = BK + 4;                        // LDS pitch of a [row][k] tile (floats)
    constexpr int BP = BN + 4;                        // LDS pitch of a [k][n] tile (floats)
    constexpr int A_SZ = BM * AP, B_SZ = BKN ? BK * BP : BN * AP;
    constexpr int AV = BM * (BK / 4) / 256;           // float4 per thread for A
    constexpr int BV = (BKN ? BK * (BN / 4) : BN * (BK / 4)) / 256;
    static_assert(AV >= 1 && BV >= 1, "tile too small");
    __shared__ __attribute__((aligned(16))) float lds[2][A_SZ + B_SZ];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t y = blockIdx.y, z = blockIdx.z;
    A += y * s1.a + z * s2.a;
    B += y * s1.b + z * s2.b;
    C += y * s1.c + z * s2.c;
    const int tm = blockIdx.x / tilesN, tn = blockIdx.x % tilesN;
    const int bm0 = tm * BM, bn0 = tn * BN;
    const int wm0 = (wave / WN) * 64, wn0 = (wave % WN) * 64;  // wave tile within the block

    // global source of each staged float4 (k offset added per chunk)
    const float *ga[AV];
    int ak[AV], arow_l[AV];
#pragma unroll
    for (int i = 0; i < AV; ++i) {
        const int idx = tid + 256 * i, row = idx / (BK / 4), c4 = idx % (BK / 4);
        ga[i] = A + (int64_t)min(bm0 + row, M - 1) * lda;
        ak[i] = 4 * c4;
        arow_l[i] = row;
    }
    const float *gb[BV];
    int bk_[BV], brow_l[BV];
#pragma unroll
    for (int i = 0; i < BV; ++i) {
        const int idx = tid + 256 * i;
        if (BKN) {
            const int kr = idx / (BN / 4), c4 = idx % (BN / 4);
            gb[i] = B + min(bn0 + 4 * c4, N - 4);  // + k*ldb per element row
            bk_[i] = kr;
            brow_l[i] = 4 * c4;
        } else {
            const int row = idx / (BK / 4), c4 = idx % (BK / 4);
            gb[i] = B + (int64_t)min(bn0 + row, N - 1) * ldb;
            bk_[i] = 4 * c4;
            brow_l[i] = row;
        }
    }
    f32x4 ra[AV], rb[BV];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < AV; ++i) ra[i] = *reinterpret_cast<const f32x4 *>(ga[i] + min(k0 + ak[i], K - 4));
#pragma unroll
        for (int i = 0; i < BV; ++i) {
            if (BKN) rb[i] = *reinterpret_cast<const f32x4 *>(gb[i] + (int64_t)min(k0 + bk_[i], K - 1) * ldb);
            else rb[i] = *reinterpret_cast<const f32x4 *>(gb[i] + min(k0 + bk_[i], K - 4));
        }
    };
    auto lstore = [&](int k0, float *buf) {
#pragma unroll
        for (int i = 0; i < AV; ++i) {
            f32x4 v = ra[i];
            if (k0 + ak[i] >= K) v = f32x4{0.f, 0.f, 0.f, 0.f};
            *reinterpret_cast<f32x4 *>(buf + arow_l[i] * AP + ak[i]) = v;
        }
#pragma unroll
        for (int i = 0; i < BV; ++i) {
            f32x4 v = rb[i];
            if (BKN) {
                if (k0 + bk_[i] >= K) v = f32x4{0.f, 0.f, 0.f, 0.f};
                *reinterpret_cast<f32x4 *>(buf + A_SZ + bk_[i] * BP + brow_l[i]) = v;
            } else {
                if (k0 + bk_[i] >= K) v = f32x4{0.f, 0.f, 0.f, 0.f};
                *reinterpret_cast<f32x4 *>(buf + A_SZ + brow_l[i] * AP + bk_[i]) = v;
            }
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int r = lane & 31, h = lane >> 5;
    // lane half h takes k = KL*h + s of the chunk in MFMA step s (the same for A and B)
    auto compute = [&](const float *buf) {
        float a[2][KL], b[2][KL];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const float *pa = buf + (wm0 + 32 * t + r) * AP + KL * h;
#pragma unroll
            for (int q = 0; q < KL / 4; ++q) {
                const f32x4 v = *reinterpret_cast<const f32x4 *>(pa + 4 * q);
                a[t][4 * q] = v.x; a[t][4 * q + 1] = v.y; a[t][4 * q + 2] = v.z; a[t][4 * q + 3] = v.w;
            }
            if (BKN) {
                const float *pb = buf + A_SZ + (KL * h) * BP + wn0 + 32 * t + r;
#pragma unroll
                for (int s = 0; s < KL; ++s) b[t][s] = pb[s * BP];
            } else {
                const float *pb = buf + A_SZ + (wn0 + 32 * t + r) * AP + KL * h;
#pragma unroll
                for (int q = 0; q < KL / 4; ++q) {
                    const f32x4 v = *reinterpret_cast<const f32x4 *>(pb + 4 * q);
                    b[t][4 * q] = v.x; b[t][4 * q + 1] = v.y; b[t][4 * q + 2] = v.z; b[t][4 * q + 3] = v.w;
                }
            }
        }
#pragma unroll
        for (int s = 0; s < KL; ++s)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
    };

    const int nc = (K + BK - 1) / BK;
    gload(0);
    lstore(0, lds[0]);
    __syncthreads();
    // The next chunk's loads are unconditional (past K the clamped addresses stay in the
    // operands and lstore zeroes the values), so the compiler's wait counts stay exact.
    for (int c = 0; c < nc; ++c) {
        gload((c + 1) * BK);
        __builtin_amdgcn_sched_barrier(0);
        compute(lds[c & 1]);
        __builtin_amdgcn_sched_barrier(0);
        lstore((c + 1) * BK, lds[(c + 1) & 1]);
        __syncthreads();
    }

    const bool live = bm0 + wm0 < M && bn0 + wn0 < N;
    if (!live) return;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = bn0 + wn0 + 32 * j + r;
            if (col >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = bm0 + wm0 + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
                if (row < M) C[(int64_t)row * ldc + col] = acc[i][j][e];
            }
        }
}


// C = 0 for a K = 0 product (the empty dot product), grid (ceil(M*N/256), inner, outer).
__global__ __launch_bounds__(256) void fill_zero_f32(float *__restrict__ C, int64_t ldc, int64_t sc1, int64_t sc2,
                                                     int M, int N) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)M * N) return;
    C[blockIdx.y * sc1 + blockIdx.z * sc2 + (i / N) * ldc + i % N] = 0.0f;
}

}  // namespace enchip
