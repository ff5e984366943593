// attention_f32.h -- scaled dot-product attention of one (32-query tile, head, sequence)
// per workgroup, with the score tile resident in LDS: the device form of
// encoder/attention.go:81-121 attentionCore up to the context (the output projection is
// the next W8A8 linear).
//
// The unfused path writes the [L, L] scores of every head to HBM, reads and rewrites them
// for the softmax and reads them again for scores . V (three round trips of 805 MB per
// BERT-base layer at 64 x 512). Here they never leave the CU:
//   1. S = Q_tile . K^T on the f32 MFMA (v_mfma_f32_32x32x2_f32): each wavefront takes
//      32-key tiles, its Q and K operands loaded straight into registers, and stores
//      S * scale (the reference's first softmax pass, an f32 multiply) into LDS.
//   2. softmaxRowScaled's remaining steps on each LDS row, as softmax_rows_scaled does
//      them (first-element max, expF32Core, float64 sum, f32 reciprocal, f32 multiply);
//      meanwhile each wavefront's V operands for step 3 are already loading (the
//      barriers fence LDS only, so they do not wait for those loads).
//   3. ctx = P . V: wavefront (output tile, key group) sums its keys on the MFMA; the
//      key groups' partial tiles are added in LDS in a fixed order and stored.
// Arithmetic differs from the unfused kernels only in summation order (the key groups of
// step 3), so results agree within the f32 MatmulBT gate. L <= ATT_MAX_L.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "encoder_ops.h"
#include "gemm_f32.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace enchip {

constexpr int ATT_QT = 32;       // query rows per workgroup
constexpr int ATT_WAVES = 8;     // 512 threads
constexpr int ATT_MAX_L = 512;   // keys per row held in LDS (and V operands in registers)
constexpr int ATT_MAX_KT = ATT_MAX_L / 32;

// LDS floats a workgroup needs for L keys: the score tile (row pitch a whole number of
// 32-key tiles plus 4 against bank conflicts), at least the 8 partial 32x32 tiles.
__host__ __device__ inline int att_pitch(int L) { return 32 * ((L + 31) / 32) + 4; }
__host__ __device__ inline int att_lds_floats(int L) {
    const int a = ATT_QT * att_pitch(L), b = ATT_WAVES * 1024;
    return a > b ? a : b;
}

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 8 consecutive floats from a 16-byte aligned address.
__device__ __forceinline__ void load8(const float *p, float *d) {
    const f32x4 a = *reinterpret_cast<const f32x4 *>(p), b = *reinterpret_cast<const f32x4 *>(p + 4);
    d[0] = a.x; d[1] = a.y; d[2] = a.z; d[3] = a.w;
    d[4] = b.x; d[5] = b.y; d[6] = b.z; d[7] = b.w;
}

// HD: head dimension (32 or 64). A 1-D grid of ceil(L/32) * heads * sequences
// workgroups of 512 threads, att_lds_floats(L) floats of dynamic LDS. Workgroups are
// mapped XCD-aware (xcd_logical_tile): the query tiles of one (head, sequence) run on one
// XCD, so its K and V (256 KB at L = 512) are fetched into one L2 (measured neutral at
// BERT-base shapes, where K and V stay in the 256 MB MALL either way).
// Row i of sequence z, head h starts at q/k/v + (z*L + i)*ld + h*HD (16-byte aligned),
// out + (z*L + i)*ldo + h*HD.
template <int HD>
__global__ __launch_bounds__(64 * ATT_WAVES, 4) void attention_f32(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v, int64_t ld,
    float *__restrict__ out, int64_t ldo, int L, int heads, float scale) {
    static_assert(HD == 32 || HD == 64, "head dimension");
    constexpr int NOT = HD / 32;                     // 32-column output tiles of the context
    constexpr int G = ATT_WAVES / NOT;               // key groups in step 3
    constexpr int KPL = HD / 2;                      // head-dim values per lane in step 1
    constexpr int T1 = ATT_MAX_KT / ATT_WAVES;       // key tiles per wavefront in step 1, at most
    constexpr int T3 = (ATT_MAX_KT + G - 1) / G;     // key tiles per wavefront in step 3, at most
    extern __shared__ __attribute__((aligned(16))) float sc[];
    const int P = att_pitch(L);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 31, hf = lane >> 5;
    const int nkt = (L + 31) / 32, nqt = (L + ATT_QT - 1) / ATT_QT;
    const int logical = xcd_logical_tile(blockIdx.x, gridDim.x);
    const int q0 = (logical % nqt) * ATT_QT, head = (logical / nqt) % heads;
    const int64_t row0 = (int64_t)(logical / nqt / heads) * L;

    // ---- 1. S = Q K^T * scale into LDS. In MFMA step s of 16-deep block b, lane half hf
    // supplies head-dim index 16b + 8hf + s of both operands; rows past L re-read row L-1.
    float qa[KPL], kb[T1][KPL];
    {
        const float *qrow = q + (row0 + min(q0 + r, L - 1)) * ld + head * HD;
#pragma unroll
        for (int b = 0; b < HD / 16; ++b) load8(qrow + 16 * b + 8 * hf, qa + 8 * b);
#pragma unroll
        for (int t = 0; t < T1; ++t) {
            const int kt = min(wave + ATT_WAVES * t, nkt - 1);
            const float *krow = k + (row0 + min(32 * kt + r, L - 1)) * ld + head * HD;
#pragma unroll
            for (int b = 0; b < HD / 16; ++b) load8(krow + 16 * b + 8 * hf, kb[t] + 8 * b);
        }
    }
#pragma unroll
    for (int t = 0; t < T1; ++t) {
        const int kt = wave + ATT_WAVES * t;
        if (kt >= nkt) break;
        f32x16 acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
        for (int s = 0; s < KPL; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[s], kb[t][s], acc, 0, 0, 0);
        const int col = 32 * kt + r;
        if (col < L) {
#pragma unroll
            for (int e = 0; e < 16; ++e) sc[(8 * (e >> 2) + 4 * hf + (e & 3)) * P + col] = acc[e] * scale;
        }
    }

    // ---- 3's V operands, loading while the softmax runs. Wavefront (ot, g) takes key
    // tiles g, g + G, ... and output columns 32*ot .. +32; in 16-key block b of a tile,
    // lane half hf supplies keys 16b + 8hf + s (s < 8) of column 32*ot + r. Keys past L
    // re-read row L-1 (their P is zero).
    const int ot = wave % NOT, g = wave / NOT;
    float vv[T3][2][8];
    {
        const float *vcol = v + row0 * ld + head * HD + 32 * ot + r;
#pragma unroll
        for (int i = 0; i < T3; ++i)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int s = 0; s < 8; ++s) {
                    const int key = 32 * (g + G * i) + 16 * b + 8 * hf + s;
                    vv[i][b][s] = vcol[(int64_t)min(key, L - 1) * ld];
                }
    }
    lds_barrier();

    // ---- 2. softmax of each LDS row (4 rows per wavefront), as softmax_rows_scaled.
    for (int row = wave; row < ATT_QT; row += ATT_WAVES) {
        float *p = sc + row * P;
        constexpr int CPL = ATT_MAX_L / 64;
        float x[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = lane + 64 * j;
            x[j] = c < L ? p[c] : -INFINITY;
        }
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < CPL; ++j) m = x[j] > m ? x[j] : m;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(m, off, 64);
            m = o > m ? o : m;
        }
        const float first = __shfl(x[0], 0, 64);
        if (first != first) m = first;
        double sum = 0.0;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = lane + 64 * j;
            const float e = c < L ? exp_f32_core(x[j] - m) : 0.0f;
            x[j] = e;
            sum += (double)e;
        }
        sum = wave_sum_f64(sum);
        const bool uniform = sum == 0.0;
        const float u = 1.0f / (float)L;
        const float inv = uniform ? 0.0f : (float)(1.0 / sum);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = lane + 64 * j;
            if (c < L) p[c] = uniform ? u : x[j] * inv;
            else if (c < 32 * nkt) p[c] = 0.0f;  // keys past L in the last tile add nothing
        }
    }
    lds_barrier();

    // ---- 3. ctx partial = P[:, this group's keys] . V[those keys, 32*ot .. +32]
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
    for (int i = 0; i < T3; ++i) {
        const int kt = g + G * i;
        if (kt >= nkt) break;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            float pv[8];
            load8(sc + r * P + 32 * kt + 16 * b + 8 * hf, pv);
#pragma unroll
            for (int s = 0; s < 8; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(pv[s], vv[i][b][s], acc, 0, 0, 0);
        }
    }
    lds_barrier();  // every wavefront is done reading P: the LDS takes the partial tiles

    float *part = sc + (g * NOT + ot) * 1024;
#pragma unroll
    for (int e = 0; e < 16; ++e) part[(8 * (e >> 2) + 4 * hf + (e & 3)) * 32 + r] = acc[e];
    lds_barrier();

    // add the G key groups in order and store: one element per thread per round
    for (int idx = threadIdx.x; idx < ATT_QT * HD; idx += 64 * ATT_WAVES) {
        const int row = idx / HD, c = idx % HD, o = c / 32, cc = c % 32;
        float s = sc[o * 1024 + row * 32 + cc];
        for (int gg = 1; gg < G; ++gg) s += sc[(gg * NOT + o) * 1024 + row * 32 + cc];
        const int qrow = q0 + row;
        if (qrow < L) out[(row0 + qrow) * ldo + head * HD + c] = s;
    }
}

}  // namespace enchip
