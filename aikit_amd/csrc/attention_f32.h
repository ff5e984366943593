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
// attention_split_bf16 adds its Q tile's bf16 hi / lo planes after the score tile: 32 rows
// of 64 values at a 144-byte pitch (bank-conflict-free 16-byte reads) per plane.
constexpr int ATT_QPITCH = 144;  // bytes per Q row per plane (head dim <= 64)
__host__ __device__ inline int att_split_lds_floats(int L) { return att_lds_floats(L) + 2 * ATT_QT * ATT_QPITCH / 4; }

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
            const float e = c < L ? exp_f32_core_nonpos(x[j] - m) : 0.0f;
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

// ---------------------------------------------------------------------------
// The same attention with both products on the bf16 MFMA (v_mfma_f32_32x32x16_bf16),
// each f32 operand split into two bfloat16 parts: the 3-product split-bfloat16 method of
// Henry, Tang and Heinecke ("Leveraging the bfloat16 Artificial Intelligence Datatype For
// Higher-Precision Computations", ARITH 2019).
//   x = hi + lo + e,  hi = bf16(x), lo = bf16(x - hi) (round to nearest even; x - hi is
//   exact in f32), |e| <= 2^-18 |x|;
//   x.y ~= hi.hi' + hi.lo' + lo.hi', the dropped terms at most 3 * 2^-18 |x y|.
// The products are exact in f32 and summed in f32 accumulators, so each dot product is
// within ~1e-5 of its f32 value relative to the sum of |terms|, inside the f32 MatmulBT
// gate of the reference (gpu/enccuda/backend_test.go:71-81, <= 2e-4 of max(|ref|, 1)).
// Per 16-deep block that is 3 MFMAs of 32 cycles against 8 f32 MFMAs of 64, plus ~3 VALU
// operations per operand value for the split.
//
// Same grid and phases as attention_f32 (LDS: att_split_lds_floats(L) floats, the extra
// holding the Q tile split once for all 8 wavefronts); operand lanes hold the same values
// (lane half hf supplies depth 8hf..8hf+7 of each 16-deep block), now as bf16x8 pairs.
// The softmax writes P already split: row r of the score tile (4P bytes) becomes a bf16
// hi plane at byte 0 and a bf16 lo plane at byte 2P + 8 (both 16-byte aligned, 32 * nkt
// entries each), and each softmax lane owns 2 adjacent columns so that both planes are
// written a 32-bit word at a time. Non-finite operands give NaN (inf - inf in the split).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void split_bf16x8(const float *x, bf16x8 &hi, bf16x8 &lo) {
#pragma unroll
    for (int s = 0; s < 8; s += 2) {
        const bf16x2 h = __builtin_convertvector((f32x2){x[s], x[s + 1]}, bf16x2);
        const bf16x2 l = __builtin_convertvector((f32x2){x[s] - (float)h[0], x[s + 1] - (float)h[1]}, bf16x2);
        hi[s] = h[0];
        hi[s + 1] = h[1];
        lo[s] = l[0];
        lo[s + 1] = l[1];
    }
}

__device__ __forceinline__ f32x16 mfma_split3(const bf16x8 &ah, const bf16x8 &al, const bf16x8 &bh, const bf16x8 &bl,
                                              f32x16 acc) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, acc, 0, 0, 0);
}

// Two f32 values -> the 32-bit words of their hi and lo bf16 parts (element 0 low).
__device__ __forceinline__ void split_pair(float a, float b, uint32_t &hw, uint32_t &lw) {
    const bf16x2 h = __builtin_convertvector((f32x2){a, b}, bf16x2);
    const bf16x2 l = __builtin_convertvector((f32x2){a - (float)h[0], b - (float)h[1]}, bf16x2);
    hw = __builtin_bit_cast(uint32_t, h);
    lw = __builtin_bit_cast(uint32_t, l);
}

// The same split into IEEE half parts (11-bit significands): x = hi + lo + e with hi =
// f16(x), lo = f16(x - hi) (x - hi is exact in f32), |e| <= 2^-22 |x| while lo is a
// normal half (|x| >= 2^-3; below that lo is subnormal and e <= 2^-25 absolute), so
// x.y ~= hi.hi' + hi.lo' + lo.hi' is within ~3 * 2^-22 |x y| -- 64 times closer than the
// bfloat16 split at the same MFMA cost. hi is finite only for |x| < 65520: a larger
// operand gives inf - inf = NaN in the products, never a finite wrong value.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void split_f16x8(const float *x, f16x8 &hi, f16x8 &lo) {
#pragma unroll
    for (int s = 0; s < 8; s += 2) {
        const f16x2 h = __builtin_convertvector((f32x2){x[s], x[s + 1]}, f16x2);
        const f16x2 l = __builtin_convertvector((f32x2){x[s] - (float)h[0], x[s + 1] - (float)h[1]}, f16x2);
        hi[s] = h[0];
        hi[s + 1] = h[1];
        lo[s] = l[0];
        lo[s + 1] = l[1];
    }
}

__device__ __forceinline__ f32x16 mfma_split3(const f16x8 &ah, const f16x8 &al, const f16x8 &bh, const f16x8 &bl,
                                              f32x16 acc) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, acc, 0, 0, 0);
}

__device__ __forceinline__ void split_pair_f16(float a, float b, uint32_t &hw, uint32_t &lw) {
    const f16x2 h = __builtin_convertvector((f32x2){a, b}, f16x2);
    const f16x2 l = __builtin_convertvector((f32x2){a - (float)h[0], b - (float)h[1]}, f16x2);
    hw = __builtin_bit_cast(uint32_t, h);
    lw = __builtin_bit_cast(uint32_t, l);
}

// The operand formats of the flash attention's split products: F16 selects the half
// split above, otherwise the bfloat16 one.
template <bool F16>
struct SplitOps;
template <>
struct SplitOps<false> {
    typedef bf16x8 vec8;
    static __device__ __forceinline__ void split8(const float *x, vec8 &h, vec8 &l) { split_bf16x8(x, h, l); }
    static __device__ __forceinline__ void pair(float a, float b, uint32_t &h, uint32_t &l) { split_pair(a, b, h, l); }
};
template <>
struct SplitOps<true> {
    typedef f16x8 vec8;
    static __device__ __forceinline__ void split8(const float *x, vec8 &h, vec8 &l) { split_f16x8(x, h, l); }
    static __device__ __forceinline__ void pair(float a, float b, uint32_t &h, uint32_t &l) { split_pair_f16(a, b, h, l); }
};

// FULL: L == ATT_MAX_L, so every bounds check of the tile loops folds away.
template <int HD, bool FULL>
__global__ __launch_bounds__(64 * ATT_WAVES, 4) void attention_split_bf16(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v, int64_t ld,
    float *__restrict__ out, int64_t ldo, int L_arg, int heads, float scale) {
    const int L = FULL ? ATT_MAX_L : L_arg;
    static_assert(HD == 32 || HD == 64, "head dimension");
    constexpr int NOT = HD / 32;
    constexpr int G = ATT_WAVES / NOT;
    constexpr int NB = HD / 16;                      // 16-deep blocks of the head dimension
    constexpr int T1 = ATT_MAX_KT / ATT_WAVES;
    constexpr int T3 = (ATT_MAX_KT + G - 1) / G;
    extern __shared__ __attribute__((aligned(16))) float sc[];
    const int P = att_pitch(L);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 31, hf = lane >> 5;
    const int nkt = (L + 31) / 32, nqt = (L + ATT_QT - 1) / ATT_QT;
    const int logical = xcd_logical_tile(blockIdx.x, gridDim.x);
    const int q0 = (logical % nqt) * ATT_QT, head = (logical / nqt) % heads;
    const int64_t row0 = (int64_t)(logical / nqt / heads) * L;

    // ---- 0. the Q tile, split once for the workgroup: thread t takes 4 consecutive values
    // of row t / (HD/4) (rows past L re-read row L-1) and writes their hi / lo words to
    // the planes after the score tile.
    char *qplanes = reinterpret_cast<char *>(sc + att_lds_floats(L));
    if (threadIdx.x < ATT_QT * HD / 4) {
        const int qr = threadIdx.x / (HD / 4), qc = 4 * (threadIdx.x % (HD / 4));
        const f32x4 v = *reinterpret_cast<const f32x4 *>(q + (row0 + min(q0 + qr, L - 1)) * ld + head * HD + qc);
        uint32_t h0, l0, h1, l1;
        split_pair(v.x, v.y, h0, l0);
        split_pair(v.z, v.w, h1, l1);
        *reinterpret_cast<uint2 *>(qplanes + qr * ATT_QPITCH + 2 * qc) = make_uint2(h0, h1);
        *reinterpret_cast<uint2 *>(qplanes + ATT_QT * ATT_QPITCH + qr * ATT_QPITCH + 2 * qc) = make_uint2(l0, l1);
    }
    // ---- 1. S = Q K^T * scale into LDS (f32), key rows past L re-read row L-1.
    float kb[T1][HD / 2];
#pragma unroll
    for (int t = 0; t < T1; ++t) {
        const int kt = min(wave + ATT_WAVES * t, nkt - 1);
        const float *krow = k + (row0 + min(32 * kt + r, L - 1)) * ld + head * HD;
#pragma unroll
        for (int b = 0; b < NB; ++b) load8(krow + 16 * b + 8 * hf, kb[t] + 8 * b);
    }
    lds_barrier();
    bf16x8 qh[NB], ql[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const char *qp = qplanes + r * ATT_QPITCH + 2 * (16 * b + 8 * hf);
        qh[b] = *reinterpret_cast<const bf16x8 *>(qp);
        ql[b] = *reinterpret_cast<const bf16x8 *>(qp + ATT_QT * ATT_QPITCH);
    }
#pragma unroll
    for (int t = 0; t < T1; ++t) {
        const int kt = wave + ATT_WAVES * t;
        if (kt >= nkt) break;
        f32x16 acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            bf16x8 kh, kl;
            split_bf16x8(kb[t] + 8 * b, kh, kl);
            acc = mfma_split3(qh[b], ql[b], kh, kl, acc);
        }
        const int col = 32 * kt + r;
        if (col < L) {
#pragma unroll
            for (int e = 0; e < 16; ++e) sc[(8 * (e >> 2) + 4 * hf + (e & 3)) * P + col] = acc[e] * scale;
        }
    }

    // ---- 3's V operands, loading while the softmax runs (as attention_f32).
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

    // ---- 2. softmax of each LDS row, as softmax_rows_scaled, lane owning columns
    // 2*lane + 128*j + {0, 1}; P written as its hi / lo bf16 planes over the row.
    for (int row = wave; row < ATT_QT; row += ATT_WAVES) {
        float *p = sc + row * P;
        constexpr int CPL2 = ATT_MAX_L / 128;
        float x[CPL2][2];
#pragma unroll
        for (int j = 0; j < CPL2; ++j) {
            const int c = 2 * lane + 128 * j;
            f32x2 t = {-INFINITY, -INFINITY};
            if (c + 1 < L) t = *reinterpret_cast<const f32x2 *>(p + c);
            else if (c < L) t[0] = p[c];
            x[j][0] = t[0];
            x[j][1] = t[1];
        }
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < CPL2; ++j) {
            m = x[j][0] > m ? x[j][0] : m;
            m = x[j][1] > m ? x[j][1] : m;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(m, off, 64);
            m = o > m ? o : m;
        }
        const float first = __shfl(x[0][0], 0, 64);
        if (first != first) m = first;
        double sum = 0.0;
#pragma unroll
        for (int j = 0; j < CPL2; ++j)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int c = 2 * lane + 128 * j + u;
                const float e = c < L ? exp_f32_core_nonpos(x[j][u] - m) : 0.0f;
                x[j][u] = e;
                sum += (double)e;
            }
        sum = wave_sum_f64(sum);
        const bool uniform = sum == 0.0;
        const float un = 1.0f / (float)L;
        const float inv = uniform ? 0.0f : (float)(1.0 / sum);
        uint32_t *ph = reinterpret_cast<uint32_t *>(p);
        uint32_t *pl = reinterpret_cast<uint32_t *>(reinterpret_cast<char *>(p) + 2 * P + 8);
#pragma unroll
        for (int j = 0; j < CPL2; ++j) {
            const int c = 2 * lane + 128 * j;
            if (c >= 32 * nkt) continue;  // keys past the last tile are never read
            // keys past L in the last tile: P = 0 (hi and lo)
            const float a = c < L ? (uniform ? un : x[j][0] * inv) : 0.0f;
            const float b = c + 1 < L ? (uniform ? un : x[j][1] * inv) : 0.0f;
            uint32_t hw, lw;
            split_pair(a, b, hw, lw);
            ph[c >> 1] = hw;
            pl[c >> 1] = lw;
        }
    }
    lds_barrier();

    // ---- 3. ctx partial = P[:, this group's keys] . V[those keys, 32*ot .. +32]
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
    {
        const char *prow = reinterpret_cast<const char *>(sc + r * P);
#pragma unroll
        for (int i = 0; i < T3; ++i) {
            const int kt = g + G * i;
            if (kt >= nkt) break;
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int key = 32 * kt + 16 * b + 8 * hf;
                const bf16x8 ph = *reinterpret_cast<const bf16x8 *>(prow + 2 * key);
                const bf16x8 pl = *reinterpret_cast<const bf16x8 *>(prow + 2 * P + 8 + 2 * key);
                bf16x8 vh, vl;
                split_bf16x8(vv[i][b], vh, vl);
                acc = mfma_split3(ph, pl, vh, vl, acc);
            }
        }
    }
    lds_barrier();  // every wavefront is done reading P: the LDS takes the partial tiles

    float *part = sc + (g * NOT + ot) * 1024;
#pragma unroll
    for (int e = 0; e < 16; ++e) part[(8 * (e >> 2) + 4 * hf + (e & 3)) * 32 + r] = acc[e];
    lds_barrier();

    for (int idx = threadIdx.x; idx < ATT_QT * HD; idx += 64 * ATT_WAVES) {
        const int row = idx / HD, c = idx % HD, o = c / 32, cc = c % 32;
        float s = sc[o * 1024 + row * 32 + cc];
        for (int gg = 1; gg < G; ++gg) s += sc[(gg * NOT + o) * 1024 + row * 32 + cc];
        const int qrow = q0 + row;
        if (qrow < L) out[(row0 + qrow) * ldo + head * HD + c] = s;
    }
}

}  // namespace enchip
