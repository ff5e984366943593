// kernels.h -- gfx950 kernels of the W8A8 linear path.
//
//   quant_rows_vec / quant_rows_scalar  per-token dynamic int8 quantization
//   gemm_w8a8                           tiled int8 MFMA GEMM + fused dequant epilogue
//   gemv_w8a8                           small-M (HBM-bound) split-K MFMA variant
//
// Data layout in HBM
//   activations (f32, caller)   a[M][K] row-major
//   quantized activations       aq[M][lda] int8 row-major, lda a multiple of 64 >= K,
//                               columns [K,lda) zero (the GEMMs read rows past M as
//                               row M-1 and never store them); or, for the persistent
//                               GEMM, fragment-major like the weights (frag_off), rows
//                               past M read but never stored
//   activation scales           as[Mp] f32
//   weights (pre-swizzled once) wf[Np/32][Kp/32][64 lanes][16 B] int8 -- one 1 KiB
//                               "fragment" per 32 output channels x 32 k; lane l holds
//                               W[n0 + l%32][k0 + 16*(l/32) .. +16], the operand
//                               layout of v_mfma_i32_32x32x32_i8. Np = roundup(N,256),
//                               padding rows/columns zero.
//   weight scales / bias        f32 [N]
//   output                      dst[M][ldo] f32 (or int32 accumulators in debug mode)
//
// Exactness: the int8 products are summed in int32 by the MFMA unit, exactly, in
// whatever order; the only roundings are the epilogue's, done in the reference's
// order with contraction disabled (see gelu_f32.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gelu_f32.h"

#pragma clang fp contract(off)

namespace enchip {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// EPI_TOPK (gemm_w8a8_pt only): the f32 outputs of EPI_F32 are not stored; each one at or
// above its row's bound goes to the row's top-k candidate list (TopkSink).
enum Epi { EPI_I32 = 0, EPI_F32 = 1, EPI_F32_GELU = 2, EPI_TOPK = 3 };

// ----------------------------------------------------------------------------
// Quantization (linalg/quant.go:43-71, activations' all-zero row -> scale 0).

// One code: math.Round(float64(v*inv)) clamped to +-127. v*inv is a single f32
// multiply; roundf is round-half-away-from-zero like Go's math.Round, and exact
// for every float32. A NaN (from an Inf or NaN input) converts to 0 as Go's
// int8(NaN) does on amd64.
// Written without branches (the if / else-if clamp compiled to divergent branches per
// value): the clamp as max / min, which turns a NaN into -127, then the NaN test picks 0.
__device__ __forceinline__ int quant_code(float v, float inv) {
    const float x = roundf(v * inv);
    const float c = fminf(fmaxf(x, -127.0f), 127.0f);
    return x == x ? (int)c : 0;
}

// Max of |v| ignoring NaN, as the reference's `if v > maxAbs` does.
__device__ __forceinline__ float absmax_step(float m, float v) {
    float t = fabsf(v);
    return t > m ? t : m;
}

// Cross-lane moves for wavefront reductions, all VALU (no LDS permute, no wait):
//   lane_dpp<CTRL>(v): v of the lane a DPP pattern names within each 16-lane row (every
//     lane has a source lane): 0xB1 = lane ^ 1, 0x4E = lane ^ 2, 0x141 = the mirror in
//     each group of 8 (lane ^ 7), 0x140 = the mirror in each row (lane ^ 15);
//   lane_swap16 / lane_swap32(v): {v, v of lane ^ 16} / {v, v of lane ^ 32}, in an order
//     that depends on the lane (v_permlane16_swap / v_permlane32_swap of v with itself).
// A reduction that applies ^1, ^2, then the 8- and 16-lane mirrors sees lane ^ 4 and
// lane ^ 8 through the mirrors, because by then each group of 4 (then 8) holds one value.
template <int CTRL>
__device__ __forceinline__ uint32_t lane_dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ void lane_swap16(uint32_t v, uint32_t &a, uint32_t &b) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    a = r[0];
    b = r[1];
}
__device__ __forceinline__ void lane_swap32(uint32_t v, uint32_t &a, uint32_t &b) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    a = r[0];
    b = r[1];
}

// The maximum over the wavefront of per-lane maxima that are never NaN (absmax_step's),
// in every lane: max is order-free there, so any pairing gives the same bits.
__device__ __forceinline__ float wave_absmax(float m) {
    auto step = [](float x, float o) { return o > x ? o : x; };
    m = step(m, __uint_as_float(lane_dpp<0xB1>(__float_as_uint(m))));
    m = step(m, __uint_as_float(lane_dpp<0x4E>(__float_as_uint(m))));
    m = step(m, __uint_as_float(lane_dpp<0x141>(__float_as_uint(m))));
    m = step(m, __uint_as_float(lane_dpp<0x140>(__float_as_uint(m))));
    uint32_t a, b;
    lane_swap16(__float_as_uint(m), a, b);
    m = step(__uint_as_float(a), __uint_as_float(b));
    lane_swap32(__float_as_uint(m), a, b);
    return step(__uint_as_float(a), __uint_as_float(b));
}

// Byte offset of code (row, k) in the fragment-major activation layout
// [Mp/32][ldq/32][64 lanes][16 B]: one 1 KiB fragment per 32 rows x 32 k, lane l
// holding row 32*rb + l%32, k 32*kb + 16*(l/32) .. +16 -- the A-operand layout of
// v_mfma_i32_32x32x32_i8, the same as the weights'. The persistent GEMM loads a
// fragment as 64 lanes x 16 contiguous bytes (8 full cache lines per instruction);
// a row-major A tile touches 32 lines per instruction and uses 32 B of each.
__device__ __forceinline__ int64_t frag_off(int64_t row, int64_t k, int64_t nk32) {
    return (((row >> 5) * nk32 + (k >> 5)) << 10) + ((((row & 31) + ((k >> 4) & 1) * 32)) << 4) + (k & 15);
}

// One wavefront per row, 4 rows per 256-thread block. Each lane holds CH float4 of
// the row in registers (K <= 256*CH, K % 4 == 0, rows 16-byte aligned), so the
// row is read from HBM exactly once. The reads are nontemporal: the f32 rows are
// read once, and caching them only evicts the codes the GEMM reads next (measured
// 1.3-1.6x faster on MI355X).
template <int CH>
__device__ __forceinline__ void load_row_raw(const float *__restrict__ a, int64_t row, int K, int lane, float4 (&v)[CH]) {
    const f32x4 *src = reinterpret_cast<const f32x4 *>(a + row * (int64_t)K);
    const int K4 = K >> 2;
    // Unconditional loads (lanes past the row re-read its last float4 and zero it), so
    // all CH are in flight at once; behind a per-chunk branch the compiler waits for
    // each load before issuing the next. The zeroing is a bit mask, not a select: the
    // compiler turns a select of a loaded value back into a branch around the load.
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int k4 = lane + 64 * c;
        const i32x4 t = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(src) + min(k4, K4 - 1));
        const int keep = k4 < K4 ? -1 : 0;
        v[c] = make_float4(__int_as_float(t.x & keep), __int_as_float(t.y & keep), __int_as_float(t.z & keep),
                           __int_as_float(t.w & keep));
    }
}

template <int CH>
__device__ __forceinline__ float row_absmax(const float4 (&v)[CH]) {
    float m = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        m = absmax_step(m, v[c].x);
        m = absmax_step(m, v[c].y);
        m = absmax_step(m, v[c].z);
        m = absmax_step(m, v[c].w);
    }
    return wave_absmax(m);
}

template <int CH>
__device__ __forceinline__ float load_row(const float *__restrict__ a, int64_t row, int K, int lane, float4 (&v)[CH]) {
    load_row_raw<CH>(a, row, K, lane, v);
    return row_absmax<CH>(v);
}

__device__ __forceinline__ int pack_codes(float4 v, float inv) {
    const int c0 = quant_code(v.x, inv), c1 = quant_code(v.y, inv);
    const int c2 = quant_code(v.z, inv), c3 = quant_code(v.w, inv);
    return (c0 & 0xff) | ((c1 & 0xff) << 8) | ((c2 & 0xff) << 16) | ((int)((unsigned)c3 << 24));
}

// pack_codes for a row whose scale s = maxAbs/127 is a normal float (s >= 2^-126, or
// +inf): then |v * inv| <= 127 * (1 + 3 * 2^-24) for every finite v of the row, so the
// rounded value needs no clamp, and v_cvt_i32_f32 turns a NaN into 0 as quant_code does
// (its float-to-int conversion is written in assembly because a C++ conversion of NaN is
// undefined). With a subnormal s the quotient can exceed 127, so such rows take
// pack_codes.
__device__ __forceinline__ int cvt_i32_f32(float x) {
    int r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(x));
    return r;
}
// math.Round of x for |x| <= 2^22 (here |x| <= 127.00003): trunc(x + copysign(h, x)) with
// h = 0.5 - 2^-25, one add and one truncation where roundf takes six operations. The sum
// stays in x's binade (below the next integer), where 2^-25 is under half an ulp: an exact
// half (n + 0.5) gives n + 1 - 2^-25, which rounds to n + 1 (for n = 0 the tie rounds to the
// even 1.0), and any x below n + 0.5 (by at least one ulp) gives a sum that rounds below
// n + 1. NaN stays NaN.
__device__ __forceinline__ float round_half_away_small(float x) {
    return __builtin_truncf(x + __builtin_copysignf(__uint_as_float(0x3effffffu), x));
}
__device__ __forceinline__ int pack_codes_normal(float4 v, float inv) {
    const int c0 = cvt_i32_f32(round_half_away_small(v.x * inv)), c1 = cvt_i32_f32(round_half_away_small(v.y * inv));
    const int c2 = cvt_i32_f32(round_half_away_small(v.z * inv)), c3 = cvt_i32_f32(round_half_away_small(v.w * inv));
    return (c0 & 0xff) | ((c1 & 0xff) << 8) | ((c2 & 0xff) << 16) | ((int)((unsigned)c3 << 24));
}
// absmax_step for values that are never signalling NaNs (results of arithmetic): the IEEE
// maximum returns the operand that is not a quiet NaN, so max(m, |v|) with m never NaN is
// `if |v| > m` (equal values have equal bits), in one instruction instead of a compare and
// a select.
__device__ __forceinline__ float absmax_step_quiet(float m, float v) {
    float r;
    asm("v_max_f32_e64 %0, %1, |%2|" : "=v"(r) : "v"(m), "v"(v));
    return r;
}

// Row-major codes q[M][ldq], written as packed 32-bit words; columns [K, ldq) zero.
template <int CH>
__global__ __launch_bounds__(256) void quant_rows_vec(const float *__restrict__ a,
                                                      int8_t *__restrict__ q, int64_t ldq,
                                                      float *__restrict__ scale, int64_t M,
                                                      int K) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    float4 v[CH];
    const float m = load_row<CH>(a, row, K, lane, v);
    int *dst = reinterpret_cast<int *>(q + row * ldq);
    const int K4 = K >> 2, ldq4 = (int)(ldq >> 2);
    if (m == 0.0f) {
        for (int k4 = lane; k4 < ldq4; k4 += 64) dst[k4] = 0;
        if (lane == 0) scale[row] = 0.0f;
        return;
    }
    const float s = m / 127.0f;
    const float inv = 1.0f / s;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int k4 = lane + 64 * c;
        if (k4 < K4) dst[k4] = pack_codes(v[c], inv);
    }
    for (int k4 = K4 + lane; k4 < ldq4; k4 += 64) dst[k4] = 0;
    if (lane == 0) scale[row] = s;
}

// Fragment-major codes (frag_off; ldq a multiple of 64, ldq <= 256*CH). Rows 8t..8t+7
// of a 32-row block fill one 128-byte line of each 1 KiB fragment (16 bytes each), so a
// single row's codes land in 16-byte pieces of ldq/16 different lines. Here a block
// quantizes 8 such rows, RPW per wavefront (all of a wavefront's row loads in flight at
// once, so short rows still keep enough bytes in flight), gathers their codes in LDS in
// line order, and then writes whole lines with 16-byte stores.
template <int CH, int RPW>
__global__ __launch_bounds__(512 / RPW) void quant_rows_frag(const float *__restrict__ a,
                                                             int8_t *__restrict__ q, int64_t ldq,
                                                             float *__restrict__ scale, int64_t M,
                                                             int K) {
    constexpr int NT = 512 / RPW;
    constexpr int CP = 144;  // LDS bytes per 16-code chunk: 8 rows x 16 B + 16 B against bank conflicts
    __shared__ __attribute__((aligned(16))) int8_t lds[16 * CH * CP];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * 8;
    const int K4 = K >> 2, ldq4 = (int)(ldq >> 2);
    // the 32-bit word of codes 4*k4 .. 4*k4+3 of block row rr
    auto word = [&](int rr, int k4) -> int * { return reinterpret_cast<int *>(lds + (k4 >> 2) * CP + rr * 16 + (k4 & 3) * 4); };
    float4 v[RPW][CH];
#pragma unroll
    for (int u = 0; u < RPW; ++u) load_row_raw<CH>(a, min(r0 + wave * RPW + u, M - 1), K, lane, v[u]);
#pragma unroll
    for (int u = 0; u < RPW; ++u) {
        const int rr = wave * RPW + u;
        const int64_t row = r0 + rr;
        if (row >= M) continue;
        const float m = row_absmax<CH>(v[u]);
        // Every one of the 64*CH words of the row is written (ldq4 <= 64*CH): past K the
        // loaded values are 0, so their codes are 0, and no per-word branch is needed.
        if (m == 0.0f) {
#pragma unroll
            for (int c = 0; c < CH; ++c) *word(rr, lane + 64 * c) = 0;
            if (lane == 0) scale[row] = 0.0f;
        } else {
            const float s = m / 127.0f;
            const float inv = 1.0f / s;
#pragma unroll
            for (int c = 0; c < CH; ++c) *word(rr, lane + 64 * c) = pack_codes(v[u][c], inv);
            if (lane == 0) scale[row] = s;
        }
    }
    __syncthreads();
    // piece p = (chunk p / 8, row p % 8): 8 consecutive threads write one whole line
    const int64_t nk32 = ldq >> 5;
    for (int p = threadIdx.x; p < 2 * ldq4; p += NT) {
        const int c = p >> 3, r2 = p & 7;
        if (r0 + r2 < M)
            *reinterpret_cast<int4 *>(q + frag_off(r0 + r2, 16 * (int64_t)c, nk32)) =
                *reinterpret_cast<const int4 *>(lds + c * CP + r2 * 16);
    }
}

// quant_rows_frag of GELUF32(a) (linalg/exp.go:260-263): the codes and scales that
// quant_rows_frag<CH, 1> writes for rows already passed through the GELU, from the
// pre-activation rows. For a linear whose input is GELU's output (FFN-down after FFN-up,
// encoder/bert.go:357-364): FFN-up then runs a bias-only epilogue and this kernel applies
// the GELU where the rows are read anyway, with many wavefronts per SIMD, where the GEMM's
// GELU epilogue issues from about one.
//
// One wavefront per row, 8 rows per block (the code lines of quant_rows_frag: each line
// holds 16 codes of each of the block's 8 rows). Each lane
// evaluates ErfF32's series branch on its 4*CH values without branching (gelu_f32_series4)
// and keeps the pre-activation of every value that needs another branch (|u| >= 1, or
// NaN: the tails). The tails are then settled part by part, PG float4 groups at a time:
// the part goes to a per-wavefront LDS buffer, each lane appends the buffer cells of its
// tail values to a wave-wide list (a loop over the set bits of its mask, so a lane pays
// per tail, not per value), the list is evaluated 64 cells at a time by the branch-free
// gelu_f32_offseries (two rounds interleaved), and the part is read back. A part with no
// tail in the wavefront is skipped. The list holds every cell of a part, so any number of
// tails fits. Same bits as gelu_f32 on every value (the series branch by
// gelu_f32_series4's, every other branch by gelu_f32_offseries's operations), so the
// codes are quant_rows_frag's of the GELU outputs. The kernel is bound by VALU issue (the
// series alone is 27 multiplies and adds per value); measured on MI355X at M = 32768,
// K = 3072, same process, bit-identical: a persistent form that prefetches each
// wavefront's next row (167 VGPRs, one block per CU) ran 160-295 us against 118-207 for
// this one, and the series constants held in SGPRs instead of literals 135 against 118.
//
// Each wavefront's LDS region holds its part buffer (PG float4 groups per lane) and, once
// its tails are settled, its row's codes (CH * 256 bytes), plus a 16-byte pad so that the 8
// regions start in different banks. PG = 4 keeps the block at 49 KB for any CH <= 16: three
// blocks (24 wavefronts) share a CU. Measured on MI355X against code staging shared by the
// block (75 KB, two blocks per CU), M = 32768, K = 3072, same process, bit-identical:
// 101 / 115 / 138 / 192 against 103 / 127 / 156 / 215 us at 0% / 1% / 20% / 67% tails.
constexpr int QG_PG = 4;

template <int CH>
__global__ __launch_bounds__(512) void quant_rows_frag_gelu(const float *__restrict__ a, int8_t *__restrict__ q,
                                                            int64_t ldq, float *__restrict__ scale, int64_t M, int K) {
    constexpr int PG = QG_PG < CH ? QG_PG : CH;
    constexpr int NPART = (CH + PG - 1) / PG;
    static_assert(PG >= 1 && 4 * PG <= 32, "a part's tail bits fit one 32-bit word");
    constexpr int RB = (PG * 1024 > CH * 256 ? PG * 1024 : CH * 256) + 16;  // bytes per wavefront
    __shared__ __attribute__((aligned(16))) int8_t lds[8 * RB];  // part buffers, then codes
    __shared__ uint16_t tl[8][PG * 256];                          // each wavefront's tail cells
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * 8;
    const int64_t row = r0 + wave;
    const int ldq4 = (int)(ldq >> 2);
    // the 32-bit word of codes 4*k4 .. 4*k4+3 of block row rr, in that row's own region
    auto word = [&](int rr, int k4) -> int * { return reinterpret_cast<int *>(lds + rr * RB + k4 * 4); };
    float4 v[CH];
    load_row_raw<CH>(a, min(row, M - 1), K, lane, v);
    if (row < M) {  // uniform across the wavefront
        // Series pass: every value by the series branch; tail values keep their input.
        uint32_t tm[NPART];  // bit 4*(c % PG) + j: value j of float4 c is a tail
#pragma unroll
        for (int p = 0; p < NPART; ++p) tm[p] = 0u;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const f32x4v y = {v[c].x, v[c].y, v[c].z, v[c].w};
            uint32_t t4;
            const f32x4v gy = gelu_f32_series4(y, t4);
            v[c] = make_float4(t4 & 1u ? y.x : gy.x, t4 & 2u ? y.y : gy.y, t4 & 4u ? y.z : gy.z, t4 & 8u ? y.w : gy.w);
            tm[c / PG] |= t4 << (4 * (c % PG));
        }
        // cell (g * 64 + lane) * 4 + j: value j of the part's float4 g
        float *cell = reinterpret_cast<float *>(lds + wave * RB);
        uint16_t *list = tl[wave];
#pragma unroll
        for (int p = 0; p < NPART; ++p) {
            const int c0 = p * PG, ng = (CH - c0) < PG ? (CH - c0) : PG;
            // each lane's place in the list: a prefix sum of the tail counts, bit-sliced
            // over ballots (counts up to 4 * PG <= 32 need 6 bits)
            const int cnt = __builtin_popcount(tm[p]);
            int excl = 0, total = 0;
#pragma unroll
            for (int b = 0; b < 6; ++b) {
                const uint64_t bm = __builtin_amdgcn_ballot_w64((cnt >> b) & 1);
                excl += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bm, 0u)) << b;
                total += __builtin_popcountll(bm) << b;
            }
            if (total == 0) continue;  // uniform
#pragma unroll
            for (int g = 0; g < PG; ++g)
                if (g < ng) *reinterpret_cast<float4 *>(&cell[(g * 64 + lane) * 4]) = v[c0 + g];
            int pos = excl;
            for (uint32_t m = tm[p]; m != 0u; m &= m - 1u, ++pos) {
                const int b = __builtin_ctz(m);
                list[pos] = (uint16_t)(((b >> 2) * 64 + lane) * 4 + (b & 3));
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            for (int base = 0; base < total; base += 128) {
                const int e0 = base + lane, e1 = base + 64 + lane;
                const int i0 = list[min(e0, total - 1)];
                if (base + 64 < total) {
                    const int i1 = list[min(e1, total - 1)];
                    const float g0 = gelu_f32_offseries(cell[i0]);
                    const float g1 = gelu_f32_offseries(cell[i1]);
                    if (e0 < total) cell[i0] = g0;
                    if (e1 < total) cell[i1] = g1;
                } else if (e0 < total) {
                    cell[i0] = gelu_f32_offseries(cell[i0]);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int g = 0; g < PG; ++g)
                if (g < ng) v[c0 + g] = *reinterpret_cast<const float4 *>(&cell[(g * 64 + lane) * 4]);
            // the next part's stores to the buffer (or the codes) come after these loads
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        float m = 0.0f;  // the GELU values are results of arithmetic: quiet NaNs at most
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            m = absmax_step_quiet(m, v[c].x);
            m = absmax_step_quiet(m, v[c].y);
            m = absmax_step_quiet(m, v[c].z);
            m = absmax_step_quiet(m, v[c].w);
        }
        m = wave_absmax(m);
        if (m == 0.0f) {
#pragma unroll
            for (int c = 0; c < CH; ++c) *word(wave, lane + 64 * c) = 0;
            if (lane == 0) scale[row] = 0.0f;
        } else {
            const float s = m / 127.0f;
            const float inv = 1.0f / s;
            if (s >= 1.17549435e-38f) {  // uniform: the row's scale is a normal float (or +inf)
#pragma unroll
                for (int c = 0; c < CH; ++c) *word(wave, lane + 64 * c) = pack_codes_normal(v[c], inv);
            } else {
#pragma unroll
                for (int c = 0; c < CH; ++c) *word(wave, lane + 64 * c) = pack_codes(v[c], inv);
            }
            if (lane == 0) scale[row] = s;
        }
    }
    __syncthreads();
    // piece p = (chunk p / 8, row p % 8): 8 consecutive threads write one whole line
    const int64_t nk32 = ldq >> 5;
    for (int p = threadIdx.x; p < 2 * ldq4; p += 512) {
        const int c = p >> 3, r2 = p & 7;
        if (r0 + r2 < M)
            *reinterpret_cast<int4 *>(q + frag_off(r0 + r2, 16 * (int64_t)c, nk32)) =
                *reinterpret_cast<const int4 *>(lds + r2 * RB + c * 16);
    }
}

// Any K and alignment: one wavefront per row, two passes over the row. FRAG as in
// quant_rows_vec.
template <bool FRAG>
__global__ __launch_bounds__(256) void quant_rows_scalar(const float *__restrict__ a,
                                                         int8_t *__restrict__ q, int64_t ldq,
                                                         float *__restrict__ scale, int64_t M,
                                                         int64_t K) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const float *src = a + row * K;
    const int64_t nk32 = ldq >> 5;
    auto dst = [&](int64_t k) -> int8_t & { return q[FRAG ? frag_off(row, k, nk32) : row * ldq + k]; };
    float m = 0.0f;
    for (int64_t k = lane; k < K; k += 64) m = absmax_step(m, src[k]);
    m = wave_absmax(m);
    if (m == 0.0f) {
        for (int64_t k = lane; k < ldq; k += 64) dst(k) = 0;
        if (lane == 0) scale[row] = 0.0f;
        return;
    }
    const float s = m / 127.0f;
    const float inv = 1.0f / s;
    for (int64_t k = lane; k < K; k += 64) dst(k) = (int8_t)quant_code(src[k], inv);
    for (int64_t k = K + lane; k < ldq; k += 64) dst(k) = 0;
    if (lane == 0) scale[row] = s;
}

// ----------------------------------------------------------------------------
// Epilogue of one output element (linalg/quant.go:291-295, encoder/linalg.go:130-140,
// linalg/exp.go:260-263): float32(acc)*aS*wS left to right, +0 for an all-zero
// activation row, then the bias as a separate rounding, then GELU. Callers without a
// bias pass b = -0.0f: y + (-0.0f) == y bit for bit for every y (-0 stays -0, NaN
// stays NaN), so the add needs no per-element select.
constexpr float kNoBias = -0.0f;

__device__ __forceinline__ float dequant(int acc, float as, float ws, float b) {
    const float y = (as == 0.0f) ? 0.0f : (float)acc * as * ws;
    return y + b;
}

template <int EPI>
__device__ __forceinline__ float epilogue(int acc, float as, float ws, float b) {
    float y = dequant(acc, as, ws, b);
    if (EPI == EPI_F32_GELU) y = gelu_f32(y);
    return y;
}

// Row of a 32x32 i32 MFMA accumulator held by lane `lane` in register r.
__device__ __forceinline__ int acc_row(int r, int lane) {
    return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}

// Map the hardware's round-robin XCD dispatch (block b runs on XCD b % 8) to a
// contiguous range of logical tiles per XCD, so tiles that share an A row-block
// run on the same XCD and share its L2.
__device__ __forceinline__ int xcd_logical_tile(int pid, int nblocks) {
    const int xcd = pid & 7, idx = pid >> 3;
    const int q = nblocks >> 3, r = nblocks & 7;
    return (xcd < r) ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

// ----------------------------------------------------------------------------
// Tiled GEMM. Block tile BM x BN, K stage of 64, 4 waves in a 2x2 grid, each wave a
// (BM/2) x (BN/2) tile of 32x32x32 i8 MFMA accumulators.
//
// LDS holds each stage as 1 KiB "fragments" in MFMA operand order (lane l's 16 bytes
// at l*16): A fragment (rb, s) = rows rb*32.., k 32*s..; W fragment (nb, s) likewise.
// Every ds_read_b128 is 64 lanes x 16 contiguous bytes, so fragment reads are free of
// bank conflicts with no swizzle. W arrives already in this order (pre-swizzled at
// registration); A is row-major in HBM and each lane fetches its 16 bytes from row
// (lane & 31), k offset 16*(lane >> 5).
//
// Pipeline: stage k+2 in flight to VGPRs, stage k+1 in the other LDS buffer, stage k
// computed; the fragments of the second k-step of a stage are read while the MFMAs
// of the first run, and the next stage's first fragments while the second runs.
template <int BM, int BN, int EPI, int MINB>
__global__ __launch_bounds__(256, MINB) void gemm_w8a8(
    const int8_t *__restrict__ A, int64_t lda, const int8_t *__restrict__ Wf,
    const float *__restrict__ aS, const float *__restrict__ wS, const float *__restrict__ bias,
    void *__restrict__ out, int64_t ldo, int M, int N, int Kp, int tilesN) {
    constexpr int WTM = BM / 2, WTN = BN / 2;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int CA = BM / 16, CB = BN / 16, C = CA + CB;  // 1 KiB chunks per stage
    constexpr int LPW = C / 4;                               // chunks each wave moves
    static_assert(C % 4 == 0 && TM >= 1 && TN >= 1, "tile shape");
    constexpr int STAGE = C * 1024;
    __shared__ __attribute__((aligned(1024))) int8_t smem[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int logical = xcd_logical_tile(blockIdx.x, gridDim.x);
    const int m0 = (logical / tilesN) * BM, n0 = (logical % tilesN) * BN;
    const int nk = Kp >> 6, nk32 = Kp >> 5;

    // Source of this wave's chunks at k = 0; chunk c < CA is A (rb = c/2, s = c%2).
    const int8_t *src[LPW];
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
        const int c = wave + 4 * i;
        if (c < CA) {
            const int rb = c >> 1, s = c & 1;
            const int gr = min(m0 + rb * 32 + (lane & 31), M - 1);  // rows past M re-read M-1, never stored
            src[i] = A + (int64_t)gr * lda + 32 * s + 16 * (lane >> 5);
        } else {
            const int cb = c - CA, nb = cb >> 1, s = cb & 1;
            src[i] = Wf + ((int64_t)((n0 >> 5) + nb) * nk32 + s) * 1024 + lane * 16;
        }
    }
    i32x4 R[LPW];
    auto gload = [&](int kt) {
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int c = wave + 4 * i;
            const int64_t koff = (c < CA) ? (int64_t)kt * 64 : (int64_t)kt * 2048;
            R[i] = *reinterpret_cast<const i32x4 *>(src[i] + koff);
        }
    };
    auto swrite = [&](int slot) {
        int8_t *base = smem + slot * STAGE + lane * 16;
#pragma unroll
        for (int i = 0; i < LPW; ++i) *reinterpret_cast<i32x4 *>(base + (wave + 4 * i) * 1024) = R[i];
    };
    const int aoff = (wm * WTM >> 5) * 2048 + lane * 16;
    const int boff = CA * 1024 + (wn * WTN >> 5) * 2048 + lane * 16;
    auto read_frags = [&](int slot, int s, i32x4 *af, i32x4 *bf) {
        const int8_t *base = smem + slot * STAGE + s * 1024;
#pragma unroll
        for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const i32x4 *>(base + aoff + i * 2048);
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const i32x4 *>(base + boff + j * 2048);
    };

    i32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    gload(0);
    swrite(0);
    if (nk > 1) gload(1);
    __syncthreads();
    i32x4 a0[TM], b0[TN], a1[TM], b1[TN];
    read_frags(0, 0, a0, b0);
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        read_frags(cur, 1, a1, b1);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0[i], b0[j], acc[i][j], 0, 0, 0);
        if (kt + 1 < nk) {
            swrite(cur ^ 1);
            if (kt + 2 < nk) gload(kt + 2);
            __syncthreads();
            read_frags(cur ^ 1, 0, a0, b0);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1[i], b1[j], acc[i][j], 0, 0, 0);
    }

    // Epilogue straight from the accumulators: for a fixed register, lanes 0-31
    // and 32-63 each write 32 consecutive outputs (128 bytes) of one row.
    const bool has_bias = bias != nullptr;
    float ws[TN], bb[TN];
    int cols[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        cols[j] = n0 + wn * WTN + j * 32 + (lane & 31);
        ws[j] = cols[j] < N ? wS[cols[j]] : 0.0f;
        bb[j] = (has_bias && cols[j] < N) ? bias[cols[j]] : kNoBias;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + wm * WTM + i * 32 + acc_row(r, lane);
            if (row >= M) continue;
            if (EPI == EPI_I32) {
                int *o = reinterpret_cast<int *>(out) + (int64_t)row * ldo;
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    if (cols[j] < N) o[cols[j]] = acc[i][j][r];
            } else {
                const float as = aS[row];
                float *o = reinterpret_cast<float *>(out) + (int64_t)row * ldo;
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    if (cols[j] < N) o[cols[j]] = epilogue<EPI>(acc[i][j][r], as, ws[j], bb[j]);
            }
        }
    }
}

// ----------------------------------------------------------------------------
// Small-M variant (M <= 32) on codes already quantized (row-major, pitch lda): HBM-bound
// on the weight stream, so every weight byte is read once and the M tile (zero-padded to
// 32 rows) rides along in the MFMA. The grid is (N/32 channel groups) x (M/8 row groups):
// each 8-wave workgroup splits K over its waves for its 32 output channels, each wave
// issuing its weight and activation fragments (NB at a time: nk32 <= 8 NB needs one
// batch) before its MFMAs, so a call costs about one HBM round trip; the exact int32
// partials of the group's 8 rows only are added through LDS and stored. Lanes of rows
// outside the group load the group's first row (their sums are dropped). Splitting the
// rows over workgroups, where each workgroup used to reduce and store all 32 rows of its
// channels: 4.42 -> 2.93 us per call at M = 16, K = 768, N = 768 and 4.64 -> 3.12 us at
// N = 3072 (MI355X, graph replay over cold weights, bit-identical).
constexpr int GV_WAVES = 8, GV_ROWS = 8;

template <int EPI, int NB>
__global__ __launch_bounds__(64 * GV_WAVES) void gemv_w8a8(
    const int8_t *__restrict__ A, int64_t lda, const int8_t *__restrict__ Wf,
    const float *__restrict__ aS, const float *__restrict__ wS, const float *__restrict__ bias,
    void *__restrict__ out, int64_t ldo, int M, int N, int Kp) {
    __shared__ int red[GV_WAVES * GV_ROWS * 32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nb = blockIdx.x, rg = blockIdx.y, nk32 = Kp >> 5;
    const int q = rg & 3, r = lane & 31;  // the group's rows 8q .. 8q + 7 of the 32-row tile
    const int8_t *arow = A + (int64_t)min((r >> 3) == q ? r : 8 * q, M - 1) * lda + (lane >> 5) * 16;
    const int8_t *wfr = Wf + (int64_t)nb * nk32 * 1024 + lane * 16;

    i32x16 acc;
#pragma unroll
    for (int k = 0; k < 16; ++k) acc[k] = 0;
    for (int k0 = wave; k0 < nk32; k0 += GV_WAVES * NB) {
        // this wave's fragments k0, k0 + GV_WAVES, ...: loads first (clamped to the last
        // fragment, whose extra copies are skipped below), then the MFMAs
        i32x4 a[NB], b[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int kk = min(k0 + u * GV_WAVES, nk32 - 1);
            a[u] = *reinterpret_cast<const i32x4 *>(arow + kk * 32);
            b[u] = *reinterpret_cast<const i32x4 *>(wfr + (int64_t)kk * 1024);
        }
#pragma unroll
        for (int u = 0; u < NB; ++u)
            if (k0 + u * GV_WAVES < nk32) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[u], b[u], acc, 0, 0, 0);
    }
    // rows 8q .. 8q + 7 are registers 4q .. 4q + 3 (acc_row(4q + i, lane) = 8q + 4 (lane / 32) + i)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * GV_ROWS + (lane >> 5) * 4 + i) * 32 + r] = acc[4 * q + i];
    __syncthreads();
    if (tid < GV_ROWS * 32) {
        const int i = tid >> 5, c = tid & 31;
        int sum = 0;
#pragma unroll
        for (int w = 0; w < GV_WAVES; ++w) sum += red[(w * GV_ROWS + i) * 32 + c];
        const int row = rg * GV_ROWS + i, col = nb * 32 + c;
        if (row < M && col < N) {
            if (EPI == EPI_I32) {
                reinterpret_cast<int *>(out)[(int64_t)row * ldo + col] = sum;
            } else {
                const float bb = bias != nullptr ? bias[col] : kNoBias;
                reinterpret_cast<float *>(out)[(int64_t)row * ldo + col] = epilogue<EPI>(sum, aS[row], wS[col], bb);
            }
        }
    }
}

// gemv_w8a8 with the per-token quantization of its (at most 32) activation rows done in
// the kernel, so a small-M linear is one launch. The grid is (N/32 channel groups) x
// (M/8 row groups): each 8-wave workgroup quantizes only its GVQ_ROWS rows, one per wave,
// with quant_rows_vec's arithmetic (the absmax of |v| over a row does not depend on the
// order it is taken in, then s = m/127, 1/s and pack_codes) into LDS in the A-operand
// fragment layout (frag_off), runs gemv_w8a8's K split over its 8 waves for its 32 output
// channels with the A fragments read from LDS, and reduces and stores only its rows.
// Codes, scales and outputs are those of quant_rows_vec + gemv_w8a8 (int32 partial sums
// are exact in any order).
//
// Splitting the rows over workgroups, not quantizing every row in every workgroup, is what
// makes the launch short: the per-element quantization (~15 VALU instructions) was the
// longest phase, measured on MI355X by s_memtime stamps in a copy of the earlier kernel
// (M = 16, K = 768: 2.4K of 8.2K shader cycles per wave with all 16 rows in each of the
// 24 workgroups). Per call in graph replay, cold weights: 5.41 us before, 3.45 us with 4
// rows per workgroup and 3.37 us with 8 (N = 768); 5.58, 4.24 and 3.54 us (N = 3072); M =
// 32, N = 768: 7.7, 3.5 and 3.4 us. The row groups' workgroups read the same weight
// fragments (block ids nb + k * N/32 share an XCD's L2 when N/32 is a multiple of 8), so
// HBM still streams each weight about once.
//
// Each row is held in registers (K <= 256 * QCH) with all of a wave's loads in flight and
// unconditional (a lane past the row re-reads its last float4 and zeroes it by a bit mask),
// and the wave's weight fragments (at most QCH: Kp <= 256 * QCH) are loaded before the
// quantization. Rows of the 32-row MFMA tile outside the group are never written in LDS:
// their sums are computed and dropped. K % 4 == 0, K <= GVQ_MAX_K, 16-byte aligned rows
// (pitch K); dynamic LDS gvq_lds_bytes(Kp) (136 KiB at K = 4096).
constexpr int GVQ_MAX_K = 4096;
constexpr int GVQ_ROWS = 8, GVQ_WAVES = 8;
__host__ __device__ inline int gvq_lds_bytes(int Kp) { return Kp * 32 + GVQ_WAVES * GVQ_ROWS * 32 * 4 + 16; }

template <int EPI, int QCH>
__global__ __launch_bounds__(64 * GVQ_WAVES) void gemv_w8a8_q(
    const float *__restrict__ a, const int8_t *__restrict__ Wf, const float *__restrict__ wS,
    const float *__restrict__ bias, void *__restrict__ out, int64_t ldo, int M, int N, int K, int Kp) {
    static_assert(GVQ_ROWS == 8 && GVQ_ROWS <= GVQ_WAVES, "one row per wave, row groups of one accumulator register quad");
    extern __shared__ __attribute__((aligned(16))) int8_t gvq[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nb = blockIdx.x, rg = blockIdx.y, nk32 = Kp >> 5, K4 = K >> 2, Kp4 = Kp >> 2;
    int *red = reinterpret_cast<int *>(gvq + Kp * 32);
    float *s_as = reinterpret_cast<float *>(gvq + Kp * 32 + GVQ_WAVES * GVQ_ROWS * 32 * 4);
    const int row = rg * GVQ_ROWS + wave;  // the row this wave quantizes (waves < GVQ_ROWS)
    const bool qwave = wave < GVQ_ROWS && row < M;
    float4 v[QCH];
    if (qwave) {
        const i32x4 *src = reinterpret_cast<const i32x4 *>(a + (int64_t)row * K);
#pragma unroll
        for (int c = 0; c < QCH; ++c) {
            const int k4 = lane + 64 * c;
            const i32x4 t = src[min(k4, K4 - 1)];
            const int keep = k4 < K4 ? -1 : 0;
            v[c] = make_float4(__int_as_float(t.x & keep), __int_as_float(t.y & keep), __int_as_float(t.z & keep),
                               __int_as_float(t.w & keep));
        }
    }
    // this wave's weight fragments wave, wave + 8, ... (clamped; extra copies skipped below)
    const int8_t *wfr = Wf + (int64_t)nb * nk32 * 1024 + lane * 16;
    i32x4 b[QCH];
#pragma unroll
    for (int u = 0; u < QCH; ++u)
        b[u] = *reinterpret_cast<const i32x4 *>(wfr + (int64_t)min(wave + u * GVQ_WAVES, nk32 - 1) * 1024);
    if (qwave) {
        float m = 0.0f;
#pragma unroll
        for (int c = 0; c < QCH; ++c) {
            m = absmax_step(m, v[c].x);
            m = absmax_step(m, v[c].y);
            m = absmax_step(m, v[c].z);
            m = absmax_step(m, v[c].w);
        }
        m = wave_absmax(m);
        const bool zero = m == 0.0f;
        const float sc = zero ? 0.0f : m / 127.0f;
        const float inv = zero ? 0.0f : 1.0f / sc;
#pragma unroll
        for (int c = 0; c < QCH; ++c) {
            const int k4 = lane + 64 * c;
            if (k4 < Kp4)
                *reinterpret_cast<int *>(gvq + frag_off(row & 31, 4 * (int64_t)k4, nk32)) =
                    (!zero && k4 < K4) ? pack_codes(v[c], inv) : 0;
        }
        if (lane == 0) s_as[wave] = sc;
    }
    __syncthreads();
    i32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0;
#pragma unroll
    for (int u = 0; u < QCH; ++u) {
        const int kk = wave + u * GVQ_WAVES;
        if (kk < nk32) {
            const i32x4 av = *reinterpret_cast<const i32x4 *>(gvq + kk * 1024 + lane * 16);
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b[u], acc, 0, 0, 0);
        }
    }
    // the group's rows 8q .. 8q + 7 of the 32-row tile are registers 4q .. 4q + 3
    // (acc_row(4q + i, lane) = 8q + 4 (lane / 32) + i)
    const int q = rg & 3;
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * GVQ_ROWS + (lane >> 5) * 4 + i) * 32 + (lane & 31)] = acc[4 * q + i];
    __syncthreads();
    if (tid < GVQ_ROWS * 32) {
        const int i = tid >> 5, c = tid & 31;
        int sum = 0;
#pragma unroll
        for (int w = 0; w < GVQ_WAVES; ++w) sum += red[(w * GVQ_ROWS + i) * 32 + c];
        const int orow = rg * GVQ_ROWS + i, col = nb * 32 + c;
        if (orow < M && col < N) {
            const float ws = wS[col];
            const float bb = bias != nullptr ? bias[col] : kNoBias;
            reinterpret_cast<float *>(out)[(int64_t)orow * ldo + col] = epilogue<EPI>(sum, s_as[i], ws, bb);
        }
    }
}

// Small-M variant for wide N (many output-channel groups, e.g. an int8 ANN index of
// 10^5..10^6 rows): one wavefront per 32 output channels with the whole K, so no
// cross-wave reduction, no LDS and no barrier; the weight stream is the only traffic that
// matters, read with nontemporal loads (each byte is used once), and every wave keeps up
// to GVW_BATCH fragment loads in flight. On MI355X this streams a 2^20 x 384 index at
// ~7 TB/s for one query; 8-fragment batches are ~5% slower, plain loads ~15%.
constexpr int GVW_WAVES = 4, GVW_BATCH = 12;

template <int EPI>
__global__ __launch_bounds__(64 * GVW_WAVES) void gemv_w8a8_wide(
    const int8_t *__restrict__ A, int64_t lda, const int8_t *__restrict__ Wf,
    const float *__restrict__ aS, const float *__restrict__ wS, const float *__restrict__ bias,
    void *__restrict__ out, int64_t ldo, int M, int N, int Kp) {
    const int lane = threadIdx.x & 63;
    const int cg = blockIdx.x * GVW_WAVES + (threadIdx.x >> 6);  // this wave's 32-channel group
    if (cg * 32 >= N) return;
    const int nk32 = Kp >> 5;
    const int8_t *arow = A + (int64_t)min(lane & 31, M - 1) * lda + (lane >> 5) * 16;
    const int8_t *wfr = Wf + (int64_t)cg * nk32 * 1024 + lane * 16;
    i32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0;
    for (int k0 = 0; k0 < nk32; k0 += GVW_BATCH) {
        i32x4 a[GVW_BATCH], b[GVW_BATCH];
#pragma unroll
        for (int u = 0; u < GVW_BATCH; ++u) {
            const int kk = min(k0 + u, nk32 - 1);
            a[u] = *reinterpret_cast<const i32x4 *>(arow + kk * 32);
            b[u] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(wfr + (int64_t)kk * 1024));
        }
#pragma unroll
        for (int u = 0; u < GVW_BATCH; ++u)
            if (k0 + u < nk32) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[u], b[u], acc, 0, 0, 0);
    }
    const int col = cg * 32 + (lane & 31);
    if (col >= N) return;
    const float ws = wS[col];
    const float bb = bias != nullptr ? bias[col] : kNoBias;
    // nontemporal stores: the scores are written once and not read here (M = 16 over a
    // 2^20 x 384 index: 89.6 -> 83.7 us on MI355X; M = 1 unchanged)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = acc_row(r, lane);
        if (row >= M) continue;
        if (EPI == EPI_I32)
            __builtin_nontemporal_store(acc[r], reinterpret_cast<int *>(out) + (int64_t)row * ldo + col);
        else
            __builtin_nontemporal_store(epilogue<EPI>(acc[r], aS[row], ws, bb),
                                        reinterpret_cast<float *>(out) + (int64_t)row * ldo + col);
    }
}

}  // namespace enchip
