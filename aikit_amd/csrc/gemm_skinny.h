// gemm_skinny.h -- W8A8 for a few rows against very many output channels with a short K:
// ann.FlatI8 scoring (M queries x an index of n rows, ann/backend.go:16-60) and its
// fused top-k. gemm_w8a8_skinny.
//
// The persistent tiled kernel (gemm_persistent.h) streams the weights once per 128-row
// block, and at a short K each tile brings only its ring's stages of weights in flight: at
// M = 256, K = 384, N = 2^20 it read the index at 1.9 TB/s. Here:
//   * each workgroup copies the codes of all M rows (MB blocks of 32 rows, MB x NK KiB in
//     MFMA operand order) into LDS once;
//   * each of its waves walks 32-channel groups (group g, then g + the grid's wave count,
//     ...). A group's NK weight fragments (1 KiB each, fragment-major) go HBM ->
//     registers, and fragment kk is reloaded with the next group's as soon as this
//     group's MB MFMAs on it are issued, so a group of loads is always in flight behind
//     the MFMAs;
//   * per group, MB x NK v_mfma_i32_32x32x32_i8 (one per row block and K step) read
//     their A fragments from LDS;
//   * the epilogue works on the accumulators in place (a lane holds one channel of 16
//     rows per row block): EPI_F32 stores the dequantized values (32 lanes write 128
//     contiguous bytes of a row); EPI_TOPK compares them with the rows' bounds and lists
//     the few at or above them (TopkSink), storing nothing else.
// Numerics: the exact int32 dot and the dequantization of the other kernels, so the
// outputs are bit-identical to theirs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "gemm_persistent.h"
#include "kernels.h"
#include "topk.h"

#pragma clang fp contract(off)

namespace enchip {

constexpr int SK_WAVES = 8;  // waves per workgroup, one workgroup per CU
constexpr int SK_LCAP = 16;  // EPI_TOPK: candidates per row a workgroup holds in LDS

// MB: row blocks staged (32 * MB >= M; fragment-major A is read up to 32 * MB rows, which
// its buffer holds: it is padded to a multiple of 128 rows and MB is 4 or 8). NK = Kp / 32.
// AF: A is fragment-major ([M/32][NK][1024]); otherwise row-major int8 at pitch lda (a
// multiple of 16, at least Kp, zero past K).
template <int MB, int NK, int EPI, bool AF>
__global__ __launch_bounds__(64 * SK_WAVES, 1) void gemm_w8a8_skinny(
    const int8_t *__restrict__ A, int64_t lda, const int8_t *__restrict__ Wf, const float *__restrict__ aS,
    const float *__restrict__ wS, const float *__restrict__ bias, float *__restrict__ out, int64_t ldo, int M,
    int N, TopkSink sink) {
    static_assert(EPI == EPI_F32 || EPI == EPI_TOPK, "f32 scores or their top-k candidates");
    __shared__ i32x4 s_a[MB * NK * 64];
    __shared__ __attribute__((aligned(16))) float s_as[MB * 32];
    __shared__ uint64_t s_thr[EPI == EPI_TOPK ? MB * 32 : 1];
    __shared__ __attribute__((aligned(16))) float s_tf[EPI == EPI_TOPK ? MB * 32 : 1];  // bound scores
    // EPI_TOPK: the workgroup's candidates, per row, until its flush at the end. A global
    // atomic that returns its value would wait (in-order vmcnt) for every weight load in
    // flight behind it, a full memory latency per group with a candidate; LDS atomics
    // count on lgkmcnt.
    constexpr int LC = EPI == EPI_TOPK ? MB * 32 : 1;
    __shared__ unsigned s_cnt[LC];
    __shared__ uint64_t s_ckey[LC * SK_LCAP];
    __shared__ float s_cscore[LC * SK_LCAP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // A fragment f = rb * NK + kk holds, in lane l, row 32 rb + (l & 31), bytes
    // 32 kk + 16 (l >> 5) .. + 15. Rows past M: padding (fragment-major) or row M - 1.
    for (int i = tid; i < MB * NK * 64; i += 64 * SK_WAVES) {
        if (AF) {
            s_a[i] = reinterpret_cast<const i32x4 *>(A)[i];
        } else {
            const int l = i & 63, f = i >> 6, rb = f / NK, kk = f - rb * NK;
            const int row = min(rb * 32 + (l & 31), M - 1);
            s_a[i] = *reinterpret_cast<const i32x4 *>(A + (int64_t)row * lda + kk * 32 + (l >> 5) * 16);
        }
    }
    for (int r = tid; r < MB * 32; r += 64 * SK_WAVES) {
        s_as[r] = aS[min(r, M - 1)];
        if (EPI == EPI_TOPK) {
            const uint64_t t = sink.thr[min(r, M - 1)];
            s_thr[r] = t;
            s_tf[r] = t == 0 ? -INFINITY : topk_key_score(t);  // -inf: no bound, every non-NaN score
            s_cnt[r] = 0;
        }
    }
    __syncthreads();

    const int groups = (N + 31) >> 5, stride = gridDim.x * SK_WAVES;
    int g = blockIdx.x * SK_WAVES + wave;
    if (EPI != EPI_TOPK && g >= groups) return;  // no barrier follows
    const int8_t *wl = Wf + lane * 16;
    auto wfrag = [&](int grp, int kk) {
        return __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(wl + ((int64_t)grp * NK + kk) * 1024));
    };
    auto chan = [&](int grp) { return min(grp * 32 + (lane & 31), N - 1); };
    const bool has_bias = bias != nullptr;
    // The weight ring: D groups of NK fragments, each slot refilled with the group D ahead
    // while its current group's MFMAs issue. Two slots where the registers allow (the
    // candidate epilogue, up to 4 row blocks and 12 K steps): with one, 2 waves per SIMD x
    // 12 KiB in flight left the index streaming at ~3 TB/s (latency-bound). The f32
    // epilogue keeps one: its stores, not the index, bound it.
    constexpr int D = EPI == EPI_TOPK && MB <= 4 && NK <= 12 ? 2 : 1;
    i32x4 b[D][NK];
    float wsr[D], bbr[D];
    const int n = g < groups ? (groups - 1 - g) / stride + 1 : 0;  // this wave's groups
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const int gd = min(g + d * stride, groups - 1);  // in bounds also past the wave's groups
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) b[d][kk] = wfrag(gd, kk);
        wsr[d] = wS[chan(gd)];
        bbr[d] = has_bias ? bias[chan(gd)] : kNoBias;
    }

    // Group i of this wave from ring slot SLOT: its MFMAs (each K step's MB A fragments read
    // from LDS first, then its MB MFMAs, then, with NEXT, the fragment of that step of group
    // i + D: a fixed order, so only one step's A fragments are live), then its epilogue.
    auto group = [&](auto slot_c, auto next_c, int i) {
        constexpr int SLOT = decltype(slot_c)::value;
        constexpr bool NEXT = decltype(next_c)::value;
        const int g = blockIdx.x * SK_WAVES + wave + i * stride, gn = g + D * stride;
        const float ws_c = wsr[SLOT], bb_c = bbr[SLOT];
        if (NEXT) {
            wsr[SLOT] = wS[chan(gn)];
            bbr[SLOT] = has_bias ? bias[chan(gn)] : kNoBias;
        }
        i32x16 acc[MB];
#pragma unroll
        for (int rb = 0; rb < MB; ++rb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[rb][r] = 0;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
            i32x4 af[MB];
#pragma unroll
            for (int rb = 0; rb < MB; ++rb) af[rb] = s_a[(rb * NK + kk) * 64 + lane];
#pragma unroll
            for (int rb = 0; rb < MB; ++rb)
                acc[rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[rb], b[SLOT][kk], acc[rb], 0, 0, 0);
            if (NEXT) b[SLOT][kk] = wfrag(gn, kk);
            __builtin_amdgcn_sched_group_barrier(0x100, MB, 0);  // LDS reads
            __builtin_amdgcn_sched_group_barrier(0x008, MB, 0);  // MFMAs
            if (NEXT) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // the VMEM load
        }

        const int col = g * 32 + (lane & 31);
        if (col >= N) return;  // the ragged last group
        // The output rows' offsets and the candidate lists' addresses depend only on the
        // lane: left to itself the compiler computes all MB x 16 of them once, before the
        // group loop, and spills. An opaque copy of the pitch (and of the row in the rare
        // path) keeps each one next to its use.
        int64_t ld = ldo;
        asm volatile("" : "+s"(ld));
        if constexpr (EPI == EPI_F32) {
#pragma unroll
            for (int rb = 0; rb < MB; ++rb)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int row0 = rb * 32 + 8 * q + 4 * (lane >> 5);  // rows row0 .. row0 + 3
                    const float4 as4 = *reinterpret_cast<const float4 *>(&s_as[row0]);
                    const float asv[4] = {as4.x, as4.y, as4.z, as4.w};
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (row0 + u < M)
                            __builtin_nontemporal_store(dequant(acc[rb][4 * q + u], asv[u], ws_c, bb_c),
                                                        out + (int64_t)(row0 + u) * ld + col);
                }
        } else {
            const uint32_t lo = 0xffffffffu - (uint32_t)col;
#pragma unroll
            for (int rb = 0; rb < MB; ++rb) {
                // bit 4q + u: value acc[rb][4q + u] is at or above its row's bound score (a
                // NaN is not), which a kept key needs; only ties at that score need the
                // index test below
                uint32_t pass = 0;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int row0 = rb * 32 + 8 * q + 4 * (lane >> 5);
                    const float4 as4 = *reinterpret_cast<const float4 *>(&s_as[row0]);
                    const float4 tf4 = *reinterpret_cast<const float4 *>(&s_tf[row0]);
                    const float asv[4] = {as4.x, as4.y, as4.z, as4.w}, tfv[4] = {tf4.x, tf4.y, tf4.z, tf4.w};
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        pass |= dequant(acc[rb][4 * q + u], asv[u], ws_c, bb_c) >= tfv[u] ? 1u << (4 * q + u) : 0u;
                }
                if (pass != 0u) {  // rare: the exact key test
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        if (!((pass >> r) & 1u)) continue;
                        int row = rb * 32 + acc_row(r, lane);
                        asm volatile("" : "+v"(row));
                        const float x = dequant(acc[rb][r], s_as[row], ws_c, bb_c);
                        const uint64_t t = s_thr[row];
                        const float tf = topk_key_score(t);
                        // key >= t: the score above t's, or equal and the index no larger;
                        // t == 0 keeps every non-NaN score
                        const bool in = row < M && (t == 0 || x > tf || (x == tf && lo >= (uint32_t)t)) && x == x;
                        if (in) {
                            const uint64_t key = ((uint64_t)topk_order(x) << 32) | lo;
                            const unsigned p = atomicAdd(&s_cnt[row], 1u);
                            if (p < (unsigned)SK_LCAP) {
                                s_ckey[row * SK_LCAP + p] = key;
                                s_cscore[row * SK_LCAP + p] = x;
                            } else {  // the row's LDS slots are full: straight to its list
                                const unsigned pos = atomicAdd(&sink.count[row], 1u);
                                if (pos < (unsigned)sink.cap) {
                                    const int64_t at = (int64_t)row * sink.cap + pos;
                                    sink.key[at] = key;
                                    sink.score[at] = x;
                                }
                            }
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);  // one row block at a time
            }
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, D - 1>;
    using T = std::true_type;
    using F = std::false_type;
    int i = 0;
    if constexpr (D == 2) {
        for (; i + 3 < n; i += 2) {
            group(S0{}, T{}, i);
            group(S1{}, T{}, i + 1);
        }
        if (n - i == 3) {
            group(S0{}, T{}, i);
            group(S1{}, F{}, i + 1);
            group(S0{}, F{}, i + 2);
        } else if (n - i == 2) {
            group(S0{}, F{}, i);
            group(S1{}, F{}, i + 1);
        } else if (n - i == 1) {
            group(S0{}, F{}, i);
        }
    } else {
        for (; i + 1 < n; ++i) group(S0{}, T{}, i);
        if (n - i == 1) group(S0{}, F{}, i);
    }
    if constexpr (EPI == EPI_TOPK) {
        // flush: one global atomic per row that holds candidates reserves their places
        __syncthreads();
        for (int r = tid; r < M && r < MB * 32; r += 64 * SK_WAVES) {
            const unsigned n = min(s_cnt[r], (unsigned)SK_LCAP);
            if (n == 0) continue;
            const unsigned base = atomicAdd(&sink.count[r], n);
            for (unsigned i = 0; i < n; ++i)
                if (base + i < (unsigned)sink.cap) {
                    const int64_t at = (int64_t)r * sink.cap + base + i;
                    sink.key[at] = s_ckey[r * SK_LCAP + i];
                    sink.score[at] = s_cscore[r * SK_LCAP + i];
                }
        }
    }
}

}  // namespace enchip
