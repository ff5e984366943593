// topk.h -- the k best scores of each row on the device: ann.I8TopKIndex.TopKBatch's
// selection (ann/backend.go:46-55), rank-identical to ScoreBatch + FlatI8.topHits
// (ann/flat_i8.go:208-242): score descending, ties broken by ascending index
// (topk.Cmp, topk/cmp.go:15-27), NaN scores never retained (topk.Selector.Push,
// topk/topk.go:85-100).
//
// Each candidate is one unique 64-bit key that orders exactly like that rule:
//   high 32 bits: the score's bits mapped to an unsigned order (negatives flipped, the
//                 sign bit set on non-negatives; -0 taken as +0, since the reference
//                 compares float64 values and -0 == +0),
//   low 32 bits:  0xffffffff - index (a lower index is a larger key).
// Key 0 is never a valid key and marks "no candidate" (a NaN score, or padding).
//
// Two stages, so the M x N score matrix is read from device memory once:
//   topk_chunk_wide (k <= 64): one 256-thread workgroup per (row, 8192-score chunk)
//     selects the k largest keys of its chunk and writes them as the chunk's k candidates,
//     by a bound from the per-thread maxima and maxima of the few keys above it, comparing
//     the scores as floats and building keys only for those it keeps. On long rows it
//     first runs on each row's first TOPK_SAMPLE_CHUNKS chunks; topk_thresh takes the k-th
//     largest of their keys as a lower bound of the row's k-th largest key; every other
//     chunk then writes its keys at or above that bound when there are at most k of them
//     (no selection), else selects its k largest.
//   topk_chunk (k > 64): the same contract over 4096-score chunks by a radix select over
//     the keys held in registers (8 bits a pass, LDS histogram).
//   topk_merge: one workgroup per row selects the k largest of the row's candidates the
//     same way (maxima in registers when k <= 64 and there are at most 4096 candidates, or
//     8192 for k > 32; else a radix select over them in memory and a bitonic sort in LDS)
//     and writes indices and scores in order.
// Keys are unique, so the radix select finds the k-th largest key exactly and the
// selected set does not depend on the order of anything; outputs are deterministic.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace enchip {

constexpr int TOPK_CHUNK = 4096;  // scores per stage-1 workgroup
constexpr int TOPK_MAX_K = 1024;  // largest k (the merge sorts it in LDS)

// The key's high half from a score's bits: unsigned order, 0 for NaN (never retained),
// -0 taken as +0.
__device__ __forceinline__ uint32_t topk_order_bits(uint32_t u) {
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0;  // NaN
    if (a == 0) return 0x80000000u;   // +-0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint32_t topk_order(float s) { return topk_order_bits(__float_as_uint(s)); }

__device__ __forceinline__ uint64_t topk_key(float s, int64_t index) {
    const uint32_t u = topk_order(s);
    return u ? ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - (uint32_t)index) : 0;
}

__device__ __forceinline__ int64_t topk_index(uint64_t key) { return (int64_t)(0xffffffffu - (uint32_t)key); }

// The smallest key among the block's `want` largest nonzero keys (keys held EPT per
// thread, all distinct), or 1 when the block has at most `want` nonzero keys (every
// nonzero key qualifies). 256 threads; hist is 256 LDS counters, bcast 2 LDS words.
template <int EPT>
__device__ uint64_t radix_threshold(const uint64_t (&key)[EPT], int want, unsigned *hist, uint64_t *bcast) {
    const int tid = threadIdx.x, lane = tid & 63;
    // count the nonzero keys
    if (tid == 0) hist[0] = 0;
    __syncthreads();
    int mine = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) mine += key[j] != 0;
    atomicAdd(&hist[0], (unsigned)mine);
    __syncthreads();
    const int valid = (int)hist[0];
    __syncthreads();
    if (valid <= want) return 1;
    uint64_t prefix = 0, mask = 0;
    int remaining = want;
    for (int shift = 56; shift >= 0; shift -= 8) {
        hist[tid] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if (key[j] != 0 && (key[j] & mask) == prefix) atomicAdd(&hist[(key[j] >> shift) & 255u], 1u);
        __syncthreads();
        if (tid < 64) {
            // lane l holds digits 255-4l .. 252-4l (descending); find the digit where
            // the running count from the top reaches `remaining`
            unsigned c[4], s = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                c[i] = hist[255 - 4 * lane - i];
                s += c[i];
            }
            unsigned incl = s;  // inclusive prefix over lanes (descending digits)
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const unsigned o = __shfl_up(incl, off, 64);
                if (lane >= off) incl += o;
            }
            const unsigned excl = incl - s;
            if (excl < (unsigned)remaining && incl >= (unsigned)remaining) {
                unsigned run = excl;
                int d = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (run + c[i] >= (unsigned)remaining) {
                        d = 255 - 4 * lane - i;
                        break;
                    }
                    run += c[i];
                }
                bcast[0] = (uint64_t)d;
                bcast[1] = (uint64_t)(remaining - (int)run);
            }
        }
        __syncthreads();
        const uint64_t d = bcast[0];
        remaining = (int)bcast[1];
        __syncthreads();
        prefix |= d << shift;
        mask |= (uint64_t)0xff << shift;
    }
    return prefix;  // keys are distinct: exactly `want` keys are >= prefix
}

constexpr int TOPK_SMALL_K = 32;  // up to this k, selection by repeated maxima
constexpr int TOPK_WIDE_K = 64;   // up to this k, stage 1 on TOPK_WCHUNK-score chunks by maxima
// Above this k the selections sort in LDS instead of taking k dependent rounds of a
// wavefront maximum. Measured on MI355X (n = 2^20, per call, 16 / 64 rows): k = 32 79 / 105
// -> 62 / 89 us sorted, k = 24 66 / 93 -> 59 / 86; k = 10 43 / 75 with rounds against 53 / 83
// sorted, k = 16 even.
constexpr int TOPK_SORT_K = 16;

// Keys topk_merge gathers in LDS at the thread-maxima bound before it falls back to the
// radix select (32 KB).
constexpr int TOPK_MERGE_POOL = 4096;

// v and the value of the lane a DPP pattern names (every lane has a source lane), larger.
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)v, CTRL, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, false);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    return o > v ? o : v;
}

// Maximum over the wavefront, in every lane: within each row of 16 lanes by DPP moves
// (lane ^ 1, lane ^ 2, the half-row mirror, the row mirror: a few cycles each), then
// across rows by the row-pair and half-wave swaps (v_permlane16_swap /
// v_permlane32_swap), all VALU.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = dpp_max_u64<0xB1>(v);   // quad_perm [1,0,3,2]
    v = dpp_max_u64<0x4E>(v);   // quad_perm [2,3,0,1]
    v = dpp_max_u64<0x141>(v);  // row_half_mirror: groups of 8
    v = dpp_max_u64<0x140>(v);  // row_mirror: groups of 16
#pragma unroll
    for (int wide = 0; wide < 2; ++wide) {
        const auto lo = wide ? __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false)
                             : __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
        const auto hi = wide ? __builtin_amdgcn_permlane32_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false)
                             : __builtin_amdgcn_permlane16_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false);
        const uint64_t a = ((uint64_t)(uint32_t)hi[0] << 32) | (uint32_t)lo[0];
        const uint64_t b = ((uint64_t)(uint32_t)hi[1] << 32) | (uint32_t)lo[1];
        v = a > b ? a : b;
    }
    return v;
}

// The block's k largest keys (held EPT per thread, distinct, 0 = none), in descending
// order, into out[0..k) (0 past the block's nonzero keys), by taking the block maximum
// k times: no atomics, so it does not slow down when the scores crowd a few values (a
// radix histogram's first passes do: every key of a chunk shares its top byte). The
// keys taken are zeroed in `key`. 256 threads; red is 4 LDS words.
template <int EPT>
__device__ void top_by_max(uint64_t (&key)[EPT], int k, uint64_t *out, uint64_t *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int r = 0; r < k; ++r) {
        uint64_t m = 0;
#pragma unroll
        for (int j = 0; j < EPT; ++j) m = key[j] > m ? key[j] : m;
        m = wave_max_u64(m);
        if (lane == 0) red[wave] = m;
        __syncthreads();
        uint64_t best = red[0];
#pragma unroll
        for (int w = 1; w < 4; ++w) best = red[w] > best ? red[w] : best;
        __syncthreads();
        if (threadIdx.x == 0) out[r] = best;
        if (best == 0) {  // no keys left: pad (uniform branch)
            for (int i = r + 1 + threadIdx.x; i < k; i += 256) out[i] = 0;
            return;
        }
#pragma unroll
        for (int j = 0; j < EPT; ++j) key[j] = key[j] == best ? 0 : key[j];
    }
}

// Bitonic sort of a[0..n) in LDS, descending (zeros sink to the end); n a power of two.
// Every thread of the 256-thread block calls it; it ends with a barrier.
__device__ void block_sort_desc(uint64_t *a, int n) {
    for (int size = 2; size <= n; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < n; i += 256) {
                const int j = i ^ stride;
                if (j > i) {
                    const uint64_t x = a[i], y = a[j];
                    const bool desc = (i & size) == 0;
                    if (desc ? x < y : x > y) {
                        a[i] = y;
                        a[j] = x;
                    }
                }
            }
            __syncthreads();
        }
}

// k rounds over one wavefront's keys (N slots per lane, only the first NB of them nonzero):
// round r writes the wavefront maximum to out[r] (lane 0) and zeroes it where it was.
template <int NB, int N>
__device__ __forceinline__ void max_rounds(uint64_t (&v)[N], int k, uint64_t *out, int lane) {
    for (int r = 0; r < k; ++r) {
        uint64_t m = 0;
#pragma unroll
        for (int i = 0; i < NB; ++i) m = v[i] > m ? v[i] : m;
        m = wave_max_u64(m);
        if (lane == 0) out[r] = m;
#pragma unroll
        for (int i = 0; i < NB; ++i) v[i] = v[i] == m ? 0 : v[i];
    }
}

// The block's k largest keys (k <= KMAX; keys held EPT per thread, distinct, 0 = none)
// in descending order into out[0..k), 0-padded, with little work per key:
//   1. each thread's largest key; wavefront 0 finds T, the k-th largest of those 256
//      maxima (or 1 when fewer than k are nonzero). At least k keys are >= T (the k
//      threads' maxima), so every one of the block's k largest keys is >= T;
//   2. the keys >= T (at most EPT keys of each of those k threads) are gathered in LDS;
//   3. wavefront 0 takes their maximum k times, over as many slots per lane as the
//      gathered count needs (a power of two: fully unrolled, no per-slot branches).
// For k > TOPK_SORT_K, steps 1 and 3 sort in LDS instead (block_sort_desc: the 256 maxima,
// then the gathered keys padded to a power of two), where k dependent rounds of a
// wavefront maximum would cost more.
// 256 threads; lds holds 256 + EPT*KMAX + 2 words.
template <int EPT, int KMAX = TOPK_SMALL_K>
__device__ void top_small_k(const uint64_t (&key)[EPT], int k, uint64_t *out, uint64_t *lds) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t *maxima = lds, *cand = lds + 256, *misc = lds + 256 + EPT * KMAX;
    uint64_t tmax = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) tmax = key[j] > tmax ? key[j] : tmax;
    maxima[tid] = tmax;
    if (tid == 0) misc[1] = 0;  // candidate count
    __syncthreads();
    if (k > TOPK_SORT_K) {  // uniform
        block_sort_desc(maxima, 256);
        const uint64_t t = maxima[k - 1] != 0 ? maxima[k - 1] : 1;  // 1: fewer than k nonzero maxima
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if (key[j] != 0 && key[j] >= t) cand[atomicAdd(reinterpret_cast<unsigned *>(&misc[1]), 1u)] = key[j];
        __syncthreads();
        const int c = (int)(unsigned)misc[1];  // <= EPT * k
        int p = 2;
        while (p < c) p <<= 1;
        for (int i = c + tid; i < p; i += 256) cand[i] = 0;
        __syncthreads();
        block_sort_desc(cand, p);
        for (int i = tid; i < k; i += 256) out[i] = i < c ? cand[i] : 0;
        return;
    }
    if (wave == 0) {
        uint64_t v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = maxima[4 * lane + i];
        uint64_t t = 1;
        for (int r = 0; r < k; ++r) {
            uint64_t m = v[0];
#pragma unroll
            for (int i = 1; i < 4; ++i) m = v[i] > m ? v[i] : m;
            m = wave_max_u64(m);
            if (m == 0) {  // fewer than k nonzero maxima: every nonzero key is a candidate
                t = 1;
                break;
            }
            t = m;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = v[i] == m ? 0 : v[i];
        }
        if (lane == 0) misc[0] = t;
    }
    __syncthreads();
    const uint64_t t = misc[0];
#pragma unroll
    for (int j = 0; j < EPT; ++j)
        if (key[j] != 0 && key[j] >= t) cand[atomicAdd(reinterpret_cast<unsigned *>(&misc[1]), 1u)] = key[j];
    __syncthreads();
    if (wave == 0) {
        const int c = (int)(unsigned)misc[1];  // <= EPT * k
        constexpr int NV = EPT * KMAX / 64;
        uint64_t v[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int idx = lane + 64 * i;
            v[i] = idx < c ? cand[idx] : 0;
        }
        const int nv = (c + 63) >> 6;  // slots holding keys; uniform
        if (nv <= 1) max_rounds<1>(v, k, out, lane);
        else if (nv <= 2) max_rounds<(NV < 2 ? NV : 2)>(v, k, out, lane);
        else if (nv <= 4) max_rounds<(NV < 4 ? NV : 4)>(v, k, out, lane);
        else if (nv <= 8) max_rounds<(NV < 8 ? NV : 8)>(v, k, out, lane);
        else if (nv <= 16) max_rounds<(NV < 16 ? NV : 16)>(v, k, out, lane);
        else max_rounds<NV>(v, k, out, lane);
    }
}

// Stage 1 for k > TOPK_WIDE_K. Grid (nchunks - chunk0, rows), 256 threads; chunk index =
// chunk0 + blockIdx.x. cand[row][chunk][k], 0 for unused slots. With `thr` (a key per row,
// 0 for none; topk_thresh_radix), a chunk first lists its keys at or above the row's key
// and stops there when they are at most k (they are then its only keys that can be among
// the row's k largest), as topk_chunk_wide does.
__global__ __launch_bounds__(256) void topk_chunk(const float *__restrict__ scores, int64_t ld, int64_t n, int k,
                                                  int nchunks, uint64_t *__restrict__ cand, int chunk0,
                                                  const uint64_t *__restrict__ thr) {
    constexpr int EPT = TOPK_CHUNK / 256;
    __shared__ unsigned hist[256];
    __shared__ uint64_t bcast[2];
    __shared__ unsigned fill;
    const int64_t row = blockIdx.y, chunk = chunk0 + (int64_t)blockIdx.x, base = chunk * TOPK_CHUNK;
    const float *p = scores + row * ld;
    uint64_t key[EPT];
    {
        // unconditional (clamped) loads, all in flight before the first is used (n > 0
        // whenever a chunk is launched)
        const int64_t last = n - 1;
        float x[EPT];
#pragma unroll
        for (int j = 0; j < EPT; ++j) x[j] = p[min(base + threadIdx.x + 256 * j, last)];  // coalesced
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const int64_t i = base + threadIdx.x + 256 * j;
            key[j] = i <= last ? topk_key(x[j], i) : 0;
        }
    }
    uint64_t *out = cand + (row * nchunks + chunk) * (int64_t)k;
    if (thr != nullptr) {
        const uint64_t t = thr[row];  // >= 2^32 when set, so padding keys (0) never pass
        if (t != 0) {
            if (threadIdx.x == 0) fill = 0;
            __syncthreads();
#pragma unroll
            for (int j = 0; j < EPT; ++j)
                if (key[j] >= t) {
                    const unsigned pos = atomicAdd(&fill, 1u);
                    if (pos < (unsigned)k) out[pos] = key[j];
                }
            __syncthreads();
            const unsigned total = fill;
            if (total <= (unsigned)k) {
                for (int i = (int)total + threadIdx.x; i < k; i += 256) out[i] = 0;
                return;
            }
            __syncthreads();  // every thread has read fill before the selection resets it
        }
    }
    const uint64_t th = radix_threshold<EPT>(key, k, hist, bcast);
    if (threadIdx.x == 0) fill = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < EPT; ++j)
        if (key[j] != 0 && key[j] >= th) out[atomicAdd(&fill, 1u)] = key[j];  // the set is exact; its order is not
    __syncthreads();
    for (int i = (int)fill + threadIdx.x; i < k; i += 256) out[i] = 0;
}

// Stage 1 for k <= TOPK_WIDE_K: one workgroup per (row, TOPK_WCHUNK-score chunk), each
// thread holding 32 scores (the index is implicit in the position) and comparing them as
// floats, so a workgroup covers 2x the scores of topk_chunk for the same selection work
// (the k-round selections are the serial part, once per chunk) and only the keys it keeps
// are built. Same output contract as
// topk_chunk: the chunk's k largest keys, in descending order, 0-padded.
//   1. each thread's largest key (ties to the lowest index: strict >, ascending positions);
//   2. wavefront 0: T = the k-th largest of the 256 thread maxima (1 when fewer than k
//      are nonzero); every one of the chunk's k largest keys is >= T;
//   3. threads whose maximum is >= T (at most k) gather their keys >= T in LDS;
//   4. wavefront 0 takes the maximum of the gathered keys k times.
// For k > TOPK_SORT_K, steps 2 and 4 sort in LDS instead (block_sort_desc), as
// top_small_k does.
constexpr int TOPK_WCHUNK = 8192;

//
// With `thr` (a key per row, 0 for none), a chunk first counts its keys >= the row's key:
// when there are at most k, they are the chunk's only keys that can be among the row's k
// largest (thr is a lower bound of the row's k-th largest key), and the chunk writes just
// those, in any order, 0-padded, with no selection rounds. Otherwise (or with no
// threshold) it selects its k largest as above. Chunk index = chunk0 + blockIdx.x.
constexpr int TOPK_SAMPLE_CHUNKS = 4;  // chunks per row whose k largest give the row's threshold

// The score whose order bits are a key's high half (the inverse of topk_order on non-NaN).
__device__ __forceinline__ float topk_key_score(uint64_t key) {
    const uint32_t th = (uint32_t)(key >> 32);
    return __uint_as_float((th & 0x80000000u) ? (th & 0x7fffffffu) : ~th);
}

__global__ __launch_bounds__(256) void topk_chunk_wide(const float *__restrict__ scores, int64_t ld, int64_t n, int k,
                                                       int nchunks, uint64_t *__restrict__ cand, int chunk0,
                                                       const uint64_t *__restrict__ thr) {
    constexpr int EPT = TOPK_WCHUNK / 256;
    __shared__ uint64_t maxima[256];
    __shared__ uint64_t gathered[TOPK_WIDE_K * EPT];  // <= k threads x EPT keys
    __shared__ uint64_t thresh;
    __shared__ unsigned count;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = blockIdx.y, chunk = chunk0 + (int64_t)blockIdx.x, base = chunk * TOPK_WCHUNK;
    const float *p = scores + row * ld + base;
    uint64_t *out = cand + (row * nchunks + chunk) * (int64_t)k;
    // last valid position of the chunk (n > 0 whenever a chunk is launched); the loads are
    // unconditional (clamped), so all of them are in flight before the first is used
    const int last = (int)(n - base < TOPK_WCHUNK ? n - base : TOPK_WCHUNK) - 1;
    float x[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) x[j] = p[min(tid + 256 * j, last)];  // coalesced
    auto lo_at = [&](int j) { return 0xffffffffu - (uint32_t)(base + tid + 256 * j); };
    // The comparisons below run on the floats themselves, which order exactly as the keys'
    // high halves do: a NaN compares false (never retained), -0 == +0, and a strict > over
    // ascending positions keeps the lowest index among equal scores.
    if (thr != nullptr) {
        const uint64_t t = thr[row];
        if (t != 0) {
            // key >= t: score above t's, or equal and index low half at least t's
            const float tf = topk_key_score(t);
            const uint32_t tl = (uint32_t)t;
            uint32_t mine = 0;
#pragma unroll
            for (int j = 0; j < EPT; ++j)
                mine |= (tid + 256 * j <= last && (x[j] > tf || (x[j] == tf && lo_at(j) >= tl))) ? 1u << j : 0u;
            if (tid == 0) count = 0;
            __syncthreads();
            if (mine != 0u) {
                unsigned pos = atomicAdd(&count, (unsigned)__builtin_popcount(mine));
                for (uint32_t m = mine; m != 0u; m &= m - 1u, ++pos) {
                    const int j = __builtin_ctz(m);
                    if (pos < (unsigned)k) gathered[pos] = ((uint64_t)topk_order(x[j]) << 32) | lo_at(j);
                }
            }
            __syncthreads();
            const unsigned total = count;
            if (total <= (unsigned)k) {
                for (int i = tid; i < k; i += 256) out[i] = i < (int)total ? gathered[i] : 0;
                return;
            }
            __syncthreads();  // every thread has read count before the selection resets it
        }
    }
    float bf = -INFINITY;
    int bj = -1;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const bool up = tid + 256 * j <= last && (x[j] > bf || (bj < 0 && x[j] == bf));  // -inf is a score
        bf = up ? x[j] : bf;
        bj = up ? j : bj;
    }
    const uint64_t tmax = bj >= 0 ? ((uint64_t)topk_order(bf) << 32) | lo_at(bj) : 0;
    maxima[tid] = tmax;
    if (tid == 0) count = 0;
    __syncthreads();
    const bool sorted = k > TOPK_SORT_K;  // uniform: steps 2 and 4 sort in LDS (top_small_k)
    if (sorted) {
        block_sort_desc(maxima, 256);
        if (tid == 0) thresh = maxima[k - 1] != 0 ? maxima[k - 1] : 1;
    } else if (wave == 0) {
        uint64_t v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = maxima[4 * lane + i];
        uint64_t t = 1;
        for (int r = 0; r < k; ++r) {
            uint64_t mx = v[0];
#pragma unroll
            for (int i = 1; i < 4; ++i) mx = v[i] > mx ? v[i] : mx;
            mx = wave_max_u64(mx);
            if (mx == 0) {  // fewer than k nonzero maxima: every nonzero key is gathered
                t = 1;
                break;
            }
            t = mx;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = v[i] == mx ? 0 : v[i];
        }
        if (lane == 0) thresh = t;
    }
    __syncthreads();
    const uint64_t t = thresh;
    if (tmax >= t && tmax != 0) {
        // key >= t: score above t's, or equal and index low half (0xffffffff - index) at
        // least t's; t == 1 takes every non-NaN score
        const bool every = t == 1;
        const uint32_t tl = (uint32_t)t;
        const float tf = topk_key_score(t);
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const uint32_t lo = lo_at(j);
            const bool in = tid + 256 * j <= last && (every ? x[j] == x[j] : (x[j] > tf || (x[j] == tf && lo >= tl)));
            if (in) gathered[atomicAdd(&count, 1u)] = ((uint64_t)topk_order(x[j]) << 32) | lo;
        }
    }
    __syncthreads();
    if (sorted) {
        const int c = (int)count;  // <= k * EPT
        int p = 2;
        while (p < c) p <<= 1;
        for (int i = c + tid; i < p; i += 256) gathered[i] = 0;
        __syncthreads();
        block_sort_desc(gathered, p);
        for (int i = tid; i < k; i += 256) out[i] = i < c ? gathered[i] : 0;
        return;
    }
    if (wave != 0) return;
    const int c = (int)count;
    if (c <= 64) {
        uint64_t v = lane < c ? gathered[lane] : 0;
        for (int r = 0; r < k; ++r) {
            const uint64_t mx = wave_max_u64(v);
            if (lane == 0) out[r] = mx;
            v = v == mx ? 0 : v;
        }
        return;
    }
    for (int r = 0; r < k; ++r) {
        uint64_t best = 0;
        int at = -1;
        for (int i = lane; i < c; i += 64) {
            const uint64_t kk = gathered[i];
            if (kk > best) {
                best = kk;
                at = i;
            }
        }
        const uint64_t mx = wave_max_u64(best);
        if (lane == 0) out[r] = mx;
        if (mx != 0 && best == mx) gathered[at] = 0;  // keys are unique: one lane
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// The row thresholds for topk_chunk_wide: the k-th largest of the keys stage 1 kept from
// each row's first TOPK_SAMPLE_CHUNKS chunks (the k largest of each, so the k-th largest
// key among all their scores, a lower bound of the row's k-th largest), or 0 when those
// chunks hold fewer than k keys. One wavefront per row; k <= TOPK_WIDE_K (the host takes
// topk_thresh_sorted above TOPK_SORT_K).
__global__ __launch_bounds__(256) void topk_thresh(const uint64_t *__restrict__ cand, int64_t rows, int nchunks, int k,
                                                   uint64_t *__restrict__ thr, unsigned *__restrict__ zero) {
    constexpr int PER_LANE = TOPK_SAMPLE_CHUNKS * TOPK_WIDE_K / 64;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint64_t *c = cand + row * nchunks * (int64_t)k;
    const int m = TOPK_SAMPLE_CHUNKS * k;  // <= 64 * PER_LANE
    uint64_t v[PER_LANE];
#pragma unroll
    for (int i = 0; i < PER_LANE; ++i) v[i] = lane + 64 * i < m ? c[lane + 64 * i] : 0;
    uint64_t t = 0;
    for (int r = 0; r < k; ++r) {
        uint64_t mx = v[0];
#pragma unroll
        for (int i = 1; i < PER_LANE; ++i) mx = v[i] > mx ? v[i] : mx;
        t = wave_max_u64(mx);
        if (t == 0) break;  // fewer than k keys: no threshold
#pragma unroll
        for (int i = 0; i < PER_LANE; ++i) v[i] = v[i] == t ? 0 : v[i];  // keys are unique: one slot
    }
    if (lane == 0) thr[row] = t;
    if (lane == 0 && zero != nullptr) zero[row] = 0;  // the row's TopkSink count
}

// topk_thresh for k > TOPK_SORT_K: one workgroup per row sorts the row's
// TOPK_SAMPLE_CHUNKS * k sample keys in LDS (block_sort_desc) and takes the k-th, where k
// dependent rounds of a wavefront maximum would cost more (k = 64: 18.8 us per 256 rows).
__global__ __launch_bounds__(256) void topk_thresh_sorted(const uint64_t *__restrict__ cand, int nchunks, int k,
                                                          uint64_t *__restrict__ thr, unsigned *__restrict__ zero) {
    __shared__ uint64_t keys[TOPK_SAMPLE_CHUNKS * TOPK_WIDE_K];
    const int64_t row = blockIdx.x;
    const uint64_t *c = cand + row * nchunks * (int64_t)k;
    const int m = TOPK_SAMPLE_CHUNKS * k;  // <= TOPK_SAMPLE_CHUNKS * TOPK_WIDE_K
    int p = 2;
    while (p < m) p <<= 1;
    for (int i = threadIdx.x; i < p; i += 256) keys[i] = i < m ? c[i] : 0;
    __syncthreads();
    block_sort_desc(keys, p);
    if (threadIdx.x == 0) {
        thr[row] = keys[k - 1];  // 0 when the sample holds fewer than k keys: no threshold
        if (zero != nullptr) zero[row] = 0;
    }
}

// The merge after the fused scoring GEMM (gemm_w8a8_pt<EPI_TOPK>): one workgroup per row
// takes the k largest (k <= KMAX) of the count[row] candidates the GEMM kept (keys at
// key[row*cap ..], their scores at score[row*cap ..], unordered), and writes indices and
// scores as topk_merge does. A row with more than cap candidates writes nothing: its
// caller runs the two-pass path instead. cap <= 256 * EPT.
template <int EPT, int KMAX>
__global__ __launch_bounds__(256) void topk_sink_merge(const unsigned *__restrict__ count,
                                                       const uint64_t *__restrict__ key,
                                                       const float *__restrict__ score_in, int cap, int k,
                                                       int32_t *__restrict__ index, int64_t ldi,
                                                       float *__restrict__ score, int64_t lds_) {
    __shared__ uint64_t lds[256 + EPT * KMAX + 2];
    __shared__ uint64_t sorted[KMAX];
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const unsigned n = count[row];
    if (n > (unsigned)cap) return;  // the same for every thread of the row
    const uint64_t *kr = key + row * cap;
    const float *sr = score_in + row * cap;
    uint64_t kk[EPT];
    float sv[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        // clamped loads, all in flight at once; past n the key is masked to 0 (none)
        const unsigned i = (unsigned)(tid + 256 * j);
        const unsigned at = i < n ? i : 0u;
        const uint64_t keep = i < n ? ~0ull : 0ull;
        kk[j] = kr[at] & keep;
        sv[j] = sr[at];
    }
    top_small_k<EPT, KMAX>(kk, k, sorted, lds);
    __syncthreads();
    for (int i = tid; i < k; i += 256) {
        const uint64_t s = sorted[i];
        index[row * ldi + i] = s ? (int32_t)topk_index(s) : -1;
        if (!s) score[row * lds_ + i] = __uint_as_float(0x7fc00000u);
    }
    // each selected key's own f32 score, from the one thread that holds it (keys are unique;
    // only keys at or above the k-th selected one can be among them)
    const uint64_t kth = sorted[k - 1];
#pragma unroll
    for (int j = 0; j < EPT; ++j)
        if (kk[j] != 0 && kk[j] >= kth)
            for (int i = 0; i < k; ++i)
                if (kk[j] == sorted[i]) score[row * lds_ + i] = sv[j];
}

// radix_threshold over m keys in device memory (read once per pass; the merge's
// candidates stay in L2), same contract.
__device__ uint64_t radix_threshold_mem(const uint64_t *__restrict__ c, int64_t m, int want, unsigned *hist,
                                        uint64_t *bcast) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid == 0) hist[0] = 0;
    __syncthreads();
    // every pass reads the m keys 8 per thread at a time (clamped loads, all in flight)
    auto sweep = [&](auto &&visit) {
        for (int64_t i0 = tid; i0 < m; i0 += 256 * 8) {
            uint64_t kk[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) kk[u] = c[min(i0 + 256 * u, m - 1)];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (i0 + 256 * u < m) visit(kk[u]);
        }
    };
    unsigned mine = 0;
    sweep([&](uint64_t kk) { mine += kk != 0; });
    atomicAdd(&hist[0], mine);
    __syncthreads();
    const int64_t valid = hist[0];
    __syncthreads();
    if (valid <= want) return 1;
    uint64_t prefix = 0, mask = 0;
    int remaining = want;
    for (int shift = 56; shift >= 0; shift -= 8) {
        hist[tid] = 0;
        __syncthreads();
        sweep([&](uint64_t kk) {
            if (kk != 0 && (kk & mask) == prefix) atomicAdd(&hist[(kk >> shift) & 255u], 1u);
        });
        __syncthreads();
        if (tid < 64) {
            unsigned cnt[4], sum = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                cnt[i] = hist[255 - 4 * lane - i];
                sum += cnt[i];
            }
            unsigned incl = sum;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const unsigned o = __shfl_up(incl, off, 64);
                if (lane >= off) incl += o;
            }
            const unsigned excl = incl - sum;
            if (excl < (unsigned)remaining && incl >= (unsigned)remaining) {
                unsigned run = excl;
                int d = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (run + cnt[i] >= (unsigned)remaining) {
                        d = 255 - 4 * lane - i;
                        break;
                    }
                    run += cnt[i];
                }
                bcast[0] = (uint64_t)d;
                bcast[1] = (uint64_t)(remaining - (int)run);
            }
        }
        __syncthreads();
        const uint64_t d = bcast[0];
        remaining = (int)bcast[1];
        __syncthreads();
        prefix |= d << shift;
        mask |= (uint64_t)0xff << shift;
    }
    return prefix;
}

// The row thresholds for topk_chunk (k > TOPK_WIDE_K): the k-th largest of the keys stage 1
// kept from each row's first TOPK_SAMPLE_CHUNKS chunks, a lower bound of the row's k-th
// largest key, or 0 when those chunks hold at most k keys. One workgroup per row.
__global__ __launch_bounds__(256) void topk_thresh_radix(const uint64_t *__restrict__ cand, int nchunks, int k,
                                                         uint64_t *__restrict__ thr) {
    __shared__ unsigned hist[256];
    __shared__ uint64_t bcast[2];
    const int64_t row = blockIdx.x;
    const uint64_t t = radix_threshold_mem(cand + row * nchunks * (int64_t)k, (int64_t)TOPK_SAMPLE_CHUNKS * k, k,
                                           hist, bcast);
    if (threadIdx.x == 0) thr[row] = t == 1 ? 0 : t;  // 1: at most k keys (a real key is >= 2^32)
}

// Stage 2. Grid (rows), 256 threads, kp * 8 bytes of dynamic LDS (kp: k rounded up to a
// power of two). The row's m = nchunks * k candidates are cand[row*m ..]. Writes
// index[row*ldi + i] (-1 past the row's non-NaN scores) and score[row*lds_ + i] (NaN
// there); the score is re-read from the row (scores, pitch ld) so a -0 stays -0.
__global__ __launch_bounds__(256) void topk_merge(const uint64_t *__restrict__ cand, int64_t m, int k, int kp,
                                                  const float *__restrict__ scores, int64_t ld,
                                                  int32_t *__restrict__ index, int64_t ldi, float *__restrict__ score,
                                                  int64_t lds_) {
    __shared__ unsigned hist[256];
    __shared__ uint64_t bcast[2], red[4];
    __shared__ unsigned fill;
    extern __shared__ uint64_t sorted[];
    const int64_t row = blockIdx.x;
    const uint64_t *c = cand + row * m;
    if (k > TOPK_SORT_K && k <= TOPK_WIDE_K && m <= 2 * TOPK_CHUNK) {
        // up to 64 of at most 8192 candidates: top_small_k over them in registers. Each
        // thread holds 32 consecutive slots (half of a chunk's list at k = 64): a list is
        // in descending order, so strided slots would give each thread one rank of many
        // lists, and the thread maxima a loose bound (thousands of keys gathered).
        constexpr int EPT = 2 * TOPK_CHUNK / 256;
        __shared__ uint64_t wide[256 + EPT * TOPK_WIDE_K + 2];
        uint64_t key[EPT];
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const int64_t i = (int64_t)threadIdx.x * EPT + j;
            key[j] = c[min(i, m - 1)] & (i < m ? ~0ull : 0ull);  // clamped loads, all in flight
        }
        top_small_k<EPT, TOPK_WIDE_K>(key, k, sorted, wide);
        __syncthreads();
        for (int i = threadIdx.x; i < k; i += 256) {
            const uint64_t kk = sorted[i];
            const int64_t col = kk ? topk_index(kk) : -1;
            index[row * ldi + i] = (int32_t)col;
            score[row * lds_ + i] = kk ? scores[row * ld + col] : __uint_as_float(0x7fc00000u);
        }
        return;
    }
    if (k <= TOPK_SMALL_K && m <= TOPK_CHUNK) {
        // few candidates, small k: hold them in registers and take the maxima in order
        constexpr int EPT = TOPK_CHUNK / 256;
        uint64_t key[EPT];
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const int64_t i = threadIdx.x + 256 * j;
            key[j] = i < m ? c[i] : 0;
        }
        top_by_max<EPT>(key, k, sorted, red);
        __syncthreads();
        for (int i = threadIdx.x; i < k; i += 256) {
            const uint64_t kk = sorted[i];
            const int64_t col = kk ? topk_index(kk) : -1;
            index[row * ldi + i] = (int32_t)col;
            score[row * lds_ + i] = kk ? scores[row * ld + col] : __uint_as_float(0x7fc00000u);
        }
        return;
    }
    if (k <= 128) {
        // The k-th largest of the 256 thread maxima over the candidates bounds the row's k-th
        // largest key from below; the keys at or above it (a few hundred on mixed lists) are
        // gathered in LDS and sorted. Two sweeps of the candidates in memory instead of the
        // radix select's eight. In step j thread t takes slot 256 j + (t + j) % 256: a
        // wavefront still reads consecutive slots, but a thread meets a different position of
        // each chunk's list (with t + 256 j alone and k dividing 256, every thread would hold
        // one list position: the chunks' best keys in a few threads, a loose bound). More
        // than TOPK_MERGE_POOL keys at the bound take the radix select below. Up to k = 128:
        // at k = 256 the bound is the least thread maximum and often too loose (measured on
        // MI355X, 2^20 scores, 64 rows: 273 -> 311 us; k = 100 and 128: 163 -> 118 and 181 -> 126).
        __shared__ uint64_t mx[256];
        __shared__ uint64_t pool[TOPK_MERGE_POOL];
        __shared__ unsigned np;
        const int64_t steps = (m + 255) / 256;
        auto sweep = [&](auto &&visit) {
            for (int64_t j0 = 0; j0 < steps; j0 += 8) {
                uint64_t kk[8];
                int64_t at[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int64_t j = j0 + u;
                    at[u] = 256 * j + ((threadIdx.x + j) & 255);
                    kk[u] = c[min(at[u], m - 1)];  // clamped, all in flight
                }
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (at[u] < m) visit(kk[u]);
            }
        };
        uint64_t tmax = 0;
        sweep([&](uint64_t kk) { tmax = kk > tmax ? kk : tmax; });
        mx[threadIdx.x] = tmax;
        if (threadIdx.x == 0) np = 0;
        __syncthreads();
        block_sort_desc(mx, 256);
        const uint64_t t = mx[k - 1] != 0 ? mx[k - 1] : 1;  // 1: fewer than k nonzero maxima
        sweep([&](uint64_t kk) {
            if (kk != 0 && kk >= t) {
                const unsigned pos = atomicAdd(&np, 1u);
                if (pos < (unsigned)TOPK_MERGE_POOL) pool[pos] = kk;
            }
        });
        __syncthreads();
        const int n = (int)np;
        if (n <= TOPK_MERGE_POOL) {  // uniform
            int p = 2;
            while (p < n) p <<= 1;
            for (int i = n + threadIdx.x; i < p; i += 256) pool[i] = 0;
            __syncthreads();
            block_sort_desc(pool, p);
            for (int i = threadIdx.x; i < k; i += 256) {
                const uint64_t kk = i < n ? pool[i] : 0;
                const int64_t col = kk ? topk_index(kk) : -1;
                index[row * ldi + i] = (int32_t)col;
                score[row * lds_ + i] = kk ? scores[row * ld + col] : __uint_as_float(0x7fc00000u);
            }
            return;
        }
        __syncthreads();  // every thread has read np before the radix select reuses LDS
    }
    const uint64_t th = radix_threshold_mem(c, m, k, hist, bcast);
    for (int i = threadIdx.x; i < kp; i += 256) sorted[i] = 0;
    if (threadIdx.x == 0) fill = 0;
    __syncthreads();
    for (int64_t i0 = threadIdx.x; i0 < m; i0 += 256 * 8) {
        uint64_t kk[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) kk[u] = c[min(i0 + 256 * u, m - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (i0 + 256 * u < m && kk[u] != 0 && kk[u] >= th) sorted[atomicAdd(&fill, 1u)] = kk[u];  // at most k
    }
    __syncthreads();
    block_sort_desc(sorted, kp);  // the zero padding sinks to the end
    for (int i = threadIdx.x; i < k; i += 256) {
        const uint64_t kk = sorted[i];
        const int64_t col = kk ? topk_index(kk) : -1;
        index[row * ldi + i] = (int32_t)col;
        score[row * lds_ + i] = kk ? scores[row * ld + col] : __uint_as_float(0x7fc00000u);
    }
}

// Rows of zero scores (n == 0): index -1 and a NaN score in each of the k slots, as the
// merge pads. Grid-stride over rows.
__global__ __launch_bounds__(256) void topk_empty(int64_t rows, int k, int32_t *__restrict__ index, int64_t ldi,
                                                  float *__restrict__ score, int64_t lds_) {
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x)
        for (int i = threadIdx.x; i < k; i += 256) {
            index[row * ldi + i] = -1;
            score[row * lds_ + i] = __uint_as_float(0x7fc00000u);
        }
}

}  // namespace enchip
