// gemm_persistent.h -- the persistent W8A8 GEMM used for M > small-M on gfx950.
//
// One workgroup per half CU (2 per CU), each walking a list of 128 x 256 output tiles.
//
// Main loop (per 64-deep K stage, 4 waves side by side along N, each 128 x 64):
//   * W fragments go HBM -> registers directly. The weights are pre-swizzled
//     fragment-major, so each load is 64 lanes x 16 contiguous bytes. Each wave owns its
//     64 output channels, so nothing is shared and nothing passes through LDS.
//   * A is staged through two LDS slots as 1 KiB fragments in MFMA operand order, and
//     all 4 waves read all of it. With AF the activations are already fragment-major
//     (quant_rows_*<FRAG>): each load is 64 lanes x 16 contiguous bytes, like the
//     weights'. Without AF they are row-major int8 at pitch lda, and each load gathers
//     32 rows x 32 bytes (measured 15-25% slower main loop on MI355X).
//   * One ring of PW stages (the loads for stage t + PW are issued during stage t)
//     carries both operands. Its refill loads are unconditional
//     and wrap into the next tile's first stages, so:
//       - the compiler's wait counts stay exact;
//       - the next tile's data is in flight during the epilogue.
//   * All LDS fragment reads of a stage are issued before its MFMAs
//     (sched_group_barrier), so no MFMA waits on a just-issued LDS read.
//
// Epilogue (per tile, no VMEM loads):
//   * The tile's aS / wS / bias are loaded with ordinary loads before its main loop,
//     so the compiler's own wait counts cover them, and staged in LDS after it.
//   * Each wave transposes its accumulators through a private LDS scratch and writes
//     16-byte row-major stores: 32 stores per wave per tile instead of 128 dword
//     stores interleaved with loads.
//   * GELU: every value of a 32-row chunk takes ErfF32's series branch without
//     branching; the few values that need another branch are gathered into a per-wave
//     list in LDS and re-evaluated 64 at a time.
//   * EPI_TOPK (ann scoring with its top-k): nothing is stored; the scores at or above
//     their row's bound go to the row's candidate list (TopkSink).
//
// Numerics are those of gemm_w8a8 (kernels.h): the int32 dot is exact, and the epilogue
// rounds in the reference's order, so the two kernels give identical bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"
#include "topk.h"

#pragma clang fp contract(off)

namespace enchip {

// Where EPI_TOPK puts the scores it keeps: row r's candidates are its scores whose top-k
// key (topk.h) is at or above thr[r] (every non-NaN score when thr[r] is 0), in no
// particular order. count[r] (zeroed before the launch) counts them all; the first cap go
// to key[r*cap ..] and, as their f32 bits (so a -0 stays -0), score[r*cap ..].
struct TopkSink {
    const uint64_t *thr = nullptr;
    unsigned *count = nullptr;
    uint64_t *key = nullptr;
    float *score = nullptr;
    int cap = 0;
};

// Tile geometry and ring depth of the persistent kernel (the host checks its
// preconditions). PT_BM_SMALL: the 64-row tile the host picks when 128-row tiles would
// leave workgroup slots idle (fewer tiles than 2 per CU); it runs 3 workgroups per CU.
constexpr int PT_BM = 128, PT_BM_SMALL = 64, PT_BN = 256, PT_BK = 64, PT_PW = 2, PT_NW = 4;

// 16-byte nontemporal store of 4 output words. The f32 outputs are written once and
// not read by this kernel; a normal store would let them evict the A row-blocks and
// weights the XCD's other tiles are still reading from L2.
__device__ __forceinline__ void store_nt(void *p, int4 v) {
    const i32x4 t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<i32x4 *>(p));
}

// PRIO: the wave priority (s_setprio) of the main loop, 0 = unchanged; the epilogue runs
// at priority 0. With 2 workgroups per CU a raised main loop lets a SIMD's MFMA-issuing
// wave go first when the other is in its epilogue (measured on MI355X: 4-10% faster on
// the BERT-base and XLM-R-large bias-only shapes except BERT-base's O, 4% slower, and the
// GELU epilogue unchanged; bit-identical either way).
template <int BM, int BN, int BK, int PW, int EPI, bool AF, int NW, int PRIO>
__global__ __launch_bounds__(64 * NW, BM == PT_BM_SMALL ? 3 : NW / 2) void gemm_w8a8_pt(
    const int8_t *__restrict__ A, int64_t lda, const int8_t *__restrict__ Wf,
    const float *__restrict__ aS, const float *__restrict__ wS, const float *__restrict__ bias,
    void *__restrict__ out, int64_t ldo, int M, int N, int Kp, int tilesN, int numTiles, TopkSink sink) {
    constexpr int NT = 64 * NW;  // threads
    constexpr int WN = BN / NW;  // output columns per wave
    constexpr int TM = BM / 32, TN = WN / 32;
    constexpr int KB = BK / 32;
    constexpr int FA = TM * KB;  // A fragments per stage
    static_assert(FA % NW == 0 && TN >= 1, "A fragments per stage must split over the waves");
    // Stage t writes stage t+1's A to LDS from the ring slot its loads went to one stage
    // earlier; with a 1-stage ring that slot would still hold stage t's A.
    static_assert(PW >= 2, "the ring needs at least 2 stages");
    static_assert(NT >= BN && NT >= BM && (BM & (BM - 1)) == 0, "constant staging: one thread per row / column");
    constexpr int FAW = FA / NW;  // A fragments each wave moves per stage
    constexpr int STAGE = FA * 1024;
    constexpr int RING_LOADS = FAW + KB * TN;  // VMEM loads per ring stage per lane
    constexpr int SP = WN + 8;    // transpose scratch pitch in ints (4*SP = 32 mod 64 banks)
    constexpr int C4 = WN / 4;    // 4-column groups per scratch row
    constexpr int RPL = 64 / C4;  // scratch rows covered by one pass of the wave
    constexpr int KR = 32 / RPL;  // passes per 32-row chunk
    constexpr int TL_CAP = 32 * (SP - WN) * 2;  // 16-bit tail-list cells in the scratch's pad columns
    static_assert(SP - WN == 8 && 32 * SP < 65536, "tail list: 16 cells per scratch row, cell indices fit 16 bits");
    static_assert(KR % 4 == 0, "row scales are read as float4");
    __shared__ __attribute__((aligned(1024))) int8_t smem[2 * STAGE];
    __shared__ __attribute__((aligned(16))) int s_tr[NW][32 * SP];
    __shared__ __attribute__((aligned(16))) float s_as[BM];
    __shared__ __attribute__((aligned(16))) float s_ws[BN];
    __shared__ __attribute__((aligned(16))) float s_b[BN];
    __shared__ __attribute__((aligned(16))) uint64_t s_thr[EPI == EPI_TOPK ? BM : 1];  // row bounds, as s_as

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nk = Kp / BK, nk32 = Kp >> 5;
    // Block b runs on XCD b % 8. Each XCD walks a contiguous range of tiles, so the
    // tiles it holds at once share A row-blocks in its L2.
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, per_xcd = gridDim.x >> 3;
    const int q = numTiles >> 3, r = numTiles & 7;
    const int xbeg = xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q;
    const int xcnt = q + (xcd < r ? 1 : 0);
    const int ntiles = slot < xcnt ? (xcnt - slot + per_xcd - 1) / per_xcd : 0;
    if (ntiles == 0) return;
    auto tile_id = [&](int i) { return xbeg + slot + i * per_xcd; };
    const uint32_t ldau = (uint32_t)lda;
    const bool has_bias = bias != nullptr;

    // 32-bit byte offsets (host guarantees M*lda and Np*Kp fit).
    uint32_t aoff_c[FAW], aoff_x[FAW];  // this lane's A rows: current / next tile
    uint32_t woff_c, woff_x;
    uint32_t acol[FAW];  // this lane's offset within its A row-block (per stage 0)
#pragma unroll
    for (int i = 0; i < FAW; ++i) {
        const int f = wave + NW * i, kb = f % KB;
        acol[i] = AF ? (uint32_t)(kb * 1024 + lane * 16) : (uint32_t)(kb * 32 + 16 * (lane >> 5));
    }
    constexpr uint32_t ASTEP = AF ? KB * 1024 : BK;  // A bytes per K stage along a row-block
    auto tile_offs = [&](int tile, uint32_t *aoff, uint32_t &woff) {
        const int m0 = (tile / tilesN) * BM, n0 = (tile % tilesN) * BN;
#pragma unroll
        for (int i = 0; i < FAW; ++i) {
            const int f = wave + NW * i, rb = f / KB;
            // rows past M are never stored: row-major A re-reads row M-1, fragment-major
            // A reads the buffer's padding rows (allocated up to a multiple of BM)
            if (AF)
                aoff[i] = (uint32_t)((m0 / 32 + rb) * nk32) * 1024u + acol[i];
            else
                aoff[i] = (uint32_t)min(m0 + rb * 32 + (lane & 31), M - 1) * ldau + acol[i];
        }
        woff = (uint32_t)(n0 / 32 + wave * TN) * (uint32_t)nk32 * 1024u + lane * 16;
    };

    i32x4 wreg[PW][KB][TN];
    i32x4 areg[PW][FAW];
    // Stage ls of the current tile, or stage ls - nk of the next one (a select, not a
    // branch).
    auto load_stage = [&](int ring, int ls) {
        const bool nx = ls >= nk;
        const uint32_t t = nx ? ls - nk : ls;
        const uint32_t wo = nx ? woff_x : woff_c;
#pragma unroll
        for (int i = 0; i < FAW; ++i) {
            const uint32_t ao = (nx ? aoff_x[i] : aoff_c[i]) + t * ASTEP;
            areg[ring][i] = *reinterpret_cast<const i32x4 *>(A + ao);
        }
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                wreg[ring][kb][j] = *reinterpret_cast<const i32x4 *>(Wf + (wo + ((uint32_t)j * nk32 + t * KB + kb) * 1024u));
    };
    auto awrite = [&](int ls, int ring) {
#pragma unroll
        for (int i = 0; i < FAW; ++i)
            *reinterpret_cast<i32x4 *>(smem + ls * STAGE + (wave + NW * i) * 1024 + lane * 16) = areg[ring][i];
    };

    i32x16 acc[TM][TN];
    tile_offs(tile_id(0), aoff_c, woff_c);
    tile_offs(tile_id(ntiles > 1 ? 1 : 0), aoff_x, woff_x);
#pragma unroll
    for (int p = 0; p < PW; ++p) load_stage(p, p);  // nk >= PW
    awrite(0, 0);
    __syncthreads();

    // Position of tile row R in s_as: the KR rows a lane needs per 32-row chunk
    // (rsub + RPL * k, k < KR) are contiguous.
    const int as_slot = (tid & ~31) + (tid % RPL) * KR + ((tid & 31) / RPL);
    int g = 0;  // stages consumed so far: LDS slot parity across tiles
    for (int it = 0; it < ntiles; ++it) {
        const int tile = tile_id(it);
        const int m0 = (tile / tilesN) * BM, n0 = (tile % tilesN) * BN;
        // The tile's epilogue constants, loaded before its main loop so their latency
        // hides behind it. Ordinary loads: the compiler counts them into the waits it
        // places before their first use (the LDS staging after the main loop), and the
        // main loop's barriers keep it from sinking them there.
        const float c_as = aS[min(m0 + (tid & (BM - 1)), M - 1)];
        const float c_ws = wS[min(n0 + tid, N - 1)];
        const float c_b = has_bias ? bias[min(n0 + tid, N - 1)] : kNoBias;
        const uint64_t c_thr = EPI == EPI_TOPK ? sink.thr[min(m0 + (tid & (BM - 1)), M - 1)] : 0;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int rr = 0; rr < 16; ++rr) acc[i][j][rr] = 0;
        for (int t0 = 0; t0 < nk; t0 += PW) {
#pragma unroll
            for (int p = 0; p < PW; ++p) {
                const int t = t0 + p;
                const int8_t *base = smem + ((g + t) & 1) * STAGE + lane * 16;
                if (PRIO) __builtin_amdgcn_s_setprio(PRIO);
                if constexpr (NW == 4) {
                    i32x4 af[KB][TM];
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                        for (int i = 0; i < TM; ++i)
                            af[kb][i] = *reinterpret_cast<const i32x4 *>(base + (i * KB + kb) * 1024);
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                        for (int i = 0; i < TM; ++i)
#pragma unroll
                            for (int j = 0; j < TN; ++j)
                                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[kb][i], wreg[p][kb][j], acc[i][j], 0, 0, 0);
                    awrite((g + t + 1) & 1, (p + 1) % PW);  // A of the next stage, maybe the next tile's
                    load_stage(p, t + PW);                   // refill this ring slot
                    // LDS reads first, then MFMAs with the LDS writes and VMEM loads interleaved
                    __builtin_amdgcn_sched_group_barrier(0x100, FA, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x200, FAW, 0);
#pragma unroll
                    for (int u = 0; u < RING_LOADS; ++u) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                    }
                    __builtin_amdgcn_sched_group_barrier(0x008, TM * TN * KB - 2 - RING_LOADS, 0);
                } else {
                    // 4 waves per SIMD: registers for one K half-stage of A fragments at a
                    // time; the other waves cover the LDS latency between the halves
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb) {
                        i32x4 af[TM];
#pragma unroll
                        for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const i32x4 *>(base + (i * KB + kb) * 1024);
#pragma unroll
                        for (int i = 0; i < TM; ++i)
#pragma unroll
                            for (int j = 0; j < TN; ++j)
                                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], wreg[p][kb][j], acc[i][j], 0, 0, 0);
                        if (kb == 0) awrite((g + t + 1) & 1, (p + 1) % PW);
                    }
                    load_stage(p, t + PW);  // after the last MFMA that reads this ring slot
                }
                __syncthreads();
            }
        }
        g += nk;
#pragma unroll
        for (int i = 0; i < FAW; ++i) aoff_c[i] = aoff_x[i];
        woff_c = woff_x;
        tile_offs(tile_id(it + 2 < ntiles ? it + 2 : ntiles - 1), aoff_x, woff_x);

        if (PRIO) __builtin_amdgcn_s_setprio(0);
        // ---- epilogue: constants to LDS, then transpose + 16-byte stores per wave
        if (tid < BM) s_as[as_slot] = c_as;
        if (EPI == EPI_TOPK && tid < BM) s_thr[as_slot] = c_thr;
        if (tid < BN) {
            s_ws[tid] = c_ws;
            s_b[tid] = c_b;
        }
        __syncthreads();
        const int c4 = lane % C4, rsub = lane / C4;
        const bool full = m0 + BM <= M && n0 + BN <= N;  // whole tile in range
        const int lcol = wave * WN + 4 * c4;  // tile column of this lane's first output
        const int col = n0 + lcol;
        const float4 ws4 = *reinterpret_cast<const float4 *>(&s_ws[lcol]);
        const float4 b4 = *reinterpret_cast<const float4 *>(&s_b[lcol]);
        const float wsv[4] = {ws4.x, ws4.y, ws4.z, ws4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
        int *scr = s_tr[wave];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int rr = 0; rr < 16; ++rr) scr[acc_row(rr, lane) * SP + j * 32 + (lane & 31)] = acc[i][j][rr];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            float asv[KR];
#pragma unroll
            for (int k4 = 0; k4 < KR; k4 += 4) {
                const float4 t = *reinterpret_cast<const float4 *>(&s_as[i * 32 + rsub * KR + k4]);
                asv[k4] = t.x, asv[k4 + 1] = t.y, asv[k4 + 2] = t.z, asv[k4 + 3] = t.w;
            }
            // This lane's 4 outputs of row rsub + RPL*k of the chunk are at p0 + k*step.
            float *const p0 = reinterpret_cast<float *>(out) + (int64_t)(m0 + i * 32 + rsub) * ldo + col;
            const int64_t step = (int64_t)RPL * ldo;
            auto row_ok = [&](int k) { return m0 + i * 32 + rsub + RPL * k < M && col < N; };
            int4 v[KR];
            if (EPI == EPI_F32_GELU) {
                // Pass 1: dequantize and apply GELU's series branch to all 32 of this
                // lane's values, in place in the scratch; remember which take another
                // branch (|u| >= 1, or NaN) and leave their dequantized value there.
                uint32_t tail_mask = 0;
#pragma unroll
                for (int k = 0; k < KR; ++k) v[k] = *reinterpret_cast<const int4 *>(&scr[(rsub + RPL * k) * SP + 4 * c4]);
#pragma unroll
                for (int k = 0; k < KR; ++k) {
                    const f32x4v y = {dequant(v[k].x, asv[k], wsv[0], bv[0]), dequant(v[k].y, asv[k], wsv[1], bv[1]),
                                      dequant(v[k].z, asv[k], wsv[2], bv[2]), dequant(v[k].w, asv[k], wsv[3], bv[3])};
                    uint32_t t4;
                    const f32x4v gy = gelu_f32_series4(y, t4);
                    const int4 o4 = make_int4(__float_as_int(t4 & 1u ? y.x : gy.x), __float_as_int(t4 & 2u ? y.y : gy.y),
                                              __float_as_int(t4 & 4u ? y.z : gy.z), __float_as_int(t4 & 8u ? y.w : gy.w));
                    tail_mask |= t4 << (4 * k);
                    *reinterpret_cast<int4 *>(&scr[(rsub + RPL * k) * SP + 4 * c4]) = o4;
                }
                // Pass 2a, only when some lane holds more than 28 tail values of its 32 (a
                // wide pre-activation distribution, much of it on ErfF32's sign branch):
                // settle every value on the sign branch (|u| > 4: erf = +-1, so GELU is x or
                // a signed zero, by gelu_f32's operations) across the chunk at once, so that
                // the per-lane rounds below only run the erf tail. Measured on MI355X (same
                // process, M = 32768 or 4096, K = 768, N = 3072): config 2's pre-activations
                // (standard deviation ~22) 65 -> 45 us. The pass costs where tails are many
                // but few on the sign branch, hence the high trigger: at 16, standard
                // deviation 3 (65% tails, 6% on the sign branch) went 341 -> 364 us; at 4,
                // standard deviation 1 (16% tails) 221 -> 249 us; 0.5 (an encoder's FFN)
                // never triggers it.
                if (__builtin_amdgcn_ballot_w64(__builtin_popcount(tail_mask) > 28)) {
#pragma unroll
                    for (int k = 0; k < KR; ++k) {
                        if (((tail_mask >> (4 * k)) & 15u) == 0u) continue;
                        int *cell4 = &scr[(rsub + RPL * k) * SP + 4 * c4];
                        int4 w = *reinterpret_cast<const int4 *>(cell4);
                        int wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const float y = __int_as_float(wv[j]);
                            const float u = y * 0.7071067811865476f;
                            if ((tail_mask >> (4 * k + j)) & 1u && fabsf(u) > 4.0f) {
                                wv[j] = __float_as_int(0.5f * y * (1.0f + (u < 0.0f ? -1.0f : 1.0f)));
                                tail_mask &= ~(1u << (4 * k + j));
                            }
                        }
                        *reinterpret_cast<int4 *>(cell4) = make_int4(wv[0], wv[1], wv[2], wv[3]);
                    }
                }
                // Pass 2: the tail values, gathered into one wave-wide list of cells (a
                // prefix sum of the lanes' counts gives each lane its place), then
                // evaluated 64 at a time, one per lane. The list lives in the scratch's
                // pad columns (WN .. SP-1 of each row, never written by the transpose):
                // 16 cells of 16 bits per row, TL_CAP in all; values beyond it stay in
                // tail_mask for the per-lane rounds below. An encoder's chunk has ~20
                // tail values, so this is one round, where one value per lane per round
                // took max-popcount rounds (~2.2). Measured on MI355X (same box, A/B of
                // whole libraries, bit-identical): FFN-up in the BERT-base encode 196 ->
                // 186 us, config 2's linear 48 -> 45 us per call.
                // The tail pass is a chain of LDS round trips and one long dependent
                // gelu_f32 per lane; at raised wave priority it issues ahead of the other
                // workgroup's wave on the SIMD (config 2, many tails: 43.8 -> 42.2 us per
                // call; the BERT-base encode unchanged to -0.5%).
                __builtin_amdgcn_s_setprio(1);
                {
                    // The prefix sum, bit-sliced: one ballot and one count of the lanes
                    // below per bit of the count (0..32), all VALU and scalar work, where a
                    // 6-step shuffle scan waits on a cross-lane LDS permute per step. Measured
                    // on MI355X, bit-identical: pass 2 10.3K -> 8.3K cycles per tile and wave
                    // on pre-activations of standard deviation 0.5; FFN-up in the BERT-base
                    // encode 177-179 -> 174-175 us.
                    const int cnt = __builtin_popcount(tail_mask);
                    int excl = 0, total = 0;
#pragma unroll
                    for (int b = 0; b < 6; ++b) {
                        const uint64_t bm = __builtin_amdgcn_ballot_w64((cnt >> b) & 1);
                        excl += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bm, 0u)) << b;
                        total += __builtin_popcountll(bm) << b;
                    }
                    if (total != 0) {
                        auto slot = [&](int e) { return reinterpret_cast<uint16_t *>(&scr[(e >> 4) * SP + WN]) + (e & 15); };
                        int pos = excl;
                        uint32_t rest = 0u;
                        for (uint32_t m = tail_mask; m != 0u; m &= m - 1u, ++pos) {
                            const int b = __builtin_ctz(m);
                            if (pos < TL_CAP)
                                *slot(pos) = (uint16_t)((rsub + RPL * (b >> 2)) * SP + 4 * c4 + (b & 3));
                            else
                                rest |= 1u << b;
                        }
                        tail_mask = rest;
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                        // two list rounds at a time, branch-free, so their dependent
                        // chains interleave (a chunk of a wide distribution has several)
                        const int n = min(total, TL_CAP);
                        for (int base = 0; base < n; base += 128) {
                            const int e0 = base + lane, e1 = base + 64 + lane;
                            const int i0 = *slot(min(e0, n - 1));
                            if (base + 64 < n) {
                                const int i1 = *slot(min(e1, n - 1));
                                const float g0 = gelu_f32_offseries(__int_as_float(scr[i0]));
                                const float g1 = gelu_f32_offseries(__int_as_float(scr[i1]));
                                if (e0 < n) scr[i0] = __float_as_int(g0);
                                if (e1 < n) scr[i1] = __float_as_int(g1);
                            } else if (e0 < n) {
                                scr[i0] = __float_as_int(gelu_f32_offseries(__int_as_float(scr[i0])));
                            }
                        }
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    }
                }
                // Pass 2b, only past TL_CAP tail values in the chunk: the rest, one value per
                // lane per round.
                for (;;) {
                    const bool pending = tail_mask != 0u;
                    if (__builtin_amdgcn_ballot_w64(pending) == 0) break;
                    if (pending) {
                        const int b = __builtin_ctz(tail_mask);
                        tail_mask &= tail_mask - 1u;
                        int *cell = &scr[(rsub + RPL * (b >> 2)) * SP + 4 * c4 + (b & 3)];
                        *cell = __float_as_int(gelu_f32(__int_as_float(*cell)));
                    }
                }
                __builtin_amdgcn_s_setprio(0);
                // Pass 3: 16-byte stores of the finished values.
#pragma unroll
                for (int k = 0; k < KR; ++k) v[k] = *reinterpret_cast<const int4 *>(&scr[(rsub + RPL * k) * SP + 4 * c4]);
            } else {
                // all of the chunk's LDS reads first, then the arithmetic
#pragma unroll
                for (int k = 0; k < KR; ++k) v[k] = *reinterpret_cast<const int4 *>(&scr[(rsub + RPL * k) * SP + 4 * c4]);
                if (EPI == EPI_F32 || EPI == EPI_TOPK) {
#pragma unroll
                    for (int k = 0; k < KR; ++k) {
                        const int vv[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
                        v[k].x = __float_as_int(dequant(vv[0], asv[k], wsv[0], bv[0]));
                        v[k].y = __float_as_int(dequant(vv[1], asv[k], wsv[1], bv[1]));
                        v[k].z = __float_as_int(dequant(vv[2], asv[k], wsv[2], bv[2]));
                        v[k].w = __float_as_int(dequant(vv[3], asv[k], wsv[3], bv[3]));
                    }
                }
            }
            // N % 4 == 0 (host check): a lane's 4 columns are all in or all out. Whole
            // tiles store without per-row checks.
            if constexpr (EPI == EPI_TOPK) {
                // The scores are not stored. A score whose key is at or above its row's
                // bound joins the row's candidates. First only the comparisons (bit 4k+j:
                // value j of this lane's row k); the few keepers (the bound is a sample's
                // k-th largest key, so about k of every sample's worth of a row clear it)
                // are then dequantized again from the accumulators still in the scratch,
                // which keeps the common path's registers those of EPI_F32.
                uint32_t keep = 0;
#pragma unroll
                for (int k = 0; k < KR; ++k) {
                    const uint64_t t = s_thr[i * 32 + rsub * KR + k];
                    const float tf = topk_key_score(t);
                    const uint32_t tl = (uint32_t)t;
                    const float x[4] = {__int_as_float(v[k].x), __int_as_float(v[k].y), __int_as_float(v[k].z),
                                        __int_as_float(v[k].w)};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        // key >= t: the score above t's, or equal and the index no larger
                        // (a NaN compares false); t == 0 keeps every non-NaN score
                        const uint32_t lo = 0xffffffffu - (uint32_t)(col + j);
                        const bool in = t == 0 ? x[j] == x[j] : (x[j] > tf || (x[j] == tf && lo >= tl));
                        keep |= in ? 1u << (4 * k + j) : 0u;
                    }
                }
                while (keep != 0u) {
                    const int k = __builtin_ctz(keep) >> 2;
                    const uint32_t grp = (keep >> (4 * k)) & 15u;
                    keep &= ~(15u << (4 * k));
                    if (!row_ok(k)) continue;
                    const int4 a = *reinterpret_cast<const int4 *>(&scr[(rsub + RPL * k) * SP + 4 * c4]);
                    const float as = s_as[i * 32 + rsub * KR + k];
                    const float x[4] = {dequant(a.x, as, wsv[0], bv[0]), dequant(a.y, as, wsv[1], bv[1]),
                                        dequant(a.z, as, wsv[2], bv[2]), dequant(a.w, as, wsv[3], bv[3])};
                    const int64_t row = m0 + i * 32 + rsub + RPL * k;
                    unsigned pos = atomicAdd(&sink.count[row], (unsigned)__builtin_popcount(grp));
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (!((grp >> j) & 1u)) continue;
                        if (pos < (unsigned)sink.cap) {
                            const int64_t at = row * sink.cap + pos;
                            sink.key[at] = ((uint64_t)topk_order(x[j]) << 32) | (0xffffffffu - (uint32_t)(col + j));
                            sink.score[at] = x[j];
                        }
                        ++pos;
                    }
                }
            } else if (full) {
#pragma unroll
                for (int k = 0; k < KR; ++k) store_nt(p0 + k * step, v[k]);
            } else {
#pragma unroll
                for (int k = 0; k < KR; ++k)
                    if (row_ok(k)) store_nt(p0 + k * step, v[k]);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
}

}  // namespace enchip
