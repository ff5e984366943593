// attention_flash.h -- scaled dot-product attention with an online softmax and split
// products: the flash product modes of enchip_attention_f32_dev (ENCHIP_ATT_FLASH_F16, the
// default, and ENCHIP_ATT_FLASH_BF16), the device form of encoder/attention.go:81-121
// attentionCore up to the context.
//
// One workgroup takes 32 * NW queries of one (head, sequence) and walks that head's keys
// in tiles of FA_KT:
//   * the tile's K and V rows (f32, read once per workgroup) are split into two 16-bit
//     parts, x = hi + lo + e, and staged in LDS, double-buffered, the next tile's loads in
//     flight during this tile's arithmetic. F16: IEEE half parts, |e| <= 2^-22 |x| (for
//     |x| >= 2^-3; 2^-25 absolute below), finite for |x| < 65520. Otherwise bfloat16 parts
//     (as attention_split_bf16 splits them), |e| <= 2^-18 |x|, any finite x;
//   * wavefront w owns queries 32w .. 32w + 31 and computes S^T = K Q^T (the A operand K
//     from LDS, its split Q^T held in registers) on v_mfma_f32_32x32x16_f16 / _bf16, three
//     products per pair (hi.lo' + lo.hi' + hi.hi'). In that accumulator lane l holds
//     query l % 32 and keys 8 (e / 4) + 4 (l / 32) + e % 4 of the 32-key block, so each
//     query's softmax state is the lane's own (plus one exchange between the two lane
//     halves);
//   * online softmax per query in base 2: with c = |scale| log2 e (Q negated when scale
//     < 0), m' = max(m, c max s), p = 2^(fma(s, c, -m')), l' = l 2^(m - m') + sum p, and
//     the context accumulator rescaled by the same factor;
//   * O^T = V^T P^T on the same MFMA: P^T is the B operand straight from the score
//     accumulator registers (its keys in the accumulator's order), V^T the A operand read
//     from LDS, where V is stored transposed with each 16-key block permuted into that
//     same order (fa_perm16), so no lane exchange is needed;
//   * at the end the context is divided by l and stored.
// The arithmetic differs from attentionCore's (exact two-pass softmax, f32 products) in
// the split products, the running maximum, the fused base-2 exponent and the hardware
// 2^x: results agree within the f32 MatmulBT gate (gpu/enccuda/backend_test.go:71-81,
// <= 2e-4 of max(|ref|, 1)), which the tests hold them to. Measured against float64 on
// inputs of standard deviation 2 and 4, the half split stays within that gate and the
// bfloat16 split does not (its three-product error is 2^6 times larger). Any L; head_dim
// 32 or 64. Non-finite operands (and, with F16, operands of magnitude 65520 or more) give
// NaN.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "attention_f32.h"

#pragma clang fp contract(off)

namespace enchip {

constexpr int FA_KT = 64;     // keys per LDS tile
// Wavefronts (32 queries each) per workgroup in the product: 16 (512 queries, 1024
// threads) for 256 < L < 512, and for L > 512 on grids of at least as many workgroups as
// CUs; else 8 (the host's rule, with measurements, is in enchip_attention_f32_dev). Each
// K / V tile is split into LDS once per workgroup, so wider workgroups split each head's
// keys fewer times; narrower ones leave two workgroups per CU whose phases drift apart.
// Up to L = 256, 16 wavefronts would leave half of each workgroup idle.
constexpr int FA_WAVES = 8;
constexpr int FA_WAVES_WIDE = 16;
constexpr int FA_WIDE_L = 256;

// LDS of one stage: K hi / lo planes, FA_KT rows of HD 16-bit parts (row pitch HD*2 + 16 bytes, so
// that 32 lanes' 16-byte reads of 32 rows fall in distinct banks), then V^T hi / lo planes,
// HD rows (one per head-dim column) of FA_KT keys (pitch FA_KT*2 + 16 bytes; each row's
// 16-byte key groups permuted by fa_vswz).
template <int HD>
struct FaLayout {
    static constexpr int KP = HD * 2 + 16;
    static constexpr int VP = FA_KT * 2 + 16;
    static constexpr int KPLANE = FA_KT * KP;
    static constexpr int VPLANE = HD * VP;
    static constexpr int STAGE = 2 * KPLANE + 2 * VPLANE;
    static constexpr int BYTES = 2 * STAGE;
};

__host__ inline int fa_lds_bytes(int hd) {
    return hd == 64 ? FaLayout<64>::BYTES : FaLayout<32>::BYTES;
}

// Position of key kk (0..15 within a 16-key block) in the order the score accumulator
// holds the block's keys as MFMA depth: lane half h has keys 4h..4h+3 and 8+4h..8+4h+3,
// which become depth 8h..8h+7. Even keys map to even positions and kk + 1 to the next one.
__device__ __forceinline__ int fa_perm16(int kk) { return (kk & 3) | ((kk & 8) >> 1) | ((kk & 4) << 1); }

constexpr float FA_LOG2E = 1.4426950408889634f;

// Byte swizzle of row R of the V^T planes: its 16-byte key groups are XOR-permuted by
// (R >> 4) & 3, so a wavefront's transposed stores (16 rows x 4 key pairs) spread over
// twice as many banks (at most 2 lanes per bank instead of 4), while each 16-byte operand
// read stays one aligned group. Measured on MI355X: 195 -> 189 us at BERT-base shape,
// bit-identical.
__device__ __forceinline__ int fa_vswz(int R) { return 16 * ((R >> 4) & 3); }

// NW wavefronts of 32 queries each; a 1-D grid of ceil(L / (32 NW)) * heads * sequences
// workgroups, FaLayout<HD>::BYTES of dynamic LDS, XCD-aware order (the query blocks of one
// (head, sequence) on one XCD). Row i of sequence z, head h starts at q/k/v + (z*L + i)*ld
// + h*HD (16-byte aligned, ld a multiple of 4), out + (z*L + i)*ldo + h*HD; VEC: ldo a
// multiple of 4 and out 16-byte aligned (16-byte stores).
template <int HD, int NW, bool VEC, bool F16>
__global__ __launch_bounds__(64 * NW) void attention_flash(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v, int64_t ld,
    float *__restrict__ out, int64_t ldo, int L, int heads, float scale) {
    static_assert(HD == 32 || HD == 64, "head dimension (and NOT <= 2, which the V^T read swizzle uses)");
    using Lay = FaLayout<HD>;
    constexpr int NT = 64 * NW;
    constexpr int QB = 32 * NW;                 // queries per workgroup
    constexpr int NB = HD / 16;                 // 16-deep head-dim blocks
    constexpr int NOT = HD / 32;                // 32-column tiles of the context
    constexpr int KCH = FA_KT * HD / 8;         // 8-float K chunks per tile
    constexpr int VCH = (FA_KT / 2) * HD / 4;   // (key pair, 4 columns) V items per tile
    constexpr int KPT = (KCH + NT - 1) / NT;    // K chunks per thread
    constexpr int VPT = (VCH + NT - 1) / NT;    // V items per thread
    using Ops = SplitOps<F16>;
    using vec8 = typename Ops::vec8;
    extern __shared__ __attribute__((aligned(16))) char fa_lds[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane & 31, hf = lane >> 5;
    const int nqb = (L + QB - 1) / QB;
    const int logical = xcd_logical_tile(blockIdx.x, gridDim.x);
    const int head = (logical / nqb) % heads;
    const int64_t row0 = (int64_t)(logical / nqb / heads) * L;
    const int qw = (logical % nqb) * QB + 32 * wave;  // this wavefront's first query
    const bool active = qw < L;
    const int nt = (L + FA_KT - 1) / FA_KT;
    const float *kbase = k + row0 * ld + head * HD;
    const float *vbase = v + row0 * ld + head * HD;

    // Q^T, the B operand of S^T = K Q^T: lane (r, hf) holds query qw + r (rows past L
    // re-read row L - 1), head dims 16b + 8hf .. +8 of block b, split.
    // A negative scale is applied as |scale| to -Q (an exact negation), so that the scores'
    // factor c = |scale| log2 e is never negative and the running maximum of the raw scores
    // s gives that of c s.
    // The Q loads are issued here and split after the first K / V tile's loads are issued,
    // so all of them are in flight together (a per-block branch between a load and the next
    // made the compiler wait for each in turn); the negation flips the sign bit (exactly -q,
    // NaN included) without a branch.
    const bool neg = scale < 0.0f;
    const float c = fabsf(scale) * FA_LOG2E;
    vec8 qh[NB], ql[NB];
    float qt[NB][8];
    {
        const float *qrow = q + (row0 + min(qw + r, L - 1)) * ld + head * HD;
#pragma unroll
        for (int b = 0; b < NB; ++b) load8(qrow + 16 * b + 8 * hf, qt[b]);
    }

    // K / V tile staging: loads of tile t into registers, then split into LDS stage s.
    // Keys past L re-read row L - 1 (their scores are masked to -inf, so P = 0).
    f32x4 kr[KPT][2], vr[VPT][2];
    // The tile's base rows are uniform 64-bit pointers; each lane adds a 32-bit offset
    // (key within the tile times ld: the host keeps FA_KT * ld below 2^31).
    const int ld32 = (int)ld;
    auto load_tile = [&](int t) {
        const int kb0 = t * FA_KT, klast = L - 1 - kb0;  // last key of the head, tile-relative
        const float *kt = kbase + (int64_t)kb0 * ld, *vt = vbase + (int64_t)kb0 * ld;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = tid + NT * i;
            if (c < KCH) {
                const int key = min(c / (HD / 8), klast), col = (c % (HD / 8)) * 8;
                const float *p = kt + (key * ld32 + col);
                kr[i][0] = *reinterpret_cast<const f32x4 *>(p);
                kr[i][1] = *reinterpret_cast<const f32x4 *>(p + 4);
            }
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int c = tid + NT * i;
            if (c < VCH) {
                const int pr = c / (HD / 4), col = (c % (HD / 4)) * 4;
                const int k0 = min(2 * pr, klast), k1 = min(2 * pr + 1, klast);
                vr[i][0] = *reinterpret_cast<const f32x4 *>(vt + (k0 * ld32 + col));
                vr[i][1] = *reinterpret_cast<const f32x4 *>(vt + (k1 * ld32 + col));
            }
        }
    };
    auto store_tile = [&](int s) {
        char *khi = fa_lds + s * Lay::STAGE, *klo = khi + Lay::KPLANE;
        char *vhi = klo + Lay::KPLANE, *vlo = vhi + Lay::VPLANE;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = tid + NT * i;
            if (c < KCH) {
                const int key = c / (HD / 8), col = (c % (HD / 8)) * 8;
                const float x[8] = {kr[i][0].x, kr[i][0].y, kr[i][0].z, kr[i][0].w,
                                    kr[i][1].x, kr[i][1].y, kr[i][1].z, kr[i][1].w};
                vec8 h, l;
                Ops::split8(x, h, l);
                *reinterpret_cast<vec8 *>(khi + key * Lay::KP + 2 * col) = h;
                *reinterpret_cast<vec8 *>(klo + key * Lay::KP + 2 * col) = l;
            }
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int c = tid + NT * i;
            if (c < VCH) {
                const int pr = c / (HD / 4), col = (c % (HD / 4)) * 4;
                const int kk = 2 * pr, pos = (kk & ~15) | fa_perm16(kk & 15);  // kk + 1 goes to pos + 1
                const float a[4] = {vr[i][0].x, vr[i][0].y, vr[i][0].z, vr[i][0].w};
                const float b[4] = {vr[i][1].x, vr[i][1].y, vr[i][1].z, vr[i][1].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t hw, lw;
                    Ops::pair(a[j], b[j], hw, lw);
                    const int vo = (col + j) * Lay::VP + ((2 * pos) ^ fa_vswz(col + j));
                    *reinterpret_cast<uint32_t *>(vhi + vo) = hw;
                    *reinterpret_cast<uint32_t *>(vlo + vo) = lw;
                }
            }
        }
    };

    f32x16 o[NOT];
#pragma unroll
    for (int i = 0; i < NOT; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[i][e] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    load_tile(0);
    {
        const uint32_t qsign = neg ? 0x80000000u : 0u;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
#pragma unroll
            for (int i = 0; i < 8; ++i) qt[b][i] = __uint_as_float(__float_as_uint(qt[b][i]) ^ qsign);
            Ops::split8(qt[b], qh[b], ql[b]);
        }
    }
    store_tile(0);
    lds_barrier();
    for (int t = 0; t < nt; ++t) {
        if (t + 1 < nt) load_tile(t + 1);  // in flight during this tile's arithmetic
        if (active) {
            const char *khi = fa_lds + (t & 1) * Lay::STAGE, *klo = khi + Lay::KPLANE;
            const char *vhi = klo + Lay::KPLANE, *vlo = vhi + Lay::VPLANE;
#pragma unroll
            for (int s = 0; s < FA_KT / 32; ++s) {
                const int key0 = t * FA_KT + 32 * s;
                if (key0 >= L) break;  // uniform: no barrier inside
                // ---- S^T for 32 keys x this wavefront's 32 queries
                f32x16 acc;
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const int off = (32 * s + r) * Lay::KP + 2 * (16 * b + 8 * hf);
                    const vec8 kh = *reinterpret_cast<const vec8 *>(khi + off);
                    const vec8 kl = *reinterpret_cast<const vec8 *>(klo + off);
                    acc = mfma_split3(kh, kl, qh[b], ql[b], acc);
                }
                // ---- online softmax of query qw + r over these keys, in base-2 units
                // (y = c s): p = 2^(y - m) with y - m as one fused multiply-add. Keys past L
                // (only in the last sub-tile, a uniform branch) are left out of the maximum
                // and get p = 0.
                // Element e holds key key0 + 4 hf + 8 (e / 4) + e % 4: past L when its
                // constant part 8 (e / 4) + e % 4 reaches lim.
                // (__builtin_expect keeps the mask's 15 compares out of the common path,
                // where the compiler otherwise hoists them.)
                const bool tail = key0 + 32 > L;
                const int lim = L - key0 - 4 * hf;
                if (__builtin_expect(tail, 0)) {
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        if (8 * (e >> 2) + (e & 3) >= lim) acc[e] = -INFINITY;
                }
                float mloc = acc[0];
#pragma unroll
                for (int e = 1; e < 16; ++e) mloc = fmaxf(mloc, acc[e]);
                {  // max with the other lane half's (finite: key0 < L is in it), by
                   // v_permlane32_swap rather than an LDS permute and its wait: measured
                   // 195 -> 189 us at BERT-base shape on MI355X, bit-identical
                    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mloc), __float_as_uint(mloc), false, false);
                    mloc = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
                }
                const float m_new = fmaxf(m_run, mloc * c);      // c >= 0: max of c s = c max s
                const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile
                float x[16];
                float psum = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; ++e) x[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[e], c, -m_new));
                if (__builtin_expect(tail, 0)) {  // also where c = 0 made the masked keys' exponent NaN
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        if (8 * (e >> 2) + (e & 3) >= lim) x[e] = 0.0f;
                }
#pragma unroll
                for (int e = 0; e < 16; ++e) psum += x[e];
                l_run = l_run * alpha + psum;
                m_run = m_new;
                // Unconditional: alpha = 1 leaves o unchanged bit for bit, and without the
                // branch the compiler keeps the sub-tile in one block (no spills at 128 VGPRs).
#pragma unroll
                for (int i = 0; i < NOT; ++i)
#pragma unroll
                    for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
                // ---- O^T += V^T P^T: P^T straight from the accumulator order, split.
                // These MFMAs issue at raised wave priority (the workgroup's waves leave each
                // tile's barrier together, in the same phase): measured 181 against 189 us at
                // BERT-base shape on MI355X; raised for the S^T products instead, or for
                // both, it gained less.
                vec8 ph[2], pl[2];
                Ops::split8(x, ph[0], pl[0]);
                Ops::split8(x + 8, ph[1], pl[1]);
                __builtin_amdgcn_s_setprio(1);
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                    for (int i = 0; i < NOT; ++i) {
                        // = (32 i + r) VP + (2 pos ^ fa_vswz(32 i + r)) for the key position
                        // pos = 32 s + 16 kb + 8 hf: with 2 pos = 64 s + 32 kb +
                        // 16 hf and i < 2 the swizzle is 32 i + 16 (r / 16), so it folds into the
                        // per-lane base and the immediate offset (no extra registers)
                        const int off = (32 * i + r) * Lay::VP + 64 * s + 32 * (kb ^ i) + 16 * (hf ^ (r >> 4));
                        const vec8 vh = *reinterpret_cast<const vec8 *>(vhi + off);
                        const vec8 vl = *reinterpret_cast<const vec8 *>(vlo + off);
                        o[i] = mfma_split3(vh, vl, ph[kb], pl[kb], o[i]);
                    }
                }
                __builtin_amdgcn_s_setprio(0);
            }
        }
        if (t + 1 < nt) store_tile((t + 1) & 1);  // that stage was last read before the previous barrier
        lds_barrier();
    }

    // ---- context = O / l: lane (r, hf) holds query qw + r, columns 32i + 8g + 4hf .. +4
    if (!active) return;
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = 1.0f / l_tot;
    const int qrow = qw + r;
    if (qrow >= L) return;
    float *orow = out + (row0 + qrow) * ldo + head * HD;
#pragma unroll
    for (int i = 0; i < NOT; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int c = 32 * i + 8 * g + 4 * hf;
            const f32x4 val = {o[i][4 * g] * inv, o[i][4 * g + 1] * inv, o[i][4 * g + 2] * inv, o[i][4 * g + 3] * inv};
            if (VEC) {
                *reinterpret_cast<f32x4 *>(orow + c) = val;
            } else {
                orow[c] = val.x;
                orow[c + 1] = val.y;
                orow[c + 2] = val.z;
                orow[c + 3] = val.w;
            }
        }
}

}  // namespace enchip
