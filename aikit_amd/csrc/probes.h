// probes.h -- roofline denominators measured on the device that runs the bench
// (the method of gpu/roofline.cu and gpu/roofline_test.go:57-140: vary one thing,
// measure its ceiling, report kernel throughput against the measured figure as well
// as the nameplate one). Integer only, results stored so nothing folds away.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace enchip {

typedef int i32x4_p __attribute__((ext_vector_type(4)));
typedef int i32x16_p __attribute__((ext_vector_type(16)));

// HBM read roof: each block walks chunks of 256 * INFLIGHT 16-byte elements, every thread
// loading INFLIGHT of them (coalesced, nontemporal, all issued before the first is summed),
// over a buffer far larger than the MALL. The kernel time is set by the bytes each CU keeps
// in flight, so the host takes the best of several INFLIGHT values and grid sizes, as the
// HBM-streaming kernels of this library are tuned (gemv_w8a8_wide keeps up to 12 loads in
// flight per lane).
constexpr int PROBE_INFLIGHT = 8;  // the write probe's stores per lane per chunk

template <int INFLIGHT>
__global__ __launch_bounds__(256) void probe_stream_read(const i32x4_p *__restrict__ src, int64_t n16,
                                                         int *__restrict__ sink) {
    constexpr int64_t CH = 256 * INFLIGHT;
    i32x4_p acc = {0, 0, 0, 0};
    int64_t i = (int64_t)blockIdx.x * CH + threadIdx.x;
    for (; i + 256 * (INFLIGHT - 1) < n16; i += (int64_t)gridDim.x * CH) {
        i32x4_p v[INFLIGHT];
#pragma unroll
        for (int j = 0; j < INFLIGHT; ++j) v[j] = __builtin_nontemporal_load(src + i + 256 * j);
#pragma unroll
        for (int j = 0; j < INFLIGHT; ++j) acc += v[j];
    }
    // the last, partial chunk (none when n16 is a multiple of 256 * INFLIGHT)
#pragma unroll
    for (int j = 0; j < INFLIGHT; ++j)
        if (i + 256 * j < n16) acc += src[i + 256 * j];
    if (acc.x + acc.y + acc.z + acc.w == 0x5eed) sink[0] = 1;  // never true for the fill used
}

// f32 VALU issue rate for the non-packed, non-fused operations the bit-exact epilogues
// are made of: 8 independent chains of x = x * z + w (a v_mul_f32 then a v_add_f32, the
// multiply-add left unfused) per lane, enough waves per SIMD to cover the issue latency.
// Counts lane-operations (2 per chain step). The chain constants z and w are held in
// VGPRs, as the epilogues' operands are: on gfx950 two wavefronts of a SIMD issue such
// instructions together (about 28 lanes per clock per SIMD, measured), while an SGPR
// operand, such as a kernel argument used directly, holds the SIMD to one issue at a
// time (about 15).
__global__ __launch_bounds__(256) void probe_valu_f32(float *__restrict__ out, int iters, float a, float b) {
    float x[8], z[8], w[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        x[c] = (float)(threadIdx.x + c);
        z[c] = a * (1.0f + 1e-6f * (float)(c + 1));  // computed by the VALU into VGPRs
        w[c] = b + 1e-6f * (float)(c + 1);
    }
#pragma unroll 4
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < 8; ++c) x[c] = x[c] * z[c] + w[c];
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) s += x[c];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

// HBM write roof: the same chunks, PROBE_INFLIGHT nontemporal 16-byte stores per thread.
__global__ __launch_bounds__(256) void probe_stream_write(i32x4_p *__restrict__ dst, int64_t n16) {
    constexpr int64_t CH = 256 * PROBE_INFLIGHT;
    const i32x4_p v = {1, 2, 3, 4};
    int64_t i = (int64_t)blockIdx.x * CH + threadIdx.x;
    for (; i + 256 * (PROBE_INFLIGHT - 1) < n16; i += (int64_t)gridDim.x * CH) {
#pragma unroll
        for (int j = 0; j < PROBE_INFLIGHT; ++j) __builtin_nontemporal_store(v, dst + i + 256 * j);
    }
#pragma unroll
    for (int j = 0; j < PROBE_INFLIGHT; ++j)
        if (i + 256 * j < n16) dst[i + 256 * j] = v;
}

// A hash of a 32-bit counter (the finaliser of a 32-bit integer hash: xor-shifts and two
// odd multipliers), for operand data made on the device.
__device__ __forceinline__ uint32_t probe_hash(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// Four int8 codes, each the sum of four uniform values in [-32, 31]: bell-shaped, standard
// deviation ~37, in [-128, 124], like a per-token or per-channel quantization of normal
// data (whose codes have standard deviation ~40 for rows of a few hundred values).
__device__ __forceinline__ int probe_codes(uint32_t seed) {
    int w = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t h = probe_hash(seed * 4u + (uint32_t)c);
        int v = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) v += (int)((h >> (8 * k)) & 63u) - 32;
        w |= (v & 0xff) << (8 * c);
    }
    return w;
}

// int8 MFMA issue rate: 8 independent v_mfma_i32_32x32x32_i8 accumulator chains per
// wave (enough to cover the instruction's latency), no memory traffic in the loop.
//   DATA = false: the same small operands in every instruction (the instruction's issue
//     rate at the clock the chip holds with idle multipliers);
//   DATA = true: 8 A and 8 B fragments of bell-shaped codes (probe_codes), a different
//     pair in every instruction: the multipliers switch as they do on real data, and the
//     chip lowers its shader clock under that power (measured on MI355X: ~2.39 GHz with
//     constant operands, ~1.75 GHz with these).
// iters is even. Thread 0 of each block writes the loop's shader-clock ticks
// (s_memtime) and constant-rate ticks (s_memrealtime) to clk[2 * block + {0, 1}].
template <bool DATA>
__global__ __launch_bounds__(256) void probe_mfma_i8(int *__restrict__ out, int iters, long long *__restrict__ clk) {
    i32x4_p a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (DATA) {
            const uint32_t base = ((blockIdx.x * 256u + threadIdx.x) * 16u + (uint32_t)i) * 4u;
            a[i] = (i32x4_p){probe_codes(base), probe_codes(base + 1), probe_codes(base + 2), probe_codes(base + 3)};
            const uint32_t bb = base + 32u;
            b[i] = (i32x4_p){probe_codes(bb), probe_codes(bb + 1), probe_codes(bb + 2), probe_codes(bb + 3)};
        } else {
            a[i] = (i32x4_p){(int)threadIdx.x, 1, 2, 3};
            b[i] = (i32x4_p){3, 2, 1, (int)threadIdx.x};
        }
    }
    i32x16_p acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0;
    const long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; it += 2) {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[(i + 3) & 7], acc[i], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[(i + 5) & 7], b[i], acc[i], 0, 0, 0);
    }
    const long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[i][r];
    out[blockIdx.x * 256 + threadIdx.x] = s;
    if (threadIdx.x == 0) {
        clk[2 * blockIdx.x] = t1 - t0;
        clk[2 * blockIdx.x + 1] = r1 - r0;
    }
}

}  // namespace enchip
