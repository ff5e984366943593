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

// HBM read roof: grid-stride 16-byte loads over a buffer far larger than the MALL.
__global__ __launch_bounds__(256) void probe_stream_read(const i32x4_p *__restrict__ src, int64_t n16,
                                                         int *__restrict__ sink) {
    i32x4_p acc = {0, 0, 0, 0};
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
        acc += src[i];
    if (acc.x + acc.y + acc.z + acc.w == 0x5eed) sink[0] = 1;  // never true for the fill used
}

// HBM write roof: grid-stride 16-byte stores.
__global__ __launch_bounds__(256) void probe_stream_write(i32x4_p *__restrict__ dst, int64_t n16) {
    const i32x4_p v = {1, 2, 3, 4};
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
        dst[i] = v;
}

// int8 MFMA issue rate: 8 independent v_mfma_i32_32x32x32_i8 accumulator chains per
// wave (enough to cover the instruction's latency), no memory traffic in the loop.
__global__ __launch_bounds__(256) void probe_mfma_i8(int *__restrict__ out, int iters) {
    const i32x4_p a = {(int)threadIdx.x, 1, 2, 3}, b = {3, 2, 1, (int)threadIdx.x};
    i32x16_p acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[i], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[i][r];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace enchip
