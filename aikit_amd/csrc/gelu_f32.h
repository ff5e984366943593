// gelu_f32.h -- exact-erf GELU for the fused GEMM epilogue, bit-identical to
// aikit's linalg.GELUF32 in the default amd64 build.
//
// The reference evaluates a fixed sequence of IEEE float32 operations with no
// multiply-add fusion (linalg/exp.go:81-117 expF32Core, :207-244 ErfF32,
// :260-263 GELUF32). Reproducing that sequence operation for operation, with
// contraction disabled, gives the same bits on gfx950: every v_mul/v_add/v_sub
// rounds to nearest even, and f32 division is compiled to the correctly rounded
// v_div_scale/v_div_fmas/v_div_fixup sequence. The constants are the same
// correctly rounded float32 values the Go compiler derives from the untyped
// constants.
#pragma once

#include <hip/hip_runtime.h>

#include <climits>

#pragma clang fp contract(off)

namespace enchip {

// linalg/exp.go:81-117 expF32Core, for the erf tail (argument -x*x, x in [1,4]) and
// softmax (argument v - max <= 0, possibly -inf or NaN). k = int32(kf) follows Go's
// amd64 conversion: a value outside the int32 range, or NaN, converts to INT32_MIN
// (the hardware's saturating conversion would give INT32_MAX / 0 there), which then
// takes the underflow branch and returns 0, as the reference does.
__device__ __forceinline__ float exp_f32_core(float x) {
    float z = x * 1.4426950408889634f;
    float t = z + 12582912.0f;
    float kf = t - 12582912.0f;
    const int k = (kf >= -2147483648.0f && kf < 2147483648.0f) ? (int)kf : INT_MIN;
    float r = x - kf * 0.693145751953125f - kf * 1.428606820309417e-06f;
    float p = 1.9875691500e-4f;
    p = p * r + 1.3981999507e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    p = p * r * r + r + 1.0f;
    const int e = k + 127;  // k <= 2^31 - 128, so no overflow
    if (e <= 0) return 0.0f;
    if (e >= 255) return p * __uint_as_float((unsigned)(e - 1) << 23) * 2.0f;
    return p * __uint_as_float((unsigned)e << 23);
}

// expF32Core for x <= 0 or NaN (softmax's v - max): bit-identical to exp_f32_core there
// (checked on the CPU over every such float32). kf <= 0, so k < 2^31 and the e >= 255
// branch never taken; p * 2^k by ldexp rounds exactly as the multiply by the power of two.
__device__ __forceinline__ float exp_f32_core_nonpos(float x) {
    float z = x * 1.4426950408889634f;
    float t = z + 12582912.0f;
    float kf = t - 12582912.0f;
    const int k = kf >= -2147483648.0f ? (int)kf : INT_MIN;  // NaN and -inf -> INT_MIN
    float r = x - kf * 0.693145751953125f - kf * 1.428606820309417e-06f;
    float p = 1.9875691500e-4f;
    p = p * r + 1.3981999507e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    p = p * r * r + r + 1.0f;
    return k <= -127 ? 0.0f : ldexpf(p, k);
}

// linalg/exp.go:207-244 ErfF32.
__device__ __forceinline__ float erf_f32(float x) {
    float sign = 1.0f;
    if (x < 0) {
        sign = -1.0f;
        x = -x;
    }
    if (x > 4) return sign;
    if (x < 1) {
        float z = x * x;
        float p = 1.3122532963802806e-08f;
        p = p * z - 1.4503852223150468e-07f;
        p = p * z + 1.4589169000933706e-06f;
        p = p * z - 1.3227513227513228e-05f;
        p = p * z + 1.0683760683760684e-04f;
        p = p * z - 7.5757575757575758e-04f;
        p = p * z + 4.6296296296296294e-03f;
        p = p * z - 2.3809523809523808e-02f;
        p = p * z + 1.0000000000000001e-01f;
        p = p * z - 3.3333333333333331e-01f;
        p = p * z + 1.0f;
        return sign * 1.1283791670955126f * x * p;
    }
    float t = 1.0f / (1.0f + 0.3275911f * x);
    float p = 1.061405429f;
    p = p * t - 1.453152027f;
    p = p * t + 1.421413741f;
    p = p * t - 0.284496736f;
    p = p * t + 0.254829592f;
    return sign * (1.0f - p * t * exp_f32_core(-x * x));
}

// linalg/exp.go:260-263 GELUF32.
__device__ __forceinline__ float gelu_f32(float x) {
    return 0.5f * x * (1.0f + erf_f32(x * 0.7071067811865476f));
}

// exp_f32_core without branches, for the erf tail's argument -x*x: bit-identical to
// exp_f32_core wherever its scaling exponent k is in [-126, 127] (then both return
// p * 2^k by the same multiply), which holds for every argument the tail uses (x in
// [1, 4]: k in [-24, -1]). Elsewhere (|x| > ~9.4, NaN) the result is meaningless; the
// caller discards it (ErfF32 takes its sign branch there, or the value is NaN anyway).
// The branches of exp_f32_core compile to divergent control flow that serialises the
// lanes of a tail list; this form lets two list rounds interleave.
__device__ __forceinline__ float exp_f32_core_tail(float x) {
    float z = x * 1.4426950408889634f;
    float t = z + 12582912.0f;
    float kf = t - 12582912.0f;
    kf = fminf(fmaxf(kf, -126.0f), 127.0f);  // fmaxf(NaN, -126) = -126: no undefined conversion
    const int k = (int)kf;
    float r = x - kf * 0.693145751953125f - kf * 1.428606820309417e-06f;
    float p = 1.9875691500e-4f;
    p = p * r + 1.3981999507e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    p = p * r * r + r + 1.0f;
    return p * __uint_as_float((unsigned)(k + 127) << 23);
}

// gelu_f32 for an argument off ErfF32's series branch (|u| >= 1, u = x * 0.7071067811865476f,
// or NaN), without branches: the erf tail (1 <= |u| <= 4) is evaluated for every such
// argument and the sign branch (|u| > 4) selected, by erf_f32's operations on each branch
// (for |u| > 4 the tail's exp underflows harmlessly, and a NaN takes the tail, as in
// erf_f32; the tail's exp by exp_f32_core_tail, exact there). Branch-free so that several
// independent arguments interleave. Not for |u| < 1.
__device__ __forceinline__ float gelu_f32_offseries(float x) {
    const float u = x * 0.7071067811865476f;
    const float sgn = u < 0 ? -1.0f : 1.0f;
    const float ax = u < 0 ? -u : u;
    const float t = 1.0f / (1.0f + 0.3275911f * ax);
    float p = 1.061405429f;
    p = p * t - 1.453152027f;
    p = p * t + 1.421413741f;
    p = p * t - 0.284496736f;
    p = p * t + 0.254829592f;
    const float tail = sgn * (1.0f - p * t * exp_f32_core_tail(-ax * ax));
    return 0.5f * x * (1.0f + (ax > 4 ? sgn : tail));
}

// GELUF32 for the arguments that take ErfF32's series branch (|u| < 1, u = x *
// 0.7071067811865476f), evaluated without branching. `tail` is set for every other
// argument (|u| >= 1, including ErfF32's |u| > 4 sign branch, and NaN), whose value the
// caller must take from gelu_f32; for them the return value is meaningless. (Those are
// rare in an FFN's pre-activations, and the caller handles them apart, so their branches
// cost nothing here.)
//
// Same bits as gelu_f32 on the series branch:
//   - the series is evaluated on z = u * u, which is |u| * |u|;
//   - sign * 1.1283791670955126f * |u| is rounded exactly as 1.1283791670955126f * u,
//     because rounding is symmetric in sign (u = -0.0 gives -0.0 either way).
__device__ __forceinline__ float gelu_f32_series(float x, bool &tail) {
    const float u = x * 0.7071067811865476f;
    const float z = u * u;
    float p = 1.3122532963802806e-08f;
    p = p * z - 1.4503852223150468e-07f;
    p = p * z + 1.4589169000933706e-06f;
    p = p * z - 1.3227513227513228e-05f;
    p = p * z + 1.0683760683760684e-04f;
    p = p * z - 7.5757575757575758e-04f;
    p = p * z + 4.6296296296296294e-03f;
    p = p * z - 2.3809523809523808e-02f;
    p = p * z + 1.0000000000000001e-01f;
    p = p * z - 3.3333333333333331e-01f;
    p = p * z + 1.0f;
    const float e = 1.1283791670955126f * u * p;
    tail = !(fabsf(u) < 1.0f);
    return 0.5f * x * (1.0f + e);
}

// gelu_f32_series on four arguments at once: the same operations on each lane of the
// vector, so each result is bit-identical to gelu_f32_series on that argument. Written
// on a 4-vector so that the four dependent Horner chains are issued interleaved (with
// packed f32 instructions disabled the backend splits every vector operation into four
// independent scalar ones), which hides each VALU instruction's latency behind the other
// three chains instead of stalling on it. Bit b of the returned mask is set when lane b
// takes another branch (|u| >= 1 or NaN) and must be taken from gelu_f32.
typedef float f32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4v gelu_f32_series4(f32x4v x, uint32_t &tail) {
    const f32x4v u = x * 0.7071067811865476f;
    const f32x4v z = u * u;
    f32x4v p = z * 1.3122532963802806e-08f;  // p0 * z == z * p0 bit for bit
    p = p - 1.4503852223150468e-07f;
    p = p * z + 1.4589169000933706e-06f;
    p = p * z - 1.3227513227513228e-05f;
    p = p * z + 1.0683760683760684e-04f;
    p = p * z - 7.5757575757575758e-04f;
    p = p * z + 4.6296296296296294e-03f;
    p = p * z - 2.3809523809523808e-02f;
    p = p * z + 1.0000000000000001e-01f;
    p = p * z - 3.3333333333333331e-01f;
    p = p * z + 1.0f;
    const f32x4v e = 1.1283791670955126f * u * p;
    tail = (fabsf(u.x) < 1.0f ? 0u : 1u) | (fabsf(u.y) < 1.0f ? 0u : 2u) | (fabsf(u.z) < 1.0f ? 0u : 4u) |
           (fabsf(u.w) < 1.0f ? 0u : 8u);
    return 0.5f * x * (1.0f + e);
}

}  // namespace enchip
