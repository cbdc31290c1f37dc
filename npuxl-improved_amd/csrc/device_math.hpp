// device_math.hpp - elementwise math shared by every gfx950 kernel.
//
// The activation math is the reference's own published method, not a libm
// call: exp(x) = 2^floor(z) * P5(z - floor(z)) with z = x*log2(e) and P5 the
// degree-5 Taylor polynomial of 2^f (reference src/internal.h:87-110 and its
// AVX2 twin src/kernels/llm.cpp:31-56, which evaluates P5 with FMA Horner as
// done here).  Using a different exp would move SiLU/GELU/softmax by ~1e-4
// relative and break parity with the reference.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace vnpu {
namespace dev {

__device__ __forceinline__ float fast_expf(float x)
{
    // z = x*log2e and f = z - floor(z) round separately, as in every build of
    // the reference (z has a second use, so it is never fused); only the
    // Horner steps are FMAs.
#pragma clang fp contract(off)
    if (x < -80.0f) return 0.0f;
    if (x > 80.0f) return __builtin_inff();
    const float z = x * 1.4426950408889634f;
    const float zi = floorf(z);
    const float f = z - zi;
    float p = fmaf(0.0013333558146428443f, f, 0.009618129107628477f);
    p = fmaf(p, f, 0.05550410866482158f);
    p = fmaf(p, f, 0.2402265069591007f);
    p = fmaf(p, f, 0.6931471805599453f);
    p = fmaf(p, f, 1.0f);
    return ldexpf(p, static_cast<int>(zi));
}

// Correctly rounded f32 multiply and add that the compiler may not fuse
// into an FMA with a neighbouring operation (HIP's __fmul_rn / __fadd_rn are
// plain operators and can be contracted).  Used wherever the result must
// round like the reference's separate multiply and add, e.g. the int8
// dequantize ((float)acc * sa) * sb + bias.
__device__ __forceinline__ float mul_rn(float a, float b)
{
#pragma clang fp contract(off)
    return a * b;
}

__device__ __forceinline__ float add_rn(float a, float b)
{
#pragma clang fp contract(off)
    return a + b;
}

// fast_expf as the reference's baseline x86-64 build evaluates it in code
// without an AVX2 target (its attention_range, llm.cpp:442-546): the same
// steps with every multiply and add of the polynomial rounded separately.
// The range tests are selects, not branches: the polynomial is evaluated for
// every x and discarded outside [-80, 80] (a NaN takes the polynomial, as in
// the reference), so lanes of a wave never diverge here.
__device__ __forceinline__ float fast_expf_unfused(float x)
{
#pragma clang fp contract(off)
    const float z = x * 1.4426950408889634f;
    const float zi = floorf(z);
    const float f = z - zi;
    const float p = 1.0f + f * (0.6931471805599453f +
                    f * (0.2402265069591007f +
                    f * (0.05550410866482158f +
                    f * (0.009618129107628477f +
                    f * 0.0013333558146428443f))));
    const float r = ldexpf(p, static_cast<int>(fminf(fmaxf(zi, -256.0f), 256.0f)));
    return x < -80.0f ? 0.0f : (x > 80.0f ? __builtin_inff() : r);
}

// fast_expf_unfused for x <= 0 or NaN (a softmax weight or rescale factor:
// x = s - max): the same result with the x > 80 test and the upper clamp of
// the exponent dropped, since neither can apply.
__device__ __forceinline__ float fast_expf_nonpos(float x)
{
#pragma clang fp contract(off)
    const float z = x * 1.4426950408889634f;
    const float zi = floorf(z);
    const float f = z - zi;
    const float p = 1.0f + f * (0.6931471805599453f +
                    f * (0.2402265069591007f +
                    f * (0.05550410866482158f +
                    f * (0.009618129107628477f +
                    f * 0.0013333558146428443f))));
    const float r = ldexpf(p, static_cast<int>(fmaxf(zi, -256.0f)));
    return x < -80.0f ? 0.0f : r;
}

// exp256_ps (reference src/kernels/llm.cpp:31-56), the vector exp of the
// reference's AVX2 SWIGLU / GELU / SOFTMAX: x clamped to [-80, 80] (a NaN
// becomes 80, as min_ps/max_ps give), then fast_expf's steps.
__device__ __forceinline__ float exp_avx2(float x)
{
#pragma clang fp contract(off)
    x = fmaxf(fminf(x, 80.0f), -80.0f);
    const float z = x * 1.4426950408889634f;
    const float zi = floorf(z);
    const float f = z - zi;
    float p = fmaf(0.0013333558146428443f, f, 0.009618129107628477f);
    p = fmaf(p, f, 0.05550410866482158f);
    p = fmaf(p, f, 0.2402265069591007f);
    p = fmaf(p, f, 0.6931471805599453f);
    p = fmaf(p, f, 1.0f);
    return ldexpf(p, static_cast<int>(zi));
}

// swiglu_avx2_range (llm.cpp:289-306): s = g / (1 + exp256(-g)), (s*u)*alpha.
__device__ __forceinline__ float swiglu_avx2(float g, float u, float alpha)
{
#pragma clang fp contract(off)
    const float s = g / (1.0f + exp_avx2(-g));
    return (s * u) * alpha;
}

// The scalar tail of swiglu_avx2_range: silu() with the scalar fast_expf
// inlined into the AVX2 function (Horner steps contracted, so dev::fast_expf;
// no clamp: a gate below -80 gives exp = inf and s = -0), then (s*u)*alpha.
__device__ __forceinline__ float swiglu_tail(float g, float u, float alpha)
{
#pragma clang fp contract(off)
    const float s = g / (1.0f + fast_expf(-g));
    return (s * u) * alpha;
}

// gelu_avx2_range (llm.cpp:308-330): inner = k0 * fma(k1, x^3, x),
// t = 2 / (1 + exp256(-2 inner)) - 1, y = (0.5 x)(1 + t).
__device__ __forceinline__ float gelu_avx2(float x)
{
#pragma clang fp contract(off)
    const float x3 = (x * x) * x;
    const float inner = 0.7978845608028654f * fmaf(0.035677408136300125f, x3, x);
    const float e = exp_avx2(-2.0f * inner);
    const float t = 2.0f / (1.0f + e) - 1.0f;
    return (0.5f * x) * (1.0f + t);
}

// reference src/internal.h:112
__device__ __forceinline__ float silu(float x) { return x / (1.0f + fast_expf(-x)); }

// reference src/internal.h:114-121
__device__ __forceinline__ float gelu_tanh(float x)
{
    const float k0 = 0.7978845608028654f;
    const float k1 = 0.035677408136300125f;
    const float x3 = x * x * x;
    const float inner = k0 * (x + k1 * x3);
    const float t = 2.0f / (1.0f + fast_expf(-2.0f * inner)) - 1.0f;
    return 0.5f * x * (1.0f + t);
}

// reference src/internal.h:123-136 (GELU_ERF evaluated as tanh-GELU)
__device__ __forceinline__ float epilogue(float v, uint32_t epi)
{
    switch (epi) {
    case 1: return v > 0.0f ? v : 0.0f;
    case 2: return silu(v);
    case 3:
    case 4: return gelu_tanh(v);
    default: return v;
    }
}

// QUANTIZE_I8 element and scale rules (reference src/kernels/llm.cpp:387-436):
// q = clamp(round_half_away(x * inv), -128, 127) with the correctly rounded
// multiply; scale = max|x| / 127, zero or non-finite -> 1.
__device__ __forceinline__ int8_t q8(float x, float inv)
{
    float q = roundf(mul_rn(x, inv));
    // Plain compares, as the reference: a NaN passes both and converts to 0.
    if (q > 127.0f) q = 127.0f;
    if (q < -128.0f) q = -128.0f;
    return q == q ? static_cast<int8_t>(static_cast<int>(q)) : static_cast<int8_t>(0);
}

__device__ __forceinline__ float scale_from_max(float maxabs)
{
    float scale = __fdiv_rn(maxabs, 127.0f);
    if (!(scale > 0.0f) || !isfinite(scale)) scale = 1.0f;
    return scale;
}

// The scalar tail loop `sum += a[i] * b[i]` of the reference's AVX2
// reductions (rmsnorm_avx2_rows llm.cpp:91, dot_avx2 :342) as its build
// compiles it: g++ -O3 gives the loop a 4-wide vector epilogue, so with four
// or more elements left the first four products are rounded (one vector
// multiply) and added to the sum in order, and the remaining one to three
// (or all of a shorter tail) are contracted into FMAs.
__device__ __forceinline__ float tail_dot(const float *a, const float *b, uint32_t n, float sum)
{
#pragma clang fp contract(off)
    uint32_t i = 0;
    if (n >= 4)
        for (; i < 4; ++i) sum = sum + a[i] * b[i];
    for (; i < n; ++i) sum = fmaf(a[i], b[i], sum);
    return sum;
}

// dot_avx2 (reference src/kernels/llm.cpp:332-343) over d in [0, D): eight
// FMA chains c = 0..7 over d = 8i + c, hsum256's pairing
// ((c0+c4) + (c1+c5)) + ((c2+c6) + (c3+c7)), then the tail d >= D & ~7
// (tail_dot).
__device__ __forceinline__ float dot_ref(const float *q, const float *k, uint32_t D)
{
#pragma clang fp contract(off)
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const uint32_t D8 = D & ~7u;
    for (uint32_t i = 0; i < D8; i += 8) {
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = fmaf(q[i + c], k[i + c], acc[c]);
    }
    const float sum = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
    return tail_dot(q + D8, k + D8, D - D8, sum);
}

// Wave-wide reductions (wave64).
__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

}  // namespace dev
}  // namespace vnpu
