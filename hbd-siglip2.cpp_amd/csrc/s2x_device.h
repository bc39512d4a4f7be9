// s2x_device.h -- device-side helpers shared by the gfx950 kernels.
//
// Every HIP translation unit of the library is compiled with
// -ffp-contract=off: a float expression rounds after each operation, exactly
// as written, and fused multiply-adds appear only as explicit fmaf() calls.
// That keeps the rounding points identical to the CPU restatement of ggml's
// arithmetic that the kernels are checked against.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace s2x {

constexpr int QK = 32;           // Q8_0 / Q8_1 block length
constexpr int WAVE = 64;         // CDNA wavefront

typedef int      v4i  __attribute__((ext_vector_type(4)));
typedef int      v16i __attribute__((ext_vector_type(16)));
typedef float    v4f  __attribute__((ext_vector_type(4)));
typedef float    v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h  __attribute__((ext_vector_type(8)));
typedef _Float16 v4h  __attribute__((ext_vector_type(4)));

// Materialise a value as an f32 register.  The AMDGPU backend otherwise
// folds fptrunc(fmul/fadd ...) into v_fma_mix*_f16, which rounds the exact
// result once to f16 instead of to f32 and then to f16 -- a different value
// at f32 ties -- even with contraction disabled.  The empty asm is opaque to
// that fold and emits no instruction.
__device__ __forceinline__ float f32_materialize(float x) {
    asm("" : "+v"(x));
    return x;
}

// fp32 -> fp16, round-to-nearest-even (v_cvt_f16_f32 under the default mode
// register), subnormals kept, overflow to inf; the argument is first rounded
// to f32 as written.
__device__ __forceinline__ _Float16 f32_to_f16(float f) {
    return (_Float16)f32_materialize(f);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, f32_to_f16(f));
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

// Butterfly reductions over groups of `W` consecutive lanes (W a power of two
// <= 64).  Every lane of the group ends with the group result.
template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, W));
    return v;
}
template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v = v + __shfl_xor(v, o, W);
    return v;
}
template <int W>
__device__ __forceinline__ int group_isum(int v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v = v + __shfl_xor(v, o, W);
    return v;
}

// The Q8_1 rule for one 32-value block given its amax:
//   d = amax/127, inv = amax ? 127/amax : 0, q = rint_half_even(x*inv)
// clamped to [-128, 127] (src/cuda/siglip2_custom_mmq.cu:63-76).
__device__ __forceinline__ int q8_round(float x, float inv) {
    int q = (int)__builtin_rintf(x * inv);
    q = q > 127 ? 127 : q;
    q = q < -128 ? -128 : q;
    return q;
}

__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) |
           ((uint32_t)(c & 0xff) << 16) | ((uint32_t)(d & 0xff) << 24);
}

// GELU tanh form, same expression and operation order as the reference's
// fused epilogue (src/cuda/siglip2_megakernel.cu:276-280).
__device__ __forceinline__ float gelu_tanh(float x) {
    const float GELU_COEF_A = 0.044715f;
    const float SQRT_2_OVER_PI = 0.79788456080286535587989211986876f;
    return 0.5f * x * (1.0f + tanhf(SQRT_2_OVER_PI * x * (1.0f + GELU_COEF_A * x * x)));
}

}  // namespace s2x
