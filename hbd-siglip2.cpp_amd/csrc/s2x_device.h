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

typedef int      v2i  __attribute__((ext_vector_type(2)));
typedef uint32_t v4u  __attribute__((ext_vector_type(4)));
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
// DPP lane exchanges (VALU, no LDS round trip).  CTRL: quad_perm codes
// 0x00-0xff, row_half_mirror 0x141 (lane i <-> 7 - i within 8), row_mirror
// 0x140 (i <-> 15 - i within 16), row_bcast15 0x142 / row_bcast31 0x143
// (last lane of the previous row / of lanes 0-31 into the rows of ROW_MASK).
// dpp_i / dpp_f: lanes outside ROW_MASK read 0 (with a full mask the
// compiler folds the exchange into the max / add that consumes it).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, false);
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, dpp_i<CTRL, ROW_MASK>(__builtin_bit_cast(int, v)));
}
// dpp_d: lanes outside ROW_MASK come back undefined (no zero is written into
// them first; a 64-bit add takes no DPP operand, so each zero would cost two
// moves): callers read only the lanes the mask covers.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double dpp_d(double v) {
    const long long b = __builtin_bit_cast(long long, v);
    const int lo = __builtin_amdgcn_mov_dpp((int)b, CTRL, ROW_MASK, 0xf, false);
    const int hi = __builtin_amdgcn_mov_dpp((int)(b >> 32), CTRL, ROW_MASK, 0xf, false);
    return __builtin_bit_cast(double, (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
// max / sum over aligned groups of 8 lanes, result in every lane of the group
__device__ __forceinline__ float group8_max(float v) {
    v = fmaxf(v, dpp_f<0xb1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f<0x4e>(v));   // quad_perm [2,3,0,1]
    return fmaxf(v, dpp_f<0x141>(v));
}
__device__ __forceinline__ uint32_t group8_umax(uint32_t v) {
    v = max(v, (uint32_t)dpp_i<0xb1>((int)v));
    v = max(v, (uint32_t)dpp_i<0x4e>((int)v));
    return max(v, (uint32_t)dpp_i<0x141>((int)v));
}
__device__ __forceinline__ int group8_isum(int v) {
    v = v + dpp_i<0xb1>(v);
    v = v + dpp_i<0x4e>(v);
    return v + dpp_i<0x141>(v);
}
// the same over aligned groups of 16 lanes (the two 8-lane halves of a
// row, joined by row_mirror)
__device__ __forceinline__ float group16_max(float v) {
    v = group8_max(v);
    return fmaxf(v, dpp_f<0x140>(v));
}
__device__ __forceinline__ uint32_t group16_umax(uint32_t v) {
    v = group8_umax(v);
    return max(v, (uint32_t)dpp_i<0x140>((int)v));
}
__device__ __forceinline__ int group16_isum(int v) {
    v = group8_isum(v);
    return v + dpp_i<0x140>(v);
}
// Sum over the wave (64 lanes), returned wave-uniform.  The summation order
// differs from a butterfly; a double sum of f32 terms is exact to ~1e-16
// relative either way.  Row sums in every lane, then rows 1 and 3 add the
// sums of rows 0 and 2 (row_bcast:15) and rows 2 and 3 add lane 31's
// (row_bcast:31): lane 63 holds the total; the lanes outside the masks of
// those two steps are never read again.
__device__ __forceinline__ double wave_dsum(double v) {
    v = v + dpp_d<0xb1>(v);
    v = v + dpp_d<0x4e>(v);
    v = v + dpp_d<0x141>(v);
    v = v + dpp_d<0x140>(v);
    v = v + dpp_d<0x142, 0xa>(v);
    v = v + dpp_d<0x143, 0xc>(v);
    const long long b = __builtin_bit_cast(long long, v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)b, 63);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(b >> 32), 63);
    return __builtin_bit_cast(double, (long long)(((unsigned long long)hi << 32) | lo));
}

template <int W>
__device__ __forceinline__ double group_dsum(double v) {
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
// clamped to [-128, 127] (src/cuda/siglip2_custom_mmq.cu:63-76), the
// conversion saturating (+inf -> 127, -inf -> -128, NaN -> 0) as
// __float2int_rn does: the case of a block whose 127 / amax overflows
// (amax < 127 / FLT_MAX) or whose amax is NaN.  The conversion is the
// instruction v_cvt_i32_f32 itself, whose saturation (values beyond the
// int32 range and +-inf to INT32_MAX / INT32_MIN, NaN to 0) the ISA
// defines; a C++ conversion of such a value would be undefined.
__device__ __forceinline__ int cvt_i32_sat(float r) {
    int q;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(q) : "v"(r));
    return q;
}
__device__ __forceinline__ int q8_round(float x, float inv) {
    int q = cvt_i32_sat(__builtin_rintf(x * inv));
    q = q > 127 ? 127 : q;
    q = q < -128 ? -128 : q;
    return q;
}
// The same for a finite inv, in two VALU operations instead of four.  With
// |x| <= amax the product is at most 127 (1 + 2^-23) in magnitude, so the
// clamp never acts, and rint is the rounding of p + 1.5 * 2^23: floats in
// [2^23, 2^24) are the integers, the add rounds to nearest with ties to
// even as rint does, and leaves 0x4B400000 + rint(p) as the bits (|p| <
// 2^22); the offset, a multiple of 256, drops out of the int8 bytes and of
// integer sums of q.  For the fc1 epilogue, where 16 values of a lane
// share one block's inv: a wave with a non-finite inv in any lane
// (q8_any_sat) takes q8_round instead, a branch the others skip (where
// fewer values share the check -- LayerNorm, the quantizer, attention --
// the branch measured slower than the two operations it saves).
__device__ __forceinline__ int q8_round_fast(float x, float inv) {
    const float p = x * inv;  // rounded to f32 first (no contraction)
    return (int)(__builtin_bit_cast(uint32_t, p + 12582912.0f) - 0x4B400000u);
}
__device__ __forceinline__ bool q8_any_sat(float inv) {
    return __builtin_amdgcn_ballot_w64(!(inv <= 3.40282347e38f)) != 0;
}

// The block scales d = a / 127 and inv = 127 / a (0 for a = 0) of a block
// amax a >= 0, equal to the IEEE quotients bit for bit where q8_scales_ok(a)
// holds (a = 0 or 2^-100 <= a <= 2^100), in about half the VALU operations
// of two IEEE divisions.  Markstein's division (P. Markstein, IA-64 and
// Elementary Functions, 2000, ch. 8):
//   d:   q0 = a RN(1/127), corrected by the exact remainder a - 127 q0 --
//        a / 127 for every positive float a;
//   inv: r0 = v_rcp_f32(a) (within 1 ulp of 1 / a), the quotient p0 =
//        127 r0 corrected by its exact remainder 127 - a p0 -- 127 / a for
//        every significand of a and either float next to 1 / a as r0 (with
//        the numerator fixed at 127 the correction needs no Newton step on
//        r0); every step scales exactly by a power of two while its values
//        stay normal, which holds for a in [2^-121, 2^126].
// Both were checked over those inputs on the CPU
// (tests/test_q8_scales_division.py).
__device__ __forceinline__ bool q8_scales_ok(float a) {
    return (a == 0.0f) | ((a >= 0x1p-100f) & (a <= 0x1p100f));  // (bitwise: no branches)
}
__device__ __forceinline__ void q8_scales(float a, float &d, float &inv) {
    const float r127 = 0x1.020408p-7f;  // RN(1/127)
    const float q0 = a * r127;
    d = fmaf(fmaf(-127.0f, q0, a), r127, q0);
    const float r0 = __builtin_amdgcn_rcpf(a);
    const float p0 = 127.0f * r0;
    const float p = fmaf(fmaf(-a, p0, 127.0f), r0, p0);
    inv = a != 0.0f ? p : 0.0f;
}

__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) |
           ((uint32_t)(c & 0xff) << 16) | ((uint32_t)(d & 0xff) << 24);
}

// tanh in f32 from IEEE primitives only (mul, add, fma, divide, rint,
// ldexp), so that it rounds identically on every IEEE machine:
//   |u| < 0.5 : Maclaurin series of tanh through u^15 (coefficients are the
//               exact series terms 2^2n (2^2n - 1) B_2n / (2n)!), Horner in
//               z = u^2; truncation error < 1e-8 relative
//   |u| < 9   : (e - 1) / (e + 1), e = e^(2|u|) by Cody-Waite reduction
//               t = k ln2 + r (ln2 split into a 9-bit head and a tail) and
//               the degree-7 Taylor polynomial of e^r, |r| <= ln2/2
//   |u| >= 9  : +-1 (tanh(9) rounds to 1 in f32)
// Accuracy: within 3 ulp of tanh.
__device__ __forceinline__ float exp_cw(float t) {
    const float k = __builtin_rintf(t * 1.44269504088896341f);
    float r = fmaf(-k, 0.693359375f, t);
    r = fmaf(-k, -2.12194440e-4f, r);
    float p = 1.0f / 5040.0f;
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)k);
}
__device__ __forceinline__ float tanh_f32(float u) {
    const float a = fabsf(u);
    float r;
    if (a >= 9.0f) {
        r = 1.0f;
    } else if (a < 0.5f) {
        const float z = a * a;
        float p = -929569.0f / 638512875.0f;
        p = fmaf(p, z, 21844.0f / 6081075.0f);
        p = fmaf(p, z, -1382.0f / 155925.0f);
        p = fmaf(p, z, 62.0f / 2835.0f);
        p = fmaf(p, z, -17.0f / 315.0f);
        p = fmaf(p, z, 2.0f / 15.0f);
        p = fmaf(p, z, -1.0f / 3.0f);
        r = fmaf(a * z, p, a);
    } else {
        const float e = exp_cw(2.0f * a);
        r = (e - 1.0f) / (e + 1.0f);
    }
    return __builtin_copysignf(r, u);
}

// x / y correctly rounded, for the operands of gelu_tanh only: y = 1 + e with
// e in [0, e^87] (y in [1, 2^126): 1 / y is normal), and y = 2 exactly
// whenever |x| < 2^-25.  Markstein's division (P. Markstein, IA-64 and
// Elementary Functions, 2000, ch. 8): v_rcp_f32 (within 1 ulp of 1 / y),
// one Newton step r1 = r0 + r0 (1 - y r0), the quotient q0 = x r1 and its
// correction by the exact remainder x - y q0.  Outside this domain it can
// miss the rounding: y with an all-ones significand (when v_rcp_f32 returns
// the lower neighbour of 1 / y, the Newton step stays there), or a remainder
// below the normal range (|x| < 2^-100 with y not a power of two).  Every
// float x in [-2^10, -2^7) and with 2^-30 <= |x| < 2^7 was checked against
// the IEEE quotient through gelu_tanh itself; below 2^-30 y is 2, above 2^7
// it is 1 or the constant of the clamp.  Six VALU operations where the
// general IEEE division takes ten.
__device__ __forceinline__ float div_gelu(float x, float y) {
    const float r0 = __builtin_amdgcn_rcpf(y);
    const float r1 = fmaf(fmaf(-y, r0, 1.0f), r0, r0);
    const float q0 = x * r1;
    return fmaf(fmaf(-y, q0, x), r1, q0);
}

// GELU tanh form: the reference's inner argument g
// (src/cuda/siglip2_megakernel.cu:276-280) through 0.5 x (1 + tanh(g)) =
// x / (1 + e^(-2g)) -- one exp_cw, one division, no branch; the same
// operations as the CPU restatement, so the bits agree.  t = -2 g is
// formed as ((-2 sqrt(2/pi)) x) (1 + a x x): scaling by -2 commutes with
// each rounding, so these are the bits of -2 * g.  The clamp's upper end,
// 87, keeps 1 + e^t below 2^126 (the domain of div_gelu); e^-17 is already
// below half an ulp of 1, so the lower end (-100) changes nothing.
__device__ __forceinline__ float gelu_tanh(float x) {
    const float GELU_COEF_A = 0.044715f;
    const float SQRT_2_OVER_PI = 0.79788456080286535587989211986876f;
    const float t = ((-2.0f * SQRT_2_OVER_PI) * x) * (1.0f + GELU_COEF_A * x * x);
    return div_gelu(x, 1.0f + exp_cw(fminf(fmaxf(t, -100.0f), 87.0f)));
}

// a / b for 0 <= a < 2^20 and b >= 1, exact: the float estimate a * (1/b)
// is within a/b * 2^-23 <= 1/8 of a/b, so one correction either way suffices
__device__ __forceinline__ int small_div(int a, int b, float inv_b) {
    int q = (int)((float)a * inv_b);
    const int r = a - q * b;
    q += (r >= b) - (r < 0);
    return q;
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup b runs on
// XCD b % 8), each with its own L2.  xcd_linear(b, G) renumbers the G
// workgroups of a launch so that each XCD takes one contiguous range of the
// new order: workgroups adjacent in it share their XCD's L2 (a bijection on
// 0 .. G-1; XCDs below G % 8 take one index more).
__device__ __forceinline__ int xcd_linear(int bid, int G) {
    constexpr int NX = 8;
    if (G < NX) return bid;
    const int xcd = bid % NX, local = bid / NX;
    const int per = G / NX, rem = G % NX;
    return xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

}  // namespace s2x
