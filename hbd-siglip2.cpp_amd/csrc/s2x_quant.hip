// s2x_quant.hip -- F32->Q8_1 activation quantizer, fused LayerNorm(+Q8_1)
// and the Q8_0 weight repack, for gfx950.
//
// All three are HBM-bound: the quantizer moves 5.125 bytes per element
// (4 in, 1 + 4/32 out), LayerNorm+quantize 5.125 bytes per element of a row.
// Mapping: one 32-value block = 8 consecutive lanes x 4 floats, so a wave
// reads 1 KiB contiguous per instruction and the block amax is a 3-step
// butterfly inside the 8-lane group.
#include <algorithm>

#include "s2x_device.h"
#include "s2x_kernels.h"

#include <type_traits>

namespace s2x {

// ---------------------------------------------------------------------------
// a1: quantizer.  Semantics: src/cuda/siglip2_custom_mmq.cu:63-76 (d, inv,
// round-half-even, clamp) plus the Q8_1 sum s = fp16(sum(q) * d).
// ---------------------------------------------------------------------------
// The block's scale word d | s << 16 at ds [row][ld_ds].
__device__ __forceinline__ void store_scales(const Q81Out &o, int64_t row, int64_t kb, int64_t ld_ds,
                                             float d, int s) {
    o.ds[row * ld_ds + kb] =
        (uint32_t)f32_to_f16_bits(d) | ((uint32_t)f32_to_f16_bits((float)s * d) << 16);
}

__global__ __launch_bounds__(256) void k_quantize_q8_1(
    const float *__restrict__ x, int64_t K, int64_t M, int64_t ldx, int64_t K_pad, Q81Out o,
    int vec4) {
    const int64_t KB = K_pad / QK;
    const int64_t g = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;
    const int sub = threadIdx.x & 7;
    if (g >= M * KB) return;  // whole 8-lane groups leave together
    const int64_t m = g / KB;
    const int64_t kb = g - m * KB;
    const int64_t c = kb * QK + sub * 4;
    const float *xr = x + m * ldx;
    float v0, v1, v2, v3;
    if (vec4 && c + 3 < K) {
        const float4 t = *reinterpret_cast<const float4 *>(xr + c);
        v0 = t.x; v1 = t.y; v2 = t.z; v3 = t.w;
    } else {
        v0 = c + 0 < K ? xr[c + 0] : 0.0f;
        v1 = c + 1 < K ? xr[c + 1] : 0.0f;
        v2 = c + 2 < K ? xr[c + 2] : 0.0f;
        v3 = c + 3 < K ? xr[c + 3] : 0.0f;
    }
    // from 0, as a running fmaxf: NaNs are passed over, a block of NaNs has amax 0
    float a = fmaxf(fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3))), 0.0f);
    a = group8_max(a);
    const float d = a / 127.0f;
    const float inv = a != 0.0f ? 127.0f / a : 0.0f;
    const int q0 = q8_round(v0, inv), q1 = q8_round(v1, inv);
    const int q2 = q8_round(v2, inv), q3 = q8_round(v3, inv);
    *reinterpret_cast<uint32_t *>(o.qs + m * K_pad + c) = pack4_i8(q0, q1, q2, q3);
    const int s = group8_isum(q0 + q1 + q2 + q3);
    if (sub == 0) store_scales(o, m, kb, o.ld_ds, d, s);
}

hipError_t launch_quantize_q8_1(const float *x, int64_t K, int64_t M, int64_t ldx,
                                int64_t K_pad, const Q81Out &o, hipStream_t stream) {
    const int64_t groups = M * (K_pad / QK);
    if (groups == 0) return hipSuccess;
    if (!o.qs || !o.ds) return hipErrorInvalidValue;
    const int vec4 = ((ldx & 3) == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
    const int64_t threads = groups * 8;
    const unsigned grid = (unsigned)((threads + 255) / 256);
    Q81Out oo = o;
    if (oo.ld_ds == 0) oo.ld_ds = K_pad / QK;
    hipLaunchKernelGGL(k_quantize_q8_1, dim3(grid), dim3(256), 0, stream, x, K, M, ldx,
                       K_pad, oo, vec4);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// a2: weight repack.  One thread per 34-byte block: the int8 qs go to a
// 16-byte aligned row-major plane, d's fp16 bits to the transposed plane
// dT [kb][dw_pos(n)] (the GEMM's weight-scale layout: in each group of 64
// columns, columns j and j + 32 share a 32-bit word).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t dw_pos(int64_t n) {
    return (n & ~(int64_t)63) | ((n & 31) << 1) | ((n >> 5) & 1);
}

__global__ __launch_bounds__(256) void k_repack_q8_0(const uint8_t *__restrict__ raw,
                                                     int64_t n_blocks, int64_t KB,
                                                     int8_t *__restrict__ qs,
                                                     uint16_t *__restrict__ dT, int64_t ldT) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_blocks) return;
    const uint16_t *src = reinterpret_cast<const uint16_t *>(raw + i * 34);  // 2-byte aligned
    const int64_t n = i / KB, kb = i - n * KB;
    dT[kb * ldT + dw_pos(n)] = src[0];
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = (uint32_t)src[1 + 2 * j] | ((uint32_t)src[2 + 2 * j] << 16);
    uint4 *dst = reinterpret_cast<uint4 *>(qs + i * QK);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// the padding columns N .. ldT-1 of every dT row
__global__ __launch_bounds__(256) void k_zero_pad_cols(uint16_t *__restrict__ dT, int64_t KB,
                                                        int64_t N, int64_t ldT) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t w = ldT - N;
    if (i >= KB * w) return;
    dT[(i / w) * ldT + dw_pos(N + i % w)] = 0;
}

hipError_t launch_repack_q8_0(const void *raw, int64_t K_pad, int64_t N, int8_t *qs,
                              uint16_t *dT, int64_t ldT, hipStream_t stream) {
    const int64_t KB = K_pad / QK, nb = N * KB;
    if (nb == 0) return hipSuccess;
    hipLaunchKernelGGL(k_repack_q8_0, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0,
                       stream, reinterpret_cast<const uint8_t *>(raw), nb, KB, qs, dT, ldT);
    if (ldT > N)
        hipLaunchKernelGGL(k_zero_pad_cols, dim3((unsigned)((KB * (ldT - N) + 255) / 256)),
                           dim3(256), 0, stream, dT, KB, N, ldT);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// F16 operands of the F16-weight GEMM: f32 activation rows -> f16 (round to
// nearest even, as ggml's F32 -> F16 of the vec_dot operand), and raw F16
// weight rows copied into rows of K_pad halves; both zero past K.  One
// thread per 4 output halves.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_f32_to_f16(const float *__restrict__ x, int64_t K,
                                                    int64_t M, int64_t ldx, int64_t K_pad,
                                                    _Float16 *__restrict__ y) {
    const int64_t q = K_pad / 4;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= M * q) return;
    const int64_t m = i / q, k0 = (i % q) * 4;
    const float *r = x + m * ldx;
    _Float16 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = k0 + j < K ? f32_to_f16(r[k0 + j]) : (_Float16)0.0f;
    *reinterpret_cast<uint2 *>(y + m * K_pad + k0) = __builtin_bit_cast(uint2, v);
}

__global__ __launch_bounds__(256) void k_repack_f16(const uint16_t *__restrict__ raw, int64_t K,
                                                    int64_t N, int64_t K_pad,
                                                    uint16_t *__restrict__ w) {
    const int64_t q = K_pad / 4;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N * q) return;
    const int64_t n = i / q, k0 = (i % q) * 4;
    uint16_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = k0 + j < K ? raw[n * K + k0 + j] : (uint16_t)0;
    *reinterpret_cast<uint2 *>(w + n * K_pad + k0) = __builtin_bit_cast(uint2, v);
}

hipError_t launch_f32_to_f16(const float *x, int64_t K, int64_t M, int64_t ldx, int64_t K_pad,
                             _Float16 *y, hipStream_t stream) {
    const int64_t n = M * (K_pad / 4);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_f32_to_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, x, K,
                       M, ldx, K_pad, y);
    return hipGetLastError();
}

hipError_t launch_repack_f16(const void *raw, int64_t K, int64_t N, int64_t K_pad, _Float16 *w16,
                             hipStream_t stream) {
    const int64_t n = N * (K_pad / 4);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_repack_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       reinterpret_cast<const uint16_t *>(raw), K, N, K_pad,
                       reinterpret_cast<uint16_t *>(w16));
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// a4: LayerNorm(+affine)(+Q8_1).  One wave per row, the row held in
// registers: a two-pass mean / variance (double sums) from wave butterflies, then
// y = ((x - mean) * scale) * w + b rounded after each operation
// (src/siglip2_vision.cpp:79-88 graph; ggml_norm's two-pass variance), then
// the 32-blocks of y quantized by 8-lane groups exactly as k_quantize_q8_1.
// ---------------------------------------------------------------------------
constexpr int LN_MAXIT = 8;        // H <= 8 * 256
constexpr int LN_MAX_BLOCKS = 2048;  // blocks stride over the rows (~3 rows per wave at M = 23,328)
constexpr int64_t LN_WREG_ROWS = 4096;

// Columns per lane in pass it: 4 (256 columns a pass), or TW in the last
// pass.  TW 2 serves rows of 256 k + 128 columns (H = 1,152: four passes of
// 4 columns and one of 2, every lane busy in each) -- the 4-column form's
// last pass would leave half the lanes idle.  A Q8_1 block is then 8 lanes
// of a 4-column pass or 16 of a 2-column one.
template <int NIT, int TW>
__device__ __forceinline__ constexpr int ln_w(int it) {
    return it == NIT - 1 ? TW : 4;
}
// Whether pass it holds the lane's columns c .. c + ln_w(it) - 1 (c = 256
// it + ln_w(it) lane): with NIT = ceil(H / 256), every pass before the last
// lies inside the row, and so does a last pass of 2 columns (H = 256 (NIT -
// 1) + 128), so only a last pass of 4 tests c (a compile-time true
// elsewhere: no exec-mask branch in those passes).
template <int NIT, int TW>
__device__ __forceinline__ bool ln_cols(int it, int64_t c, int64_t H) {
    return it < NIT - 1 || TW == 2 || c < H;
}

// ln_w(it) columns per lane per pass (the rest of v[it] zero); a missing
// row (ok false) or a column past H reads as zeros
template <int NIT, int TW>
__device__ __forceinline__ void ln_load_row(float (&v)[NIT][4], const float *xr, int64_t H,
                                            int lane, bool ok, int vec4) {
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        constexpr int W4 = 4;
        const int W = ln_w<NIT, TW>(it);
        const int64_t c = (int64_t)it * 256 + lane * W;
#pragma unroll
        for (int j = 0; j < W4; ++j) v[it][j] = 0.0f;
        if (ok && ln_cols<NIT, TW>(it, c, H)) {
            if ((vec4 & 1) && W == 4) {
                const float4 t = *reinterpret_cast<const float4 *>(xr + c);
                v[it][0] = t.x; v[it][1] = t.y; v[it][2] = t.z; v[it][3] = t.w;
            } else if ((vec4 & 1) && W == 2) {
                const float2 t = *reinterpret_cast<const float2 *>(xr + c);
                v[it][0] = t.x; v[it][1] = t.y;
            } else {
#pragma unroll
                for (int j = 0; j < W4; ++j)
                    if (j < W) v[it][j] = xr[c + j];
            }
        }
    }
}

// NIT = ceil(H / 256) column passes.  w and b: in LDS, staged once per
// workgroup (WREG false: many rows per wave), or in the registers of the
// lanes' own columns (WREG true: launches of few rows, where the staging
// barrier in front of the first row is most of a wave's time).  Each wave
// walks rows row, row + 4 * gridDim.x, ... and loads its next row before
// reducing the current one, so HBM reads overlap the reductions.
// vec4: bit 0 x rows 16-byte aligned, bit 1 y rows, bit 2 w and b.
// The Q8_1 blocks are quantized with q8_scales and the two-operation
// rounding, then, in a wave where a block's amax fails q8_scales_ok, again
// with the IEEE divisions and the saturating rounding, over the same bytes.
// That amax is taken on the bit patterns of |x| (for non-negative floats
// the integer order is the numeric one, and a NaN sorts above +inf), so a
// block holding a NaN or an infinity fails too: where none does, every
// value is finite and at most amax in magnitude, the two-operation
// rounding's domain, and the amax equals fmaxf's.  The same bits either way.
// AFF: w and b both present (the model's LayerNorms), a kernel of its own:
// instantiated inside one kernel with the general case, the two affine
// forms were merged into one with two selects per element.
template <bool QUANT, bool WRITE_Y, int NIT, bool WREG, int TW, bool AFF>
__global__ __launch_bounds__(256) void k_layernorm(
    const float *__restrict__ x, int64_t H, int64_t M, int64_t ldx,
    const float *__restrict__ w, const float *__restrict__ b, float eps, Q81Out q,
    float *__restrict__ y, int64_t ldy, int vec4) {
    __shared__ __align__(16) float sw[WREG ? 4 : NIT * 256], sb[WREG ? 4 : NIT * 256];
    const int lane = threadIdx.x & 63;
    const int64_t stride = (int64_t)gridDim.x * 4;
    int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    // the first row's loads in flight before w and b are fetched
    float v[NIT][4], wr[NIT][4], br[NIT][4];
    ln_load_row<NIT, TW>(v, x + row * ldx, H, lane, row < M, vec4);
    if constexpr (WREG) {
        // few rows per wave: w and b of the lane's own columns in registers,
        // no staging barrier in front of the first row
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int W = ln_w<NIT, TW>(it);
            const int64_t c = (int64_t)it * 256 + lane * W;
            if ((vec4 & 4) && W == 4 && ln_cols<NIT, TW>(it, c, H)) {  // (H % 32 == 0: c + 3 < H)
                const float4 tw = w ? *reinterpret_cast<const float4 *>(w + c) : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
                const float4 tb = b ? *reinterpret_cast<const float4 *>(b + c) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                wr[it][0] = tw.x; wr[it][1] = tw.y; wr[it][2] = tw.z; wr[it][3] = tw.w;
                br[it][0] = tb.x; br[it][1] = tb.y; br[it][2] = tb.z; br[it][3] = tb.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    wr[it][j] = w && j < W && c + j < H ? w[c + j] : 1.0f;
                    br[it][j] = b && j < W && c + j < H ? b[c + j] : 0.0f;
                }
            }
        }
    } else {
        // many rows per wave: w and b staged once per workgroup in LDS
        for (int i = threadIdx.x; i < H; i += 256) {
            sw[i] = w ? w[i] : 1.0f;
            sb[i] = b ? b[i] : 0.0f;
        }
        __syncthreads();
    }
    // Many rows per wave: the first row's loads complete here, on every
    // path.  Left pending into the loop (the path where the staging loop
    // above does not run), they make the compiler's wait analysis, which
    // merges the loop entry with the back edge, wait for every outstanding
    // load at the top of each iteration -- the next row's, just issued,
    // included -- so that no row's load would overlap the previous row's
    // arithmetic (batch-32 LayerNorm 32.5 -> 30.5 us).  With w and b in
    // registers a wave has one row, and its first sums need only the row.
    if constexpr (!WREG) __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0); expcnt, lgkmcnt: no wait
    for (; row < M; row += stride) {  // wave-uniform
        float vn[NIT][4];
        const int64_t next = row + stride;
        ln_load_row<NIT, TW>(vn, x + next * ldx, H, lane, next < M, vec4);
        // sums in double, as ggml's CPU norm accumulates: the f32 mean and
        // variance then equal the CPU's (the double sum's rounding, whatever
        // its order, is ~1e-16 relative and vanishes in the f32 conversion)
        double s = 0.0;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int W = ln_w<NIT, TW>(it);
            const int64_t c = (int64_t)it * 256 + lane * W;
            if (ln_cols<NIT, TW>(it, c, H)) {
                if (W == 4)
                    s = s + (((double)v[it][0] + (double)v[it][1]) +
                             ((double)v[it][2] + (double)v[it][3]));
                else
                    s = s + ((double)v[it][0] + (double)v[it][1]);
            }
        }
        const float mean = (float)(wave_dsum(s) / (double)H);
        double s2 = 0.0;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int W = ln_w<NIT, TW>(it);
            const int64_t c = (int64_t)it * 256 + lane * W;
            if (ln_cols<NIT, TW>(it, c, H)) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (j >= W) continue;
                    const float t = v[it][j] - mean;
                    s2 = s2 + (double)(t * t);
                }
            }
        }
        const float var = (float)(wave_dsum(s2) / (double)H);
        const float scale = 1.0f / sqrtf(var + eps);
        // every pass normalized first (o), then written; the quantization's
        // form is chosen once per row.  With both w and b (the model's
        // LayerNorms) the affine step has no per-element test: the loop is
        // instantiated for that case and for the general one.
        float o[NIT][4], am[NIT];
        const auto normalize = [&](auto aff_c) {
            constexpr bool AFC = decltype(aff_c)::value;
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int W = ln_w<NIT, TW>(it);
                const int64_t c = (int64_t)it * 256 + lane * W;
                am[it] = 0.0f;
                if (!ln_cols<NIT, TW>(it, c, H)) continue;  // H % 32 == 0: whole 8-lane groups skip together
                float wa[4], ba[4];
                if constexpr (WREG) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        wa[j] = wr[it][j];
                        ba[j] = br[it][j];
                    }
                } else if (W == 4) {
                    const float4 wv = *reinterpret_cast<const float4 *>(sw + c);
                    const float4 bv = *reinterpret_cast<const float4 *>(sb + c);
                    wa[0] = wv.x; wa[1] = wv.y; wa[2] = wv.z; wa[3] = wv.w;
                    ba[0] = bv.x; ba[1] = bv.y; ba[2] = bv.z; ba[3] = bv.w;
                } else {
                    const float2 wv = *reinterpret_cast<const float2 *>(sw + c);
                    const float2 bv = *reinterpret_cast<const float2 *>(sb + c);
                    wa[0] = wv.x; wa[1] = wv.y; wa[2] = wa[3] = 1.0f;
                    ba[0] = bv.x; ba[1] = bv.y; ba[2] = ba[3] = 0.0f;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (j >= W) {
                        o[it][j] = 0.0f;
                        continue;
                    }
                    float t = (v[it][j] - mean) * scale;
                    if (AFC || w) t = t * wa[j];
                    if (AFC || b) t = t + ba[j];  // skipped, not + 0.0f, which would turn -0 into +0
                    o[it][j] = t;
                }
                if (WRITE_Y) {
                    float *yr = y + row * ldy + c;
                    if ((vec4 & 2) && W == 4) {
                        *reinterpret_cast<float4 *>(yr) = make_float4(o[it][0], o[it][1], o[it][2], o[it][3]);
                    } else if ((vec4 & 2) && W == 2) {
                        *reinterpret_cast<float2 *>(yr) = make_float2(o[it][0], o[it][1]);
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            if (j < W) yr[j] = o[it][j];
                    }
                }
                if (QUANT) {
                    uint32_t ab = 0;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (j < W) ab = max(ab, __builtin_bit_cast(uint32_t, o[it][j]) & 0x7fffffffu);
                    am[it] = __builtin_bit_cast(float, W == 4 ? group8_umax(ab) : group16_umax(ab));
                }
            }
        };
        if constexpr (AFF)
            normalize(std::true_type{});
        else
            normalize(std::false_type{});
        if constexpr (QUANT) {
            bool fast = true;
#pragma unroll
            for (int it = 0; it < NIT; ++it) fast = fast & q8_scales_ok(am[it]);  // (no branch per pass)
            const auto quantize = [&](auto fast_c) {
#pragma unroll
                for (int it = 0; it < NIT; ++it) {
                    const int W = ln_w<NIT, TW>(it);
                    const int64_t c = (int64_t)it * 256 + lane * W;
                    if (!ln_cols<NIT, TW>(it, c, H)) continue;
                    float d, inv;
                    int qv[4] = {0, 0, 0, 0};
                    if constexpr (decltype(fast_c)::value) {
                        q8_scales(am[it], d, inv);
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            if (j < W) qv[j] = q8_round_fast(o[it][j], inv);
                    } else {
                        // the amax as a running fmaxf from 0 takes it (a NaN
                        // is passed over; a block of NaNs has amax 0)
                        float a = 0.0f;
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            if (j < W) a = fmaxf(a, fabsf(o[it][j]));
                        a = W == 4 ? group8_max(a) : group16_max(a);
                        d = a / 127.0f;
                        inv = a != 0.0f ? 127.0f / a : 0.0f;
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            if (j < W) qv[j] = q8_round(o[it][j], inv);
                    }
                    int sq;
                    if (W == 4) {
                        *reinterpret_cast<uint32_t *>(q.qs + row * H + c) = pack4_i8(qv[0], qv[1], qv[2], qv[3]);
                        sq = group8_isum(qv[0] + qv[1] + qv[2] + qv[3]);
                    } else {
                        *reinterpret_cast<uint16_t *>(q.qs + row * H + c) =
                            (uint16_t)((qv[0] & 0xff) | ((qv[1] & 0xff) << 8));
                        sq = group16_isum(qv[0] + qv[1]);
                    }
                    if ((lane & (32 / W - 1)) == 0) store_scales(q, row, c / QK, q.ld_ds, d, sq);
                }
            };
            quantize(std::true_type{});
            if (__builtin_amdgcn_ballot_w64(!fast) != 0) quantize(std::false_type{});
        }
#pragma unroll
        for (int it = 0; it < NIT; ++it)
#pragma unroll
            for (int j = 0; j < 4; ++j) v[it][j] = vn[it][j];
    }
}

template <int NIT, bool WREG, int TW>
void launch_ln_cfg(const float *x, int64_t H, int64_t M, int64_t ldx, const float *w,
                   const float *b, float eps, bool quant, const Q81Out &qo, float *y,
                   int64_t ldy, int vec4, dim3 grid, hipStream_t stream) {
    using KFn = void (*)(const float *, int64_t, int64_t, int64_t, const float *, const float *, float,
                         Q81Out, float *, int64_t, int);
    KFn kern;
    if (w && b)
        kern = quant && y ? k_layernorm<true, true, NIT, WREG, TW, true>
               : quant    ? k_layernorm<true, false, NIT, WREG, TW, true>
                          : k_layernorm<false, true, NIT, WREG, TW, true>;
    else
        kern = quant && y ? k_layernorm<true, true, NIT, WREG, TW, false>
               : quant    ? k_layernorm<true, false, NIT, WREG, TW, false>
                          : k_layernorm<false, true, NIT, WREG, TW, false>;
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, x, H, M, ldx, w, b, eps, qo, y, ldy, vec4);
}

template <int NIT>
void launch_ln_nit(const float *x, int64_t H, int64_t M, int64_t ldx, const float *w,
                   const float *b, float eps, bool quant, const Q81Out &qo, float *y,
                   int64_t ldy, int vec4, dim3 grid, hipStream_t stream) {
    // registers for w and b below LN_WREG_ROWS rows (at most ~1.5 rows per wave);
    // rows of 256 k + 128 columns end on a pass of 2 columns per lane
    const bool wreg = M <= LN_WREG_ROWS, tail2 = H % 256 == 128;
    if (wreg && tail2)
        launch_ln_cfg<NIT, true, 2>(x, H, M, ldx, w, b, eps, quant, qo, y, ldy, vec4, grid, stream);
    else if (wreg)
        launch_ln_cfg<NIT, true, 4>(x, H, M, ldx, w, b, eps, quant, qo, y, ldy, vec4, grid, stream);
    else if (tail2)
        launch_ln_cfg<NIT, false, 2>(x, H, M, ldx, w, b, eps, quant, qo, y, ldy, vec4, grid, stream);
    else
        launch_ln_cfg<NIT, false, 4>(x, H, M, ldx, w, b, eps, quant, qo, y, ldy, vec4, grid, stream);
}

hipError_t launch_layernorm(const float *x, int64_t H, int64_t M, int64_t ldx,
                            const float *w, const float *b, float eps, const Q81Out *q,
                            float *y, int64_t ldy, hipStream_t stream) {
    if (M == 0) return hipSuccess;
    int vec4 = ((ldx & 3) == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
    if (y && ((ldy & 3) == 0) && ((reinterpret_cast<uintptr_t>(y) & 15) == 0)) vec4 |= 2;
    if (((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(b)) & 15) == 0) vec4 |= 4;
    if (H <= 0 || H % QK != 0 || H > LN_MAXIT * 256 || (!q && !y)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)std::min<int64_t>((M + 3) / 4, LN_MAX_BLOCKS));
    const bool quant = q != nullptr;
    Q81Out qo = q ? *q : Q81Out{};
    if (quant && (!qo.qs || !qo.ds)) return hipErrorInvalidValue;
    if (quant && qo.ld_ds == 0) qo.ld_ds = H / QK;
    switch ((H + 255) / 256) {
    case 1: launch_ln_nit<1>(x, H, M, ldx, w, b, eps, quant, qo, y, ldy, vec4, grid, stream); break;
    case 2: launch_ln_nit<2>(x, H, M, ldx, w, b, eps, quant, qo, y, ldy, vec4, grid, stream); break;
    case 3: launch_ln_nit<3>(x, H, M, ldx, w, b, eps, quant, qo, y, ldy, vec4, grid, stream); break;
    case 4: launch_ln_nit<4>(x, H, M, ldx, w, b, eps, quant, qo, y, ldy, vec4, grid, stream); break;
    case 5: launch_ln_nit<5>(x, H, M, ldx, w, b, eps, quant, qo, y, ldy, vec4, grid, stream); break;
    case 6: launch_ln_nit<6>(x, H, M, ldx, w, b, eps, quant, qo, y, ldy, vec4, grid, stream); break;
    case 7: launch_ln_nit<7>(x, H, M, ldx, w, b, eps, quant, qo, y, ldy, vec4, grid, stream); break;
    default: launch_ln_nit<8>(x, H, M, ldx, w, b, eps, quant, qo, y, ldy, vec4, grid, stream); break;
    }
    return hipGetLastError();
}

}  // namespace s2x
