// s2x_misc.hip -- pointwise epilogues, position-embedding resize, Q8_0
// get_rows, pooling and packing helpers for gfx950.  All HBM-bound.
#include <algorithm>

#include "s2x_device.h"
#include "s2x_kernels.h"

namespace s2x {

// ---------------------------------------------------------------------------
// a5: standalone epilogues (src/cuda/siglip2_megakernel.cu:287-315).  The
// GEMM applies the same expressions in its own epilogue; these exist for the
// unfused graph and for callers holding a plain MUL_MAT output.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_bias_residual(const float *__restrict__ mm,
                                                       const float *__restrict__ bias,
                                                       const float *__restrict__ resid,
                                                       float *__restrict__ y, int64_t H,
                                                       int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    y[i] = (mm[i] + bias[i % H]) + resid[i];
}

__global__ __launch_bounds__(256) void k_bias_gelu(const float *__restrict__ mm,
                                                   const float *__restrict__ bias,
                                                   float *__restrict__ y, int64_t H,
                                                   int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    y[i] = gelu_tanh(mm[i] + bias[i % H]);
}

hipError_t launch_bias_residual(const float *mm, const float *bias, const float *resid,
                                float *y, int64_t H, int64_t n_pos, hipStream_t stream) {
    const int64_t total = H * n_pos;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_bias_residual, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       stream, mm, bias, resid, y, H, total);
    return hipGetLastError();
}

hipError_t launch_bias_gelu(const float *mm, const float *bias, float *y, int64_t H,
                            int64_t n_pos, hipStream_t stream) {
    const int64_t total = H * n_pos;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_bias_gelu, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       stream, mm, bias, y, H, total);
    return hipGetLastError();
}

// 16 bytes per thread (grid-stride), then the tail bytes
__global__ __launch_bounds__(256) void k_fill_zero(uint8_t *__restrict__ p, int64_t n16, int64_t bytes) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        reinterpret_cast<uint4 *>(p)[i] = make_uint4(0, 0, 0, 0);
    const int64_t t = n16 * 16 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < bytes) p[t] = 0;
}

hipError_t launch_fill_zero(void *p, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return hipSuccess;
    if (reinterpret_cast<uintptr_t>(p) & 15) return hipErrorInvalidValue;
    const int64_t n16 = (int64_t)(bytes / 16);
    const int64_t blocks = std::min<int64_t>((n16 + 255) / 256 + 1, 8192);
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)blocks), dim3(256), 0, stream,
                       reinterpret_cast<uint8_t *>(p), n16, (int64_t)bytes);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_add(const float *__restrict__ a,
                                             const float *__restrict__ b, float *__restrict__ y,
                                             int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = a[i] + b[i];
}

hipError_t launch_add(const float *a, const float *b, float *y, int64_t n,
                      hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_add, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a, b, y,
                       n);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// a8: anti-aliased bilinear resize, PyTorch F.interpolate(antialias=True,
// align_corners=False) semantics (triangle filter, support max(scale, 1),
// window clipped to the grid and renormalised) -- the HF Siglip2 definition
// of the position-embedding resize that ggml_interpolate(BILINEAR|ANTIALIAS)
// performs in the reference (src/siglip2_vision.cpp:680-690).  Separable:
// the width pass result for each needed source row is recomputed in the
// same order as a two-pass implementation, so both agree bit for bit.
// ---------------------------------------------------------------------------
constexpr int AA_MAXTAPS = 64;

__device__ int aa_taps(int64_t in_size, int64_t out_size, int64_t i, float *w, int *lo_out) {
    const float scale = (float)in_size / (float)out_size;
    const float support = scale >= 1.0f ? scale : 1.0f;
    const float invscale = scale >= 1.0f ? 1.0f / scale : 1.0f;
    const float center = scale * ((float)i + 0.5f);
    int64_t lo = (int64_t)(center - support + 0.5f);
    if (lo < 0) lo = 0;
    int64_t hi = (int64_t)(center + support + 0.5f);
    if (hi > in_size) hi = in_size;
    int n = (int)(hi - lo);
    if (n > AA_MAXTAPS) n = AA_MAXTAPS;
    float total = 0.0f;
    for (int j = 0; j < n; ++j) {
        float t = ((float)(j + lo) - center + 0.5f) * invscale;
        if (t < 0.0f) t = -t;
        const float wt = t < 1.0f ? 1.0f - t : 0.0f;
        w[j] = wt;
        total += wt;
    }
    if (total != 0.0f)
        for (int j = 0; j < n; ++j) w[j] /= total;
    *lo_out = (int)lo;
    return n;
}

__global__ __launch_bounds__(256) void k_resize_pos(const float *__restrict__ pos,
                                                    int64_t n_side, int64_t H, int64_t out_h,
                                                    int64_t out_w, float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= out_h * out_w * H) return;
    const int64_t c = i % H;
    const int64_t x = (i / H) % out_w;
    const int64_t yy = i / (H * out_w);
    float wx[AA_MAXTAPS], wy[AA_MAXTAPS];
    int lx, ly;
    const int nx = aa_taps(n_side, out_w, x, wx, &lx);
    const int ny = aa_taps(n_side, out_h, yy, wy, &ly);
    float acc = 0.0f;
    for (int j = 0; j < ny; ++j) {
        const int64_t sy = ly + j;
        float t = 0.0f;
        for (int k = 0; k < nx; ++k) t += pos[(sy * n_side + lx + k) * H + c] * wx[k];
        acc += t * wy[j];
    }
    out[i] = acc;
}

hipError_t launch_resize_pos_embed(const float *pos, int64_t n_side, int64_t H, int64_t out_h,
                                   int64_t out_w, float *out, hipStream_t stream) {
    const int64_t total = out_h * out_w * H;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_resize_pos, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                       pos, n_side, H, out_h, out_w, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// a11: Q8_0 get_rows: out[i][c] = q * fp16(d) of table row ids[i]
// (ggml dequantize_row_q8_0), plus row (i % add_rows) of `add` if given --
// the token embedding + position embedding of src/siglip2_text.cpp:649-658.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_get_rows_q8_0(const uint8_t *__restrict__ table,
                                                       int64_t K, int64_t n_rows,
                                                       const int32_t *__restrict__ ids,
                                                       int64_t n_ids, const float *__restrict__ add,
                                                       int64_t add_rows, float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_ids * K) return;
    const int64_t r = i / K, c = i % K;
    const int64_t KB = K / QK;
    // ids live in device memory the host cannot check: clamp, never read outside the table
    const int64_t id = min(max((int64_t)ids[r], (int64_t)0), n_rows - 1);
    const uint8_t *blk = table + (id * KB + c / QK) * 34;
    const uint16_t dh = (uint16_t)blk[0] | ((uint16_t)blk[1] << 8);
    float v = (float)(int8_t)blk[2 + c % QK] * f16_bits_to_f32(dh);
    if (add) v = v + add[(r % add_rows) * K + c];
    out[i] = v;
}

hipError_t launch_get_rows_q8_0(const void *table_raw, int64_t K, int64_t n_rows,
                                const int32_t *ids, int64_t n_ids, const float *add,
                                int64_t add_rows, float *out, hipStream_t stream) {
    const int64_t total = n_ids * K;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_get_rows_q8_0, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       stream, reinterpret_cast<const uint8_t *>(table_raw), K, n_rows, ids, n_ids,
                       add, add_rows, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// pooling / packing
// ---------------------------------------------------------------------------
// mean over a segment's rows (ggml_mean: double sum, then float divide;
// src/siglip2_vision.cpp:699-701)
__global__ __launch_bounds__(256) void k_mean_pool(const float *__restrict__ x, int64_t H,
                                                   const int32_t *__restrict__ seg_start,
                                                   const int32_t *__restrict__ seg_len,
                                                   float *__restrict__ out) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int s = blockIdx.y;
    if (c >= H) return;
    const int64_t r0 = seg_start[s];
    const int n = seg_len[s];
    double acc = 0.0;
    for (int p = 0; p < n; ++p) acc += (double)x[(r0 + p) * H + c];
    out[(int64_t)s * H + c] = (float)acc / (float)n;
}

hipError_t launch_mean_pool(const float *x, int64_t H, const int32_t *seg_start,
                            const int32_t *seg_len, int64_t n_seg, float *out,
                            hipStream_t stream) {
    if (n_seg == 0) return hipSuccess;
    hipLaunchKernelGGL(k_mean_pool, dim3((unsigned)((H + 255) / 256), (unsigned)n_seg), dim3(256),
                       0, stream, x, H, seg_start, seg_len, out);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_gather_rows(const float *__restrict__ x, int64_t H,
                                                     const int32_t *__restrict__ rows, int64_t n,
                                                     float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * H) return;
    out[i] = x[(int64_t)rows[i / H] * H + i % H];
}

hipError_t launch_gather_rows(const float *x, int64_t H, const int32_t *rows, int64_t n,
                              float *out, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_gather_rows, dim3((unsigned)((n * H + 255) / 256)), dim3(256), 0, stream,
                       x, H, rows, n, out);
    return hipGetLastError();
}

// one workgroup per (row, segment); float4 copies of a row
__global__ __launch_bounds__(256) void k_pack_rows(const float *__restrict__ padded,
                                                   int64_t row_len, int64_t max_rows,
                                                   const int32_t *__restrict__ seg_start,
                                                   const int32_t *__restrict__ seg_len,
                                                   float *__restrict__ packed) {
    const int p = blockIdx.x, s = blockIdx.y;
    if (p >= seg_len[s]) return;
    const float *src = padded + ((int64_t)s * max_rows + p) * row_len;
    float *dst = packed + ((int64_t)seg_start[s] + p) * row_len;
    for (int64_t c = threadIdx.x; c < row_len; c += blockDim.x) dst[c] = src[c];
}

hipError_t launch_pack_rows(const float *padded, int64_t row_len, int64_t max_rows,
                            const int32_t *seg_start, const int32_t *seg_len, int64_t n_seg,
                            float *packed, hipStream_t stream) {
    if (n_seg == 0) return hipSuccess;
    hipLaunchKernelGGL(k_pack_rows, dim3((unsigned)max_rows, (unsigned)n_seg), dim3(256), 0,
                       stream, padded, row_len, max_rows, seg_start, seg_len, packed);
    return hipGetLastError();
}

}  // namespace s2x
