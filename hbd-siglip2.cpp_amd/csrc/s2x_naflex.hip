// s2x_naflex.hip -- the NaFlex front end on the GPU: target patch grid,
// anti-aliased bilinear resize of an RGB u8 image, rescale + normalise +
// patchify into the vision tower's (n_h*n_w, 3*p*p) channel-last rows.
//
// Algorithm and arithmetic of the reference's src/siglip2_preproc.cpp as its
// release build compiles it (CMakeLists.txt: -O3 -march=native, GCC's default
// contraction): every a*b+c of that file is one fused multiply-add -- in
// double for the filter centres, in float for both filter passes and the
// rescale.  Division and the double-to-float conversions are IEEE on both
// sides, so the output is the reference's bit for bit.
//
//   target grid   largest scale with ceil(h*s/p)*ceil(w*s/p) <= max_patches,
//                 bisection to 1e-5 (:20-53)
//   filter        per output pixel i: centre c = (i + 0.5)*scale - 0.5, taps
//                 k in [ceil(c - r), floor(c + r)], r = max(scale, 1), weight
//                 (float)max(0, 1 - |k - c|/r) * (float)(1/sum) (:76-107)
//   pass 1        along the height, source rows clamped, into floats
//                 (th, w, 3) (:120-139)
//   pass 2        along the width, lrintf, clamped to [0, 255] (:141-166)
//   patchify      v = fma(u8, rescale, -mean) / std at row (y/p)*n_w + x/p,
//                 column ((y%p)*p + x%p)*3 + c (:176-207)
//
// The filters are set up on the GPU, once per output row in pass 1 (per
// block) and once per output column and 16 rows in pass 2 (per thread): two
// passes over the taps, the double sum, then the normalised weights, kept
// in LDS; no tables are built on the host or uploaded.
#include "s2x_device.h"
#include "s2x_kernels.h"

#include <cmath>

namespace s2x {

namespace {

int nf_scaled(double scale, int size, int p) {
    const double v = (double)size * scale;
    const int r = (int)std::ceil(v / (double)p) * p;
    return r > p ? r : p;
}

struct NfAxis {
    double scale, r;  // src/dst, max(scale, 1)
};

__host__ __device__ inline NfAxis nf_axis(int src, int dst) {
    NfAxis a;
    a.scale = (double)src / (double)dst;
    a.r = a.scale > 1.0 ? a.scale : 1.0;
    return a;
}

// The filter of output pixel i: first tap, tap count, 1/sum as float.
struct NfTaps {
    double center;
    int k0, n;
    float inv;
};

__device__ inline NfTaps nf_taps(const NfAxis &a, int i) {
    NfTaps f;
    f.center = fma((double)i + 0.5, a.scale, -0.5);
    f.k0 = (int)ceil(f.center - a.r);
    const int k1 = (int)floor(f.center + a.r);
    f.n = k1 - f.k0 + 1;
    double sum = 0.0;
    for (int t = 0; t < f.n; ++t) {
        const double d = ((double)(f.k0 + t) - f.center) / a.r;
        const double w = 1.0 - fabs(d);
        sum += w > 0.0 ? w : 0.0;
    }
    f.inv = (float)(1.0 / sum);
    return f;
}

__device__ inline float nf_weight(const NfAxis &a, const NfTaps &f, int t) {
    const double d = ((double)(f.k0 + t) - f.center) / a.r;
    const double w = 1.0 - fabs(d);
    return (float)(w > 0.0 ? w : 0.0) * f.inv;
}

// pass 1: tmp[y][x][c]; a block is 256 columns of one output row y
// (blockIdx.x = y, blockIdx.y = column chunk, blockIdx.z = image of a batch
// of same-size images, rgb_stride bytes / tmp_stride floats apart).  The
// row's filter is set up once per block: its tap weights in LDS when there
// are at most NF_MAXT taps, else each thread evaluates them.
constexpr int NF_MAXT = 64;

__global__ __launch_bounds__(256) void k_nf_vpass(const uint8_t *__restrict__ rgb, int h, int w,
                                                  int th, NfAxis ay, float *__restrict__ tmp,
                                                  int64_t rgb_stride, int64_t tmp_stride) {
    __shared__ float wts[NF_MAXT];
    const int y = blockIdx.x, x = blockIdx.y * 256 + threadIdx.x;
    rgb += blockIdx.z * rgb_stride;
    tmp += blockIdx.z * tmp_stride;
    const NfTaps f = nf_taps(ay, y);  // block-uniform
    const bool cached = f.n <= NF_MAXT;
    if (cached) {
        if ((int)threadIdx.x < f.n) wts[threadIdx.x] = nf_weight(ay, f, threadIdx.x);
        __syncthreads();
    }
    if (x >= w) return;
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f;
    for (int t = 0; t < f.n; ++t) {
        int sy = f.k0 + t;
        sy = sy < 0 ? 0 : sy >= h ? h - 1 : sy;
        const float wt = cached ? wts[t] : nf_weight(ay, f, t);
        const uint8_t *sp = rgb + ((int64_t)sy * w + x) * 3;
        a0 = fmaf(wt, (float)sp[0], a0);
        a1 = fmaf(wt, (float)sp[1], a1);
        a2 = fmaf(wt, (float)sp[2], a2);
    }
    float *out = tmp + ((int64_t)y * w + x) * 3;
    out[0] = a0;
    out[1] = a1;
    out[2] = a2;
}

// pass 2 + rescale, normalise, patchify: a block is 256 output columns x
// NF_RY output rows of one image (blockIdx.z as in pass 1, out_stride floats
// between images).  Each thread sets up its column's filter once and keeps
// the tap weights in LDS when there are at most NF_MAXT_H, then walks the
// rows.
constexpr int NF_RY = 16;
constexpr int NF_MAXT_H = 16;

__global__ __launch_bounds__(256) void k_nf_hpass(const float *__restrict__ tmp, int w, int th,
                                                  int tw, NfAxis ax, int p, float rescale,
                                                  float m0, float m1, float m2, float s0,
                                                  float s1, float s2, float *__restrict__ out,
                                                  int64_t tmp_stride, int64_t out_stride) {
    __shared__ float wts[NF_MAXT_H][256];
    const int x = blockIdx.x * 256 + threadIdx.x, y0 = blockIdx.y * NF_RY;
    if (x >= tw) return;  // no block-wide barrier below
    tmp += blockIdx.z * tmp_stride;
    out += blockIdx.z * out_stride;
    const NfTaps f = nf_taps(ax, x);
    const bool cached = f.n <= NF_MAXT_H;
    if (cached)
        for (int t = 0; t < f.n; ++t) wts[t][threadIdx.x] = nf_weight(ax, f, t);
    const float mean[3] = {m0, m1, m2}, stdv[3] = {s0, s1, s2};
    const int nw = tw / p, pw = x / p, px = x - pw * p;
    const int y1 = min(y0 + NF_RY, th);
    for (int y = y0; y < y1; ++y) {
        float a[3] = {0.0f, 0.0f, 0.0f};
        for (int t = 0; t < f.n; ++t) {
            int sx = f.k0 + t;
            sx = sx < 0 ? 0 : sx >= w ? w - 1 : sx;
            const float wt = cached ? wts[t][threadIdx.x] : nf_weight(ax, f, t);
            const float *sp = tmp + ((int64_t)y * w + sx) * 3;
            a[0] = fmaf(wt, sp[0], a[0]);
            a[1] = fmaf(wt, sp[1], a[1]);
            a[2] = fmaf(wt, sp[2], a[2]);
        }
        const int ph = y / p, py = y - ph * p;
        float *dst = out + ((int64_t)ph * nw + pw) * (3 * p * p) + ((int64_t)py * p + px) * 3;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            float r = __builtin_rintf(a[c]);  // lrintf: nearest, ties to even
            r = r < 0.0f ? 0.0f : r > 255.0f ? 255.0f : r;
            dst[c] = fmaf(r, rescale, -mean[c]) / stdv[c];
        }
    }
}

}  // namespace

void nf_target_size(int h, int w, int p, int max_patches, int *out_h, int *out_w) {
    const double eps = 1e-5;
    double lo = eps / 10.0, hi = 100.0;
    while (hi - lo >= eps) {
        const double mid = 0.5 * (lo + hi);
        const long long n =
            (long long)(nf_scaled(mid, h, p) / p) * (long long)(nf_scaled(mid, w, p) / p);
        if (n <= (long long)max_patches)
            lo = mid;
        else
            hi = mid;
    }
    *out_h = nf_scaled(lo, h, p);
    *out_w = nf_scaled(lo, w, p);
}

size_t nf_workspace_bytes(int h, int w, int p, int max_patches) {
    int th = 0, tw = 0;
    nf_target_size(h, w, p, max_patches, &th, &tw);
    return (size_t)th * (size_t)w * 3 * sizeof(float);
}

hipError_t launch_nf_preprocess_batch(const uint8_t *rgb, int n_img, int h, int w,
                                      int max_patches, int p, float rescale, const float mean[3],
                                      const float stdv[3], float *out, int64_t out_cap, int *n_h,
                                      int *n_w, void *ws, size_t ws_bytes, hipStream_t stream) {
    if (!rgb || !out || !ws || n_img <= 0 || n_img > 65535 || h <= 0 || w <= 0 || p <= 0 ||
        max_patches <= 0)
        return hipErrorInvalidValue;
    int th = 0, tw = 0;
    nf_target_size(h, w, p, max_patches, &th, &tw);
    const int nh = th / p, nw = tw / p;
    const int64_t out_stride = (int64_t)nh * nw * 3 * p * p;
    const int64_t tmp_stride = (int64_t)th * w * 3;
    if (out_stride > out_cap || ws_bytes < (size_t)n_img * (size_t)tmp_stride * sizeof(float))
        return hipErrorInvalidValue;
    float *tmp = reinterpret_cast<float *>(ws);
    hipLaunchKernelGGL(k_nf_vpass, dim3((unsigned)th, (unsigned)((w + 255) / 256), (unsigned)n_img),
                       dim3(256), 0, stream, rgb, h, w, th, nf_axis(h, th), tmp,
                       (int64_t)h * w * 3, tmp_stride);
    hipLaunchKernelGGL(k_nf_hpass,
                       dim3((unsigned)((tw + 255) / 256), (unsigned)((th + NF_RY - 1) / NF_RY),
                            (unsigned)n_img),
                       dim3(256),
                       0, stream, tmp, w, th, tw, nf_axis(w, tw), p, rescale, mean[0], mean[1],
                       mean[2], stdv[0], stdv[1], stdv[2], out, tmp_stride, out_stride);
    *n_h = nh;
    *n_w = nw;
    return hipGetLastError();
}

hipError_t launch_nf_preprocess(const uint8_t *rgb, int h, int w, int max_patches, int p,
                                float rescale, const float mean[3], const float stdv[3],
                                float *out, int64_t out_cap, int *n_h, int *n_w, void *ws,
                                size_t ws_bytes, hipStream_t stream) {
    return launch_nf_preprocess_batch(rgb, 1, h, w, max_patches, p, rescale, mean, stdv, out,
                                      out_cap, n_h, n_w, ws, ws_bytes, stream);
}

}  // namespace s2x
