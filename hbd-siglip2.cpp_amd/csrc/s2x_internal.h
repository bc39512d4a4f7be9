// s2x_internal.h -- host-side internals shared by the C-ABI and the encoders.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "s2x.h"
#include "s2x_kernels.h"

constexpr int64_t QK_ = 32;

// The opaque weight handle of the C-ABI: repacked planes in device memory.
struct s2x_weight {
    s2x::WeightView view;
    void *mem = nullptr;  // base of the planes
    bool owns = false;    // hipFree on destroy
};

namespace s2x {

int fail(int status, const char *fmt, ...);
int hip_fail(hipError_t e, const char *what);
bool aligned(const void *p, size_t a);

inline int64_t round_up_i(int64_t a, int64_t b) { return (a + b - 1) / b * b; }

// Planes of a repacked (K_pad, N) weight in one buffer, each at a 256-byte
// boundary: int8 qs [N][K_pad] and the fp16 bits of d transposed,
// dT [KB][gemm_ld_dw(N)] (columns N.. of each dT row are zero).
struct WeightPlanes {
    size_t qs, dT, total;
};
inline WeightPlanes weight_planes(int64_t K_pad, int64_t N) {
    const int64_t KB = K_pad / QK_;
    WeightPlanes p;
    p.qs = 0;
    p.dT = p.qs + (size_t)round_up_i(K_pad * N, 256);
    p.total = p.dT + (size_t)round_up_i(KB * gemm_ld_dw(N) * 2, 256);
    return p;
}
inline size_t weight_planes_bytes(int64_t K_pad, int64_t N) {
    return weight_planes(K_pad, N).total;
}
inline WeightView planes_view(void *base, int64_t K_pad, int64_t N) {
    const WeightPlanes p = weight_planes(K_pad, N);
    uint8_t *b = reinterpret_cast<uint8_t *>(base);
    WeightView v;
    v.qs = reinterpret_cast<const int8_t *>(b + p.qs);
    v.dT = reinterpret_cast<const uint16_t *>(b + p.dT);
    v.ldT = gemm_ld_dw(N);
    v.K_pad = K_pad;
    v.N = N;
    return v;
}
inline hipError_t repack_into(const void *raw, const WeightView &v, hipStream_t s) {
    return launch_repack_q8_0(raw, v.K_pad, v.N, const_cast<int8_t *>(v.qs),
                              const_cast<uint16_t *>(v.dT), v.ldT, s);
}

// Workspace of the drop-in MUL_MAT: repacked W, then X as Q8_1 (int8
// quants [M][K_pad] and ds words [M][K_pad/32]).
struct MulMatWs {
    size_t w_off, xq_off, ds_off, total;
};
inline MulMatWs mul_mat_ws_layout(int64_t K_pad, int64_t N, int64_t M) {
    MulMatWs L;
    L.w_off = 0;
    L.xq_off = weight_planes_bytes(K_pad, N);
    L.ds_off = L.xq_off + (size_t)round_up_i(M * K_pad, 256);
    L.total = L.ds_off + (size_t)round_up_i(M * (K_pad / QK_) * 4, 256);
    return L;
}

// Upload raw Q8_0 blocks (host or device) and repack into a new owned weight.
// Synchronous with respect to the staging copy; the repack is queued on
// `stream`.
int weight_upload(const void *raw, bool is_host, int64_t K_pad, int64_t N, hipStream_t stream,
                  s2x_weight **out);

}  // namespace s2x
