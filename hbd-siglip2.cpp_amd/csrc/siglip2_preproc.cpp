// siglip2_preproc.cpp -- siglip2::preprocess_image_rgb (the reference's C++
// surface, src/siglip2_preproc.h:9-55) over the s2x NaFlex C-ABI: the image
// goes to the device, the GPU kernels resize and patchify it, the rows come
// back to host memory.
#include "siglip2_preproc.h"

#include <hip/hip_runtime.h>

#include "s2x.h"

namespace siglip2 {

namespace {

struct DevMem {
    void *p = nullptr;
    ~DevMem() {
        if (p) (void)hipFree(p);
    }
    bool alloc(size_t n) { return hipMalloc(&p, n ? n : 1) == hipSuccess; }
};

}  // namespace

bool preprocess_image_file(const std::string &image_path, int, int, float, float *, float *,
                           PreprocResult &, std::string &error) {
    error = "preprocess_image_file: image decoding is not part of libs2x (" + image_path +
            "); decode to RGB u8 and call preprocess_image_rgb";
    return false;
}

bool preprocess_image_rgb(const uint8_t *rgb, int height, int width, int max_num_patches,
                          int patch_size, float rescale_factor, float image_mean[3],
                          float image_std[3], PreprocResult &out, std::string &error) {
    if (!rgb || height <= 0 || width <= 0) {
        error = "empty input";
        return false;
    }
    if (patch_size <= 0 || max_num_patches <= 0) {
        error = "invalid patch_size or max_num_patches";
        return false;
    }
    int32_t th = 0, tw = 0;
    if (s2x_nf_target_size(height, width, patch_size, max_num_patches, &th, &tw) != S2X_OK) {
        error = s2x_last_error();
        return false;
    }
    const int64_t n_out = (int64_t)(th / patch_size) * (tw / patch_size) * 3 * patch_size * patch_size;
    const size_t img_bytes = (size_t)height * width * 3;
    const size_t ws_bytes = s2x_nf_workspace_size(height, width, patch_size, max_num_patches);
    DevMem d_rgb, d_out, d_ws;
    if (!d_rgb.alloc(img_bytes) || !d_out.alloc((size_t)n_out * sizeof(float)) ||
        !d_ws.alloc(ws_bytes)) {
        error = "preprocess_image_rgb: device allocation failed";
        return false;
    }
    if (hipMemcpy(d_rgb.p, rgb, img_bytes, hipMemcpyHostToDevice) != hipSuccess) {
        error = "preprocess_image_rgb: upload failed";
        return false;
    }
    int32_t nh = 0, nw = 0;
    if (s2x_nf_preprocess_rgb_dev(static_cast<const uint8_t *>(d_rgb.p), height, width,
                                  max_num_patches, patch_size, rescale_factor, image_mean,
                                  image_std, static_cast<float *>(d_out.p), n_out, &nh, &nw,
                                  d_ws.p, ws_bytes, nullptr) != S2X_OK) {
        error = s2x_last_error();
        return false;
    }
    out.pixel_values.resize((size_t)n_out);
    if (hipMemcpy(out.pixel_values.data(), d_out.p, (size_t)n_out * sizeof(float),
                  hipMemcpyDeviceToHost) != hipSuccess) {
        error = "preprocess_image_rgb: download failed";
        return false;
    }
    out.n_patches_h = nh;
    out.n_patches_w = nw;
    return true;
}

}  // namespace siglip2
