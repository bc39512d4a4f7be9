// C entry point over the reference's own NaFlex preprocessing
// (src/siglip2_preproc.cpp, compiled from the reference tree by `make ref`
// into oracle/_ref/): test infrastructure only, used by the CPU tests to pin
// the oracle's restatement (orc_nf_preprocess_rgb) to the reference.
#include <cstdint>
#include <cstring>
#include <string>

#include "siglip2_preproc.h"

extern "C" int ref_nf_preprocess_rgb(const uint8_t *rgb, int h, int w, int max_patches, int p,
                                     float rescale, const float *mean, const float *std_,
                                     float *out, int64_t out_cap, int *n_h, int *n_w) {
    float m[3] = {mean[0], mean[1], mean[2]}, s[3] = {std_[0], std_[1], std_[2]};
    siglip2::PreprocResult r;
    std::string err;
    if (!siglip2::preprocess_image_rgb(rgb, h, w, max_patches, p, rescale, m, s, r, err)) return -1;
    if ((int64_t)r.pixel_values.size() > out_cap) return -1;
    std::memcpy(out, r.pixel_values.data(), r.pixel_values.size() * sizeof(float));
    *n_h = r.n_patches_h;
    *n_w = r.n_patches_w;
    return 0;
}
