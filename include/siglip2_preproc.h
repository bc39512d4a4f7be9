// siglip2_preproc.h -- drop-in siglip2::preprocess_image_rgb over the s2x
// C-ABI: the NaFlex front end (target grid, anti-aliased resize, rescale,
// normalise, patchify) run on the gfx950 GPU.
//
// Same struct and function signatures as the reference
// (src/siglip2_preproc.h:9-55); the output equals the reference's release
// build bit for bit.  Image-file decoding (preprocess_image_file, stb_image
// in the reference) is not part of this library: decode to RGB u8 and call
// preprocess_image_rgb; preprocess_image_file returns false with a message.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace siglip2 {

// pixel_values: n_patches_h * n_patches_w rows of num_channels * patch^2
// floats, channel-last within a patch (the vision encoder's input rows).
struct PreprocResult {
    std::vector<float> pixel_values;
    int                n_patches_h = 0;
    int                n_patches_w = 0;
};

bool preprocess_image_file(
    const std::string & image_path,
    int                 max_num_patches,
    int                 patch_size,
    float               rescale_factor,
    float               image_mean[3],
    float               image_std[3],
    PreprocResult &     out,
    std::string &       error);

// rgb: height x width x 3 u8, channel-last (host memory).  Synchronous.
bool preprocess_image_rgb(
    const uint8_t * rgb,
    int             height,
    int             width,
    int             max_num_patches,
    int             patch_size,
    float           rescale_factor,
    float           image_mean[3],
    float           image_std[3],
    PreprocResult & out,
    std::string &   error);

}  // namespace siglip2
