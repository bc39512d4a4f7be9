// siglip2_vision.h -- drop-in siglip2::VisionEncoder over the s2x C-ABI.
//
// Same class, enum and method signatures as the reference
// (src/siglip2_vision.h:9-68); the encoder runs on the gfx950 kernels of
// libs2x.so.  Weights come from a siglip2 GGUF file (load) or from host
// tensors (load_weights: raw Q8_0 blocks and f32, s2x_vision_weights).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "s2x.h"

namespace siglip2 {

enum class Pooling {
    MEAN,   // mean over patches (HF last_hidden_state.mean(dim=1))
    PROBE,  // Siglip2MultiheadAttentionPoolingHead
};

struct VisionConfig {
    int   hidden_size         = 1152;
    int   intermediate_size   = 4304;
    int   num_attention_heads = 16;
    int   num_hidden_layers   = 27;
    int   patch_size          = 16;
    int   num_patches         = 256;  // native 16x16 grid
    int   num_channels        = 3;
    float layer_norm_eps      = 1e-6f;
};

class VisionEncoder {
public:
    VisionEncoder();
    ~VisionEncoder();
    VisionEncoder(const VisionEncoder &) = delete;
    VisionEncoder &operator=(const VisionEncoder &) = delete;

    // Reference entry point: read the vision tower of a siglip2 GGUF file
    // (s2x_gguf_*) and upload it.  private_backend is accepted and ignored
    // (the encoder always owns its HIP stream).
    bool load(const std::string &gguf_path, bool private_backend = false);
    // Upload + repack the weights onto the current HIP device.
    bool load_weights(const s2x_vision_weights &w);
    void close();

    const VisionConfig &config() const { return config_; }
    const std::string &last_error() const { return error_msg_; }

    // pixel_values: host fp32 [n_patches, num_channels*patch_size^2],
    // n_patches == n_patches_h * n_patches_w.  Synchronous.
    bool encode(const float *pixel_values, int n_patches_h, int n_patches_w, Pooling pooling,
                std::vector<float> &out_embedding);

    // Device-resident batch of n_images images of one grid; out_dev
    // [n_images, hidden].  Asynchronous on the encoder's stream.
    bool encode_batch_device(const float *pixel_values_dev, int n_images, int n_patches_h,
                             int n_patches_w, Pooling pooling, float *out_dev);

    s2x_vision *handle() const { return v_; }

private:
    VisionConfig config_;
    std::string error_msg_;
    s2x_vision *v_ = nullptr;
};

}  // namespace siglip2
