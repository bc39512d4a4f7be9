// siglip2_api.cpp -- siglip2::VisionEncoder / TextEncoder (the reference's
// C++ surface, src/siglip2_vision.h:37-68, src/siglip2_text.h:25-75) as thin
// wrappers over the s2x C-ABI.
#include "siglip2_text.h"
#include "siglip2_vision.h"

namespace siglip2 {

// Read a GGUF file's tower weights (host mapping) and upload them; the
// mapping is released once the encoder holds its device copies.
template <class W, class Bind, class Load>
static bool load_gguf(const std::string &path, Bind bind, Load load, std::string &err) {
    s2x_gguf *g = nullptr;
    if (s2x_gguf_open(path.c_str(), &g) != S2X_OK) {
        err = s2x_last_error();
        return false;
    }
    W w{};
    bool ok = bind(g, &w) == S2X_OK;
    if (!ok) err = s2x_last_error();
    if (ok) ok = load(w);
    s2x_gguf_close(g);
    return ok;
}

VisionEncoder::VisionEncoder() = default;
VisionEncoder::~VisionEncoder() { close(); }

void VisionEncoder::close() {
    s2x_vision_destroy(v_);
    v_ = nullptr;
}

bool VisionEncoder::load(const std::string &gguf_path, bool) {
    close();
    return load_gguf<s2x_vision_weights>(
        gguf_path, s2x_gguf_vision_weights,
        [this](const s2x_vision_weights &w) { return load_weights(w); }, error_msg_);
}

bool VisionEncoder::load_weights(const s2x_vision_weights &w) {
    close();
    if (s2x_vision_create(&w, &v_) != S2X_OK) {
        error_msg_ = s2x_last_error();
        v_ = nullptr;
        return false;
    }
    config_.hidden_size = w.hidden;
    config_.intermediate_size = w.inter;
    config_.num_attention_heads = w.n_head;
    config_.num_hidden_layers = w.n_layer;
    config_.num_patches = w.n_side * w.n_side;
    config_.layer_norm_eps = w.eps;
    return true;
}

bool VisionEncoder::encode(const float *pixel_values, int n_patches_h, int n_patches_w,
                           Pooling pooling, std::vector<float> &out_embedding) {
    if (!v_) {
        error_msg_ = "VisionEncoder not loaded";
        return false;
    }
    if (n_patches_h <= 0 || n_patches_w <= 0) {
        error_msg_ = "n_patches_h and n_patches_w must be positive";
        return false;
    }
    out_embedding.assign((size_t)config_.hidden_size, 0.0f);
    const int pool = pooling == Pooling::PROBE ? S2X_POOL_PROBE : S2X_POOL_MEAN;
    if (s2x_vision_encode(v_, pixel_values, n_patches_h, n_patches_w, pool,
                          out_embedding.data()) != S2X_OK) {
        error_msg_ = s2x_last_error();
        return false;
    }
    return true;
}

bool VisionEncoder::encode_batch_device(const float *pixel_values_dev, int n_images,
                                        int n_patches_h, int n_patches_w, Pooling pooling,
                                        float *out_dev) {
    if (!v_) {
        error_msg_ = "VisionEncoder not loaded";
        return false;
    }
    const int pool = pooling == Pooling::PROBE ? S2X_POOL_PROBE : S2X_POOL_MEAN;
    if (s2x_vision_encode_batch_dev(v_, pixel_values_dev, n_images, n_patches_h, n_patches_w,
                                    pool, out_dev) != S2X_OK) {
        error_msg_ = s2x_last_error();
        return false;
    }
    return true;
}

TextEncoder::TextEncoder() = default;
TextEncoder::~TextEncoder() { close(); }

void TextEncoder::close() {
    s2x_text_destroy(t_);
    t_ = nullptr;
}

bool TextEncoder::load(const std::string &gguf_path, bool) {
    close();
    return load_gguf<s2x_text_weights>(
        gguf_path, s2x_gguf_text_weights,
        [this](const s2x_text_weights &w) { return load_weights(w); }, error_msg_);
}

bool TextEncoder::load_weights(const s2x_text_weights &w) {
    close();
    if (s2x_text_create(&w, &t_) != S2X_OK) {
        error_msg_ = s2x_last_error();
        t_ = nullptr;
        return false;
    }
    config_.hidden_size = w.hidden;
    config_.intermediate_size = w.inter;
    config_.num_attention_heads = w.n_head;
    config_.num_hidden_layers = w.n_layer;
    config_.vocab_size = w.vocab;
    config_.max_position_embeddings = w.max_pos;
    config_.projection_size = w.proj;
    config_.layer_norm_eps = w.eps;
    return true;
}

bool TextEncoder::encode(const int32_t *token_ids, int n_tokens, const int32_t *attention_mask,
                         std::vector<float> &out_embedding) {
    if (!t_) {
        error_msg_ = "TextEncoder not loaded";
        return false;
    }
    out_embedding.assign((size_t)config_.projection_size, 0.0f);
    if (s2x_text_encode(t_, token_ids, n_tokens, attention_mask, out_embedding.data()) != S2X_OK) {
        error_msg_ = s2x_last_error();
        return false;
    }
    return true;
}

bool TextEncoder::encode_batch(const int32_t *token_ids, int n_tokens, int n_batch,
                               const int32_t *attention_mask,
                               std::vector<float> &out_embeddings) {
    if (!t_) {
        error_msg_ = "TextEncoder not loaded";
        return false;
    }
    if (n_batch <= 0) {
        error_msg_ = "n_batch must be > 0";
        return false;
    }
    if (n_batch == 1) return encode(token_ids, n_tokens, attention_mask, out_embeddings);
    if (attention_mask != nullptr) {
        // src/siglip2_text.cpp:766-772
        error_msg_ = "encode_batch with attention_mask is not implemented (HF path doesn't use one)";
        return false;
    }
    out_embeddings.assign((size_t)config_.projection_size * (size_t)n_batch, 0.0f);
    if (s2x_text_encode_batch(t_, token_ids, n_tokens, n_batch, out_embeddings.data()) != S2X_OK) {
        error_msg_ = s2x_last_error();
        return false;
    }
    return true;
}

}  // namespace siglip2
