// siglip2_text.h -- drop-in siglip2::TextEncoder over the s2x C-ABI.
//
// Same class and method signatures as the reference (src/siglip2_text.h:
// 9-75), running on libs2x.so's gfx950 kernels.  Weights come from a
// siglip2 GGUF file (load) or from host tensors (load_weights,
// s2x_text_weights).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "s2x.h"

namespace siglip2 {

struct TextConfig {
    int   hidden_size             = 1152;
    int   intermediate_size       = 4304;
    int   num_attention_heads     = 16;
    int   num_hidden_layers       = 27;
    int   vocab_size              = 256000;
    int   max_position_embeddings = 64;
    int   projection_size         = 1152;
    float layer_norm_eps          = 1e-6f;
};

class TextEncoder {
public:
    TextEncoder();
    ~TextEncoder();
    TextEncoder(const TextEncoder &) = delete;
    TextEncoder &operator=(const TextEncoder &) = delete;

    bool load(const std::string &gguf_path, bool private_backend = false);
    bool load_weights(const s2x_text_weights &w);
    void close();

    const TextConfig &config() const { return config_; }
    const std::string &last_error() const { return error_msg_; }

    // token_ids: n_tokens ids (0 < n_tokens <= max_position_embeddings);
    // attention_mask: n_tokens flags (1 = valid) or nullptr.  Pools the last
    // position (n_tokens - 1), then the head.
    bool encode(const int32_t *token_ids, int n_tokens, const int32_t *attention_mask,
                std::vector<float> &out_embedding);

    // n_batch prompts of n_tokens ids each (batch major); attention_mask must
    // be nullptr, as in the reference.
    bool encode_batch(const int32_t *token_ids, int n_tokens, int n_batch,
                      const int32_t *attention_mask, std::vector<float> &out_embeddings);

private:
    TextConfig config_;
    std::string error_msg_;
    s2x_text *t_ = nullptr;
};

}  // namespace siglip2
