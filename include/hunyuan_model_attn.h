// hunyuan_model_attn.h -- the attention half, the decoder layer and the backbone
// helpers of the reference's src/hunyuan_model.h, src/hunyuan_image_gen.h and
// src/hunyuan_full_model.h, served by the MI355X library with the reference's names,
// signatures and struct layouts.  Host arrays in and out; each call runs on the GPU
// through hy_attn.h / hy_moe.h and blocks until done.  The arithmetic is fp32 in
// another summation order than the reference's loops (results agree to float
// rounding); the MoE half keeps its exact q semantics.
//
// A code base that keeps its own headers does not include this file: the
// declarations are the same, and the definitions link from libhy_moe.so.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "hunyuan_model_moe.h"
#include "hy_attn.h"

// src/hunyuan_model.h:93-101
struct AttentionWeights {
    std::vector<float> qkv_weight;  // [qkv_total, hidden_size]
    std::vector<float> o_weight;    // [hidden_size, hidden_size_q]
    std::vector<float> q_norm_weight;
    std::vector<float> k_norm_weight;
};

// src/hunyuan_model.h:161-174
struct DecoderLayerWeights {
    std::vector<float> input_ln_weight;      // [hidden_size]
    std::vector<float> post_attn_ln_weight;  // [hidden_size]
    AttentionWeights attn;
    MoEWeights moe;
    // safetensors shard reader of the reference; declared for API parity, not provided
    // by this library (weights come from GGUF files or host arrays)
    bool load(int layer_idx, const std::string& shard_path);
};

// src/hunyuan_model.h:80-88 / src/rms_norm.cpp:97-152 (q, k rotated in place)
void rope_f32(float* q, float* k, uint32_t seq_len, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
              float theta, const int* positions);
// src/hunyuan_model.h:103-113 / src/attention.cpp:10-185
void attention_forward_cpu(const float* hidden_states, const AttentionWeights& w, uint32_t n_tokens,
                           const HunyuanConfig& cfg, const int* positions, float* output, float* debug_q = nullptr,
                           float* debug_k = nullptr, float* debug_v = nullptr);
// src/hunyuan_model.h:176-182 / src/decoder_layer.cpp:9-48
void decoder_layer_forward_cpu(const float* hidden_states, const DecoderLayerWeights& w, uint32_t n_tokens,
                               const HunyuanConfig& cfg, const int* positions, float* output);
// src/hunyuan_image_gen.h:15-34 / src/hunyuan_image_gen.cpp:11-117
void build_2d_rope(uint32_t seq_len, uint32_t n_elem, uint32_t text_len, uint32_t img_h, uint32_t img_w, float base,
                   float* cos_out, float* sin_out);
void apply_rope_2d_f32(float* q, float* k, const float* cos, const float* sin, uint32_t n_tokens, uint32_t n_heads,
                       uint32_t n_kv_heads, uint32_t head_dim);
// src/hunyuan_full_model.h:105-121 / src/hunyuan_full_model.cpp:276-318
void embedding_lookup_f32(const int* input_ids, const float* embedding_table, float* out, uint32_t n_tokens,
                          uint32_t hidden_size);
void lm_head_f32(const float* hidden_states, const float* lm_head_weight, float* logits, uint32_t n_tokens,
                 uint32_t hidden_size, uint32_t vocab_size);

namespace hy {

// RAII handle of the resident backbone (hy_model_*): HunyuanFullModel's forward with
// every weight on the device.  Throws hy::Error on failure.
class Backbone {
public:
    explicit Backbone(const hy_model_config& cfg);
    ~Backbone();
    Backbone(const Backbone&) = delete;
    Backbone& operator=(const Backbone&) = delete;
    hy_attn_ctx* attn() { return hy_model_attn(ctx_); }
    hy_moe_ctx* moe() { return hy_model_moe(ctx_); }
    void upload_globals(const float* embedding, const float* final_norm, const float* lm_head);
    // layer l from DecoderLayerWeights (F32 MoE weights require a model created with
    // wtype HY_TYPE_F32)
    void upload_layer(uint32_t layer, const DecoderLayerWeights& w, const HunyuanConfig& cfg);
    // device pointers, stream-ordered
    void forward(const int32_t* ids_dev, uint32_t T, const int32_t* positions_dev, float* logits_dev,
                 void* stream = nullptr);
    hy_model_ctx* handle() { return ctx_; }

private:
    hy_model_ctx* ctx_ = nullptr;
};

}  // namespace hy
