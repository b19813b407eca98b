// hunyuan_model_moe.h -- the MoE part of the reference's src/hunyuan_model.h, served
// by the MI355X library: HunyuanConfig, MoEWeights, swiglu_ffn_f32, moe_forward_cpu and
// rms_norm_f32 with the reference's names, signatures and struct layouts.  Host arrays
// in and out; each call runs on the GPU through hy_moe.h and blocks until done.
//
// A code base that keeps its own hunyuan_model.h does not include this file: its
// declarations are the same, and the definitions link from libhy_moe.so.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

// src/hunyuan_model.h:13-45, field for field (same order, types and defaults), so the
// reference's own declaration and this one describe the same object layout.
struct HunyuanConfig {
    uint32_t hidden_size = 4096;
    uint32_t num_hidden_layers = 32;
    uint32_t num_attention_heads = 32;
    uint32_t num_key_value_heads = 8;
    uint32_t attention_head_dim = 128;
    uint32_t intermediate_size = 3072;
    uint32_t moe_intermediate_size = 3072;
    uint32_t num_experts = 64;
    uint32_t moe_topk = 8;
    uint32_t num_shared_expert = 1;
    uint32_t vocab_size = 133120;
    uint32_t max_position_embeddings = 22800;
    float rms_norm_eps = 1e-5f;
    float rope_theta = 10000.0f;
    bool use_qk_norm = true;
    bool use_mixed_mlp_moe = true;

    // Derived
    uint32_t num_kv_groups;
    uint32_t hidden_size_q;   // num_heads * head_dim
    uint32_t hidden_size_kv;  // num_kv_heads * head_dim
    uint32_t qkv_total;       // hidden_size_q + 2 * hidden_size_kv

    void compute_derived() {
        num_kv_groups = num_attention_heads / num_key_value_heads;
        hidden_size_q = num_attention_heads * attention_head_dim;
        hidden_size_kv = num_key_value_heads * attention_head_dim;
        qkv_total = hidden_size_q + 2 * hidden_size_kv;
    }

    // config.json reader of the reference (src/hunyuan_model.cpp); declared for layout
    // and API parity, not provided by this library.
    static HunyuanConfig from_json(const std::string& path);
};

// src/hunyuan_model.h:130-145
struct MoEWeights {
    std::vector<float> shared_gate_up;  // [2*intermediate, hidden_size]
    std::vector<float> shared_down;     // [hidden_size, intermediate]
    std::vector<float> router_weight;   // [num_experts, hidden_size]
    struct ExpertW {
        std::vector<float> gate_up;  // [2*intermediate, hidden_size]
        std::vector<float> down;     // [hidden_size, intermediate]
    };
    std::vector<ExpertW> experts;
    uint32_t num_experts = 0;
};

// src/hunyuan_model.h:118-125 / src/rms_norm.cpp:39-91
void swiglu_ffn_f32(const float* x, const float* gate_up_weight, const float* down_weight, float* out, uint32_t n,
                    uint32_t hidden_size, uint32_t intermediate_size);
// src/hunyuan_model.h:147-156 / src/attention.cpp:191-313
void moe_forward_cpu(const float* hidden_states, const MoEWeights& w, uint32_t n_tokens, const HunyuanConfig& cfg,
                     float* output, float* debug_router_logits = nullptr, float* debug_router_weights = nullptr,
                     int32_t* debug_router_indices = nullptr);
// src/rms_norm.cpp:9-33
void rms_norm_f32(const float* x, const float* weight, float* out, uint32_t n_tokens, uint32_t hidden_size, float eps);
