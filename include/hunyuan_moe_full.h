// hunyuan_moe_full.h -- the reference's MoE-block C++ API, served by the MI355X library.
//
// Same names, types and argument meaning as the reference's src/hunyuan_moe_full.h
// (MoERoutingConfig, MoEGateOutput, topkgating_full/_easy, einsum_dispatch/_combine,
// moe_forward_full, softmax_f32, topk_f32).  The MoE part of src/hunyuan_model.h
// (HunyuanConfig, MoEWeights, swiglu_ffn_f32, moe_forward_cpu, rms_norm_f32) is in
// hunyuan_model_moe.h, so a code base that keeps its own hunyuan_model.h can use this
// header alongside it.  Inputs and outputs are host arrays as in the reference; every
// call runs on the GPU through the C ABI of hy_moe.h (upload, HIP kernels, download)
// and blocks until done.
//
// Differences from the reference, all deliberate:
//  * errors throw hy::Error (std::runtime_error) instead of undefined behaviour, and
//    no output is written on error;
//  * expert selection compares logits (softmax is monotone), so experts whose
//    probabilities round to the same float but whose logits differ are ordered by
//    logit rather than by index (with group-limited greedy the selection compares the
//    masked probabilities, as the reference does);
//  * token dropping over more than 16384 tokens in one moe_forward_full call throws
//    hy::Error (the capacity slots span the whole batch, which the GPU context holds
//    up to 16384 tokens at a time);
//  * MoEGateOutput cannot be copied (the reference's implicit copy double-frees).
// Beyond the reference: quantized-weight (GGUF Q8_0 / Q4_0) overloads and
// hy::MoeStack, a resident multi-layer context.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "hy_moe.h"

// src/hunyuan_moe_full.h:25-47
struct MoERoutingConfig {
    uint32_t num_experts = 64;
    uint32_t moe_topk = 8;
    bool group_limited_greedy = false;
    uint32_t n_group = 0;
    uint32_t topk_group = 0;
    bool drop_tokens = false;
    bool random_routing_dropped_token = false;
    float capacity_factor = 1.0f;
    uint32_t min_capacity = 8;
    bool norm_topk_prob = true;
    float routed_scaling_factor = 1.0f;
    bool compute_aux_loss = false;
};

// src/hunyuan_moe_full.h:49-70
struct MoEGateOutput {
    float* combine_weights = nullptr;  // [tokens, experts, capacity]
    bool* dispatch_mask = nullptr;     // [tokens, experts, capacity]
    int32_t* exp_counts = nullptr;     // [num_experts]
    float aux_loss = 0.0f;
    float exp_capacity_rate = 0.0f;
    uint32_t expert_capacity = 0;
    float* topk_weights = nullptr;     // [tokens, topk]
    int32_t* topk_indices = nullptr;   // [tokens, topk]
    float* router_probs = nullptr;     // [tokens, experts]
    uint32_t n_tokens = 0;
    bool use_dispatch_mask = false;

    MoEGateOutput() = default;
    MoEGateOutput(const MoEGateOutput&) = delete;
    MoEGateOutput& operator=(const MoEGateOutput&) = delete;
    ~MoEGateOutput();
    void alloc(uint32_t tokens, uint32_t experts, uint32_t topk, uint32_t capacity, bool dispatch);
};

void topkgating_full(const float* logits, uint32_t n_tokens, const MoERoutingConfig& cfg, MoEGateOutput& out);
void topkgating_easy(const float* logits, uint32_t n_tokens, uint32_t num_experts, uint32_t topk,
                     float* topk_weights, int32_t* topk_indices);
void einsum_dispatch(const float* input, uint32_t n_tokens, uint32_t hidden_size, const bool* dispatch_mask,
                     uint32_t num_experts, uint32_t expert_capacity, float* dispatched_input);
void einsum_combine(const float* combine_weights, const float* expert_output, uint32_t n_tokens,
                    uint32_t hidden_size, uint32_t num_experts, uint32_t expert_capacity, float* combined_output);
void moe_forward_full(const float* hidden_states, uint32_t n_tokens, uint32_t hidden_size,
                      const float* router_weight, const float* shared_gate_up, const float* shared_down,
                      const float* expert_gate_up_stacked, const float* expert_down_stacked, uint32_t num_experts,
                      uint32_t intermediate_size, const MoERoutingConfig& routing_cfg, float* output);
void softmax_f32(float* x, uint32_t n);
void topk_f32(const float* x, uint32_t n, uint32_t k, float* topk_vals, int32_t* topk_idx);

// Quantized-weight overload: weights in ggml layout (ne0 = in-features) of type
// ggml_type HY_TYPE_Q8_0 / HY_TYPE_Q4_0 / HY_TYPE_F32, experts stacked.
void moe_forward_full(const float* hidden_states, uint32_t n_tokens, uint32_t hidden_size,
                      const float* router_weight, const void* shared_gate_up, const void* shared_down,
                      const void* expert_gate_up_stacked, const void* expert_down_stacked, int ggml_type,
                      uint32_t num_experts, uint32_t intermediate_size, const MoERoutingConfig& routing_cfg,
                      float* output);

namespace hy {

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

// Resident multi-layer MoE context (RAII over hy_moe_ctx): upload each layer once,
// then forward device buffers many times.
class MoeStack {
public:
    explicit MoeStack(const hy_moe_config& cfg);
    ~MoeStack();
    MoeStack(const MoeStack&) = delete;
    MoeStack& operator=(const MoeStack&) = delete;
    void upload_layer(uint32_t layer, const float* router, const void* shared_gu, const void* shared_dn,
                      const void* gu, const void* dn);
    void forward(uint32_t layer, const float* x_dev, uint32_t T, float* out_dev, void* stream = nullptr);
    void stack_forward(uint32_t first, uint32_t n, const float* x_dev, uint32_t T, float eps, float* out_dev,
                       void* stream = nullptr);
    hy_moe_ctx* handle() { return ctx_; }

private:
    hy_moe_ctx* ctx_ = nullptr;
};

}  // namespace hy
