// ref_shim.cpp -- C entry points over the reference's own hunyuan_moe_full.cpp.
//
// TEST INFRASTRUCTURE ONLY: linked with the unmodified reference source file
// (src/hunyuan_moe_full.cpp, compiled from where it lies) into oracle/_ref/libhy_ref.so
// so the tests can check the oracle's restatement against the real thing.
//
// hunyuan_moe_full.cpp calls swiglu_ffn_f32 (src/rms_norm.cpp) only for the shared
// expert.  rms_norm.cpp includes ggml.h, which the reference tree does not ship, so it
// is not built: the symbol stays unresolved (lazy binding) and ref_moe_forward_full
// always passes a null shared expert, the path on which it is never called.
#include "hunyuan_moe_full.h"
#include "hy_oracle.h"

#include <algorithm>
#include <cstring>
#include <vector>

static MoERoutingConfig to_cfg(const hyo_routing_cfg* c) {
    MoERoutingConfig r;
    r.num_experts = c->num_experts;
    r.moe_topk = c->moe_topk;
    r.group_limited_greedy = c->group_limited_greedy != 0;
    r.n_group = c->n_group;
    r.topk_group = c->topk_group;
    r.drop_tokens = c->drop_tokens != 0;
    r.random_routing_dropped_token = c->random_routing_dropped_token != 0;
    r.capacity_factor = c->capacity_factor;
    r.min_capacity = c->min_capacity;
    r.norm_topk_prob = c->norm_topk_prob != 0;
    r.routed_scaling_factor = c->routed_scaling_factor;
    r.compute_aux_loss = c->compute_aux_loss != 0;
    return r;
}

extern "C" {

void ref_softmax_f32(float* x, uint32_t n) { softmax_f32(x, n); }

void ref_topk_f32(const float* x, uint32_t n, uint32_t k, float* v, int32_t* i) {
    topk_f32(x, n, k, v, i);
}

void ref_topkgating_easy(const float* logits, uint32_t T, uint32_t E, uint32_t K, float* w,
                         int32_t* idx) {
    topkgating_easy(logits, T, E, K, w, idx);
}

// Upper bound on the capacity topkgating_full can choose, so its [T,E,C] writes fit.
uint32_t ref_capacity_bound(uint32_t T, const hyo_routing_cfg* c) {
    uint32_t K = c->moe_topk, E = c->num_experts;
    uint32_t a = std::max(T, c->min_capacity);
    a = std::max(a, K);
    a = std::max(a, (uint32_t)(c->capacity_factor * K * T / E));
    return a;
}

// Outputs are written with the capacity the reference picks (*capacity); the caller
// sizes mask/cw for ref_capacity_bound().
void ref_topkgating_full(const float* logits, uint32_t T, const hyo_routing_cfg* c, uint8_t* mask,
                         float* cw, int32_t* counts, float* probs, uint32_t* capacity,
                         float* aux, float* rate) {
    MoERoutingConfig cfg = to_cfg(c);
    MoEGateOutput g;
    uint32_t cap = ref_capacity_bound(T, c);
    g.alloc(T, cfg.num_experts, cfg.moe_topk, cap, true);
    topkgating_full(logits, T, cfg, g);
    const size_t n = (size_t)T * cfg.num_experts * g.expert_capacity;
    for (size_t i = 0; i < n; i++) mask[i] = g.dispatch_mask[i] ? 1 : 0;
    memcpy(cw, g.combine_weights, n * sizeof(float));
    memcpy(counts, g.exp_counts, cfg.num_experts * sizeof(int32_t));
    memcpy(probs, g.router_probs, (size_t)T * cfg.num_experts * sizeof(float));
    *capacity = g.expert_capacity;
    *aux = g.aux_loss;
    *rate = g.exp_capacity_rate;
}

void ref_einsum_dispatch(const float* x, uint32_t T, uint32_t H, const uint8_t* mask, uint32_t E,
                         uint32_t C, float* out) {
    const size_t n = (size_t)T * E * C;
    bool* bm = new bool[n];
    for (size_t i = 0; i < n; i++) bm[i] = mask[i] != 0;
    einsum_dispatch(x, T, H, bm, E, C, out);
    delete[] bm;
}

void ref_einsum_combine(const float* cw, const float* eo, uint32_t T, uint32_t H, uint32_t E,
                        uint32_t C, float* out) {
    einsum_combine(cw, eo, T, H, E, C, out);
}

// moe_forward_full without a shared expert.  Without token dropping, min_capacity is
// raised to T so the caller-side capacity (K*T/E+1, min min_capacity) and the gating's
// own capacity (max count, min min_capacity) coincide and the reference's buffers are
// consistent; with dropping both sides use the same capacity rule and it is kept.
void ref_moe_forward_full_noshared(const float* x, uint32_t T, uint32_t H, const float* wr,
                                   const float* gu, const float* dn, uint32_t E, uint32_t I,
                                   const hyo_routing_cfg* c, float* out) {
    MoERoutingConfig cfg = to_cfg(c);
    cfg.num_experts = E;
    if (!cfg.drop_tokens && cfg.min_capacity < T) cfg.min_capacity = T;
    moe_forward_full(x, T, H, wr, nullptr, nullptr, gu, dn, E, I, cfg, out);
}

}  // extern "C"
