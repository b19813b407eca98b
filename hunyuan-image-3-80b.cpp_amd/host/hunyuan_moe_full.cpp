// hunyuan_moe_full.cpp -- the reference's MoE-block C++ API (include/hunyuan_moe_full.h)
// on top of the C ABI.  Host arrays in and out; the work runs on the GPU.
#include "../../include/hunyuan_moe_full.h"
#include "../../include/hunyuan_model_moe.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace {

void check(int rc) {
    if (rc != HY_OK) throw hy::Error(rc, hy_last_error());
}

// Device buffer owned for the duration of one call.
class Dev {
public:
    explicit Dev(size_t bytes) : n_(bytes ? bytes : 1) { check(hy_malloc(&p_, n_)); }
    ~Dev() {
        if (p_) hy_free(p_);
    }
    Dev(const Dev&) = delete;
    Dev& operator=(const Dev&) = delete;
    template <typename T>
    T* as() const {
        return static_cast<T*>(p_);
    }
    void up(const void* host, size_t bytes) { check(hy_memcpy_h2d(p_, host, bytes)); }
    void down(void* host, size_t bytes) const {
        check(hy_device_synchronize());
        check(hy_memcpy_d2h(host, p_, bytes));
    }

private:
    void* p_ = nullptr;
    size_t n_;
};

bool use_groups(const MoERoutingConfig& c) { return c.group_limited_greedy && c.n_group > 0 && c.topk_group > 0; }

// Expert capacity under token dropping (src/hunyuan_moe_full.cpp:210-214): float
// arithmetic left to right, truncated to uint32, at least K, at least min_capacity.
uint32_t drop_capacity(const MoERoutingConfig& c, uint32_t T) {
    const float v = c.capacity_factor * c.moe_topk * T / c.num_experts;
    if (!(v >= 0.0f) || !(v < 4294967040.0f))
        throw hy::Error(HY_ERR_INVALID, "capacity_factor gives no capacity in uint32 range");
    uint32_t cap = (uint32_t)v;
    if (cap < c.moe_topk) cap = c.moe_topk;
    if (cap < c.min_capacity) cap = c.min_capacity;
    return cap;
}

hy_moe_config layer_config(uint32_t H, uint32_t I, uint32_t E, uint32_t K, uint32_t T, int wtype, bool shared,
                           const MoERoutingConfig* rc) {
    hy_moe_config c{};
    c.hidden = H;
    c.intermediate = I;
    c.num_experts = E;
    c.topk = K;
    c.num_layers = 1;
    c.max_tokens = std::max<uint32_t>(1, std::min<uint32_t>(T, 16384));
    c.wtype = wtype;
    c.has_shared = shared ? 1 : 0;
    // with a MoERoutingConfig: topkgating_full's rule (renormalise only when K > 1,
    // src/hunyuan_moe_full.cpp:230); without one (moe_forward_cpu, swiglu_ffn_f32):
    // renormalise at every K as src/attention.cpp:268-275 does
    c.norm_topk_prob = rc ? (rc->norm_topk_prob ? HY_NORM_TOPK : HY_NORM_OFF) : HY_NORM_ALWAYS;
    c.routed_scaling_factor = rc ? rc->routed_scaling_factor : 1.0f;
    c.device = 0;
    if (rc) {
        // moe_forward_full routes with every option of its config; the aux loss it
        // computes is not returned (src/hunyuan_moe_full.cpp:425-434), so it is not run
        c.group_limited_greedy = rc->group_limited_greedy ? 1 : 0;
        c.n_group = rc->n_group;
        c.topk_group = rc->topk_group;
        c.drop_tokens = rc->drop_tokens ? 1 : 0;
        c.capacity_factor = rc->capacity_factor;
        c.min_capacity = rc->min_capacity;
    }
    return c;
}

// One layer forward over host arrays, in token chunks of at most max_tokens.
void run_layer(const float* x, uint32_t T, uint32_t H, const float* router, const void* sgu, const void* sdn,
               const void* gu, const void* dn, int wtype, uint32_t E, uint32_t I, uint32_t K,
               const MoERoutingConfig* rc, float* out, float* dbg_logits, float* dbg_w, int32_t* dbg_idx) {
    if (T == 0) return;
    // token dropping gives capacity slots over the whole batch: one call, no chunks
    if (rc && rc->drop_tokens && T > 16384)
        throw hy::Error(HY_ERR_UNSUPPORTED, "token dropping over more than 16384 tokens in one call");
    const bool shared = sgu && sdn;
    hy::MoeStack m(layer_config(H, I, E, K, T, wtype, shared, rc));
    m.upload_layer(0, router, sgu, sdn, gu, dn);
    const uint32_t chunk = std::min<uint32_t>(T, 16384);
    Dev xd((size_t)chunk * H * 4), od((size_t)chunk * H * 4);
    Dev lg((size_t)chunk * E * 4), wd((size_t)chunk * K * 4), id((size_t)chunk * K * 4);
    for (uint32_t t0 = 0; t0 < T; t0 += chunk) {
        const uint32_t n = std::min(chunk, T - t0);
        xd.up(x + (size_t)t0 * H, (size_t)n * H * 4);
        check(hy_moe_forward_debug(m.handle(), 0, xd.as<float>(), n, od.as<float>(), lg.as<float>(),
                                   wd.as<float>(), id.as<int32_t>(), nullptr));
        od.down(out + (size_t)t0 * H, (size_t)n * H * 4);
        if (dbg_logits) lg.down(dbg_logits + (size_t)t0 * E, (size_t)n * E * 4);
        if (dbg_w) wd.down(dbg_w + (size_t)t0 * K, (size_t)n * K * 4);
        if (dbg_idx) id.down(dbg_idx + (size_t)t0 * K, (size_t)n * K * 4);
    }
}

}  // namespace

// ------------------------------------------------------------------ MoEGateOutput
MoEGateOutput::~MoEGateOutput() {
    free(combine_weights);
    free(dispatch_mask);
    free(exp_counts);
    free(topk_weights);
    free(topk_indices);
    free(router_probs);
}

void MoEGateOutput::alloc(uint32_t tokens, uint32_t experts, uint32_t topk, uint32_t capacity, bool dispatch) {
    n_tokens = tokens;
    use_dispatch_mask = dispatch;
    if (dispatch) {
        const size_t n = (size_t)tokens * experts * capacity;
        dispatch_mask = static_cast<bool*>(calloc(n ? n : 1, sizeof(bool)));
        combine_weights = static_cast<float*>(calloc(n ? n : 1, sizeof(float)));
        exp_counts = static_cast<int32_t*>(calloc(experts, sizeof(int32_t)));
    } else {
        topk_weights = static_cast<float*>(malloc((size_t)tokens * topk * sizeof(float)));
        topk_indices = static_cast<int32_t*>(malloc((size_t)tokens * topk * sizeof(int32_t)));
    }
    router_probs = static_cast<float*>(malloc((size_t)tokens * experts * sizeof(float)));
    if ((dispatch && (!dispatch_mask || !combine_weights || !exp_counts)) ||
        (!dispatch && (!topk_weights || !topk_indices)) || !router_probs)
        throw hy::Error(HY_ERR_NOMEM, "MoEGateOutput::alloc: out of host memory");
}

// ------------------------------------------------------------------ small routing helpers
void softmax_f32(float* x, uint32_t n) {
    if (n == 0) return;
    Dev d((size_t)n * 4);
    d.up(x, (size_t)n * 4);
    check(hy_softmax_rows(d.as<float>(), 1, n, nullptr));
    d.down(x, (size_t)n * 4);
}

void topk_f32(const float* x, uint32_t n, uint32_t k, float* vals, int32_t* idx) {
    Dev d((size_t)n * 4), v((size_t)k * 4), i((size_t)k * 4);
    d.up(x, (size_t)n * 4);
    check(hy_topk_rows(d.as<float>(), 1, n, k, v.as<float>(), i.as<int32_t>(), nullptr));
    v.down(vals, (size_t)k * 4);
    i.down(idx, (size_t)k * 4);
}

void topkgating_easy(const float* logits, uint32_t T, uint32_t E, uint32_t K, float* w, int32_t* idx) {
    if (T == 0) return;
    Dev l((size_t)T * E * 4), wd((size_t)T * K * 4), id((size_t)T * K * 4);
    l.up(logits, (size_t)T * E * 4);
    check(hy_topkgating_easy(l.as<float>(), T, E, K, wd.as<float>(), id.as<int32_t>(), nullptr));
    wd.down(w, (size_t)T * K * 4);
    id.down(idx, (size_t)T * K * 4);
}

// Routing on the GPU (group-limited greedy, the aux loss and token dropping included);
// the dense [T,E,C] outputs are assembled from the expert-sorted positions (the slot c
// of a pair is its position inside its expert, in the reference's k-major priority
// order; a pair at c >= C is dropped).  The buffers of `out` are (re)allocated with the
// capacity this function picks, which keeps the strides consistent.
// random_routing_dropped_token is read by nothing in the reference and by nothing here.
void topkgating_full(const float* logits, uint32_t T, const MoERoutingConfig& cfg, MoEGateOutput& out) {
    const uint32_t E = cfg.num_experts, K = cfg.moe_topk;
    if (T == 0) return;
    const size_t pairs = (size_t)T * K;
    const bool groups = use_groups(cfg);
    Dev l((size_t)T * E * 4), p((size_t)T * E * 4), gates((size_t)T * E * 4), wd(pairs * 4), id(pairs * 4),
        cnt((size_t)E * 4), off((size_t)(E + 1) * 4), pos(pairs * 4), aux(4);
    l.up(logits, (size_t)T * E * 4);
    p.up(logits, (size_t)T * E * 4);
    check(hy_route_logits_groups(l.as<float>(), T, E, K, cfg.norm_topk_prob ? HY_NORM_TOPK : HY_NORM_OFF,
                                 cfg.routed_scaling_factor, groups ? cfg.n_group : 0, groups ? cfg.topk_group : 0,
                                 wd.as<float>(), id.as<int32_t>(), gates.as<float>(), nullptr));
    check(hy_dispatch_pairs(id.as<int32_t>(), wd.as<float>(), T, K, E, cnt.as<int32_t>(), off.as<int32_t>(),
                            pos.as<int32_t>(), nullptr));
    // the reference keeps router_probs from before the group mask (:124-125)
    check(hy_softmax_rows(p.as<float>(), T, E, nullptr));
    float aux_loss = 0.0f;
    if (cfg.compute_aux_loss) {
        check(hy_aux_loss(gates.as<float>(), cnt.as<int32_t>(), T, E, aux.as<float>(), nullptr));
        aux.down(&aux_loss, 4);
    }
    std::vector<float> w(pairs), probs((size_t)T * E);
    std::vector<int32_t> idx(pairs), counts(E), offs(E + 1), ps(pairs);
    wd.down(w.data(), pairs * 4);
    id.down(idx.data(), pairs * 4);
    cnt.down(counts.data(), (size_t)E * 4);
    off.down(offs.data(), (size_t)(E + 1) * 4);
    pos.down(ps.data(), pairs * 4);
    p.down(probs.data(), (size_t)T * E * 4);

    uint32_t C = 0;
    if (cfg.drop_tokens) {
        C = drop_capacity(cfg, T);
    } else {
        for (uint32_t e = 0; e < E; e++) C = std::max(C, (uint32_t)counts[e]);
        C = std::max(C, cfg.min_capacity);
    }
    free(out.combine_weights);
    free(out.dispatch_mask);
    free(out.exp_counts);
    free(out.router_probs);
    out.combine_weights = nullptr;
    out.dispatch_mask = nullptr;
    out.exp_counts = nullptr;
    out.router_probs = nullptr;
    out.alloc(T, E, K, C, true);
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t k = 0; k < K; k++) {
            const size_t pr = (size_t)t * K + k;
            const int e = idx[pr];
            const uint32_t c = (uint32_t)(ps[pr] - offs[e]);
            if (c >= C) continue;  // no capacity slot left: dropped (:296-304)
            out.dispatch_mask[((size_t)t * E + e) * C + c] = true;
            out.combine_weights[((size_t)t * E + e) * C + c] = w[pr];
        }
    memcpy(out.exp_counts, counts.data(), (size_t)E * 4);
    memcpy(out.router_probs, probs.data(), (size_t)T * E * 4);
    out.expert_capacity = C;
    out.aux_loss = aux_loss;
    float placed = 0;
    for (size_t i = 0; i < (size_t)T * E * C; i++)
        if (out.dispatch_mask[i]) placed += 1;
    out.exp_capacity_rate = placed / (float)(T * K);
}

void einsum_dispatch(const float* input, uint32_t T, uint32_t H, const bool* mask, uint32_t E, uint32_t C,
                     float* outp) {
    const size_t nm = (size_t)T * E * C;
    std::vector<uint8_t> m(nm);
    for (size_t i = 0; i < nm; i++) m[i] = mask[i] ? 1 : 0;
    Dev x((size_t)T * H * 4), md(nm), o((size_t)E * C * H * 4);
    x.up(input, (size_t)T * H * 4);
    md.up(m.data(), nm);
    check(hy_einsum_dispatch(x.as<float>(), T, H, md.as<uint8_t>(), E, C, o.as<float>(), nullptr));
    o.down(outp, (size_t)E * C * H * 4);
}

void einsum_combine(const float* cw, const float* eo, uint32_t T, uint32_t H, uint32_t E, uint32_t C, float* outp) {
    Dev w((size_t)T * E * C * 4), y((size_t)E * C * H * 4), o((size_t)T * H * 4);
    w.up(cw, (size_t)T * E * C * 4);
    y.up(eo, (size_t)E * C * H * 4);
    check(hy_einsum_combine(w.as<float>(), y.as<float>(), T, H, E, C, o.as<float>(), nullptr));
    o.down(outp, (size_t)T * H * 4);
}

// ------------------------------------------------------------------ layer forwards
void moe_forward_full(const float* x, uint32_t T, uint32_t H, const float* router, const float* sgu, const float* sdn,
                      const float* gu, const float* dn, uint32_t E, uint32_t I, const MoERoutingConfig& rc,
                      float* out) {
    moe_forward_full(x, T, H, router, sgu, sdn, gu, dn, HY_TYPE_F32, E, I, rc, out);
}

void moe_forward_full(const float* x, uint32_t T, uint32_t H, const float* router, const void* sgu, const void* sdn,
                      const void* gu, const void* dn, int wtype, uint32_t E, uint32_t I, const MoERoutingConfig& rc,
                      float* out) {
    run_layer(x, T, H, router, sgu, sdn, gu, dn, wtype, E, I, rc.moe_topk, &rc, out, nullptr, nullptr, nullptr);
}

void swiglu_ffn_f32(const float* x, const float* gu, const float* dn, float* out, uint32_t n, uint32_t H, uint32_t I) {
    // one routed expert with weight exactly 1: softmax of a single logit is 1 and the
    // combine adds 1 * y to zero
    std::vector<float> router(H, 0.0f);
    run_layer(x, n, H, router.data(), nullptr, nullptr, gu, dn, HY_TYPE_F32, 1, I, 1, nullptr, out, nullptr, nullptr,
              nullptr);
}

void moe_forward_cpu(const float* x, const MoEWeights& w, uint32_t T, const HunyuanConfig& cfg, float* out,
                     float* dbg_logits, float* dbg_w, int32_t* dbg_idx) {
    const uint32_t H = cfg.hidden_size, I = cfg.moe_intermediate_size, E = w.num_experts, K = cfg.moe_topk;
    if (w.experts.size() < E) throw hy::Error(HY_ERR_INVALID, "MoEWeights has fewer experts than num_experts");
    // stacked [E*2I, H] / [E*H, I] (the StackedExpertWeights layout, src/hunyuan_extended.cpp:8-26)
    std::vector<float> gu((size_t)E * 2 * I * H), dn((size_t)E * H * I);
    for (uint32_t e = 0; e < E; e++) {
        memcpy(gu.data() + (size_t)e * 2 * I * H, w.experts[e].gate_up.data(), (size_t)2 * I * H * 4);
        memcpy(dn.data() + (size_t)e * H * I, w.experts[e].down.data(), (size_t)H * I * 4);
    }
    std::vector<float> logits(dbg_logits ? (size_t)T * E : 0);
    run_layer(x, T, H, w.router_weight.data(), w.shared_gate_up.data(), w.shared_down.data(), gu.data(), dn.data(),
              HY_TYPE_F32, E, I, K, nullptr, out, dbg_logits ? logits.data() : nullptr, dbg_w, dbg_idx);
    if (dbg_logits) {
        // the reference copies its router buffer after the in-place softmax
        // (src/attention.cpp:278): probabilities
        Dev p((size_t)T * E * 4);
        p.up(logits.data(), (size_t)T * E * 4);
        check(hy_softmax_rows(p.as<float>(), T, E, nullptr));
        p.down(dbg_logits, (size_t)T * E * 4);
    }
}

void rms_norm_f32(const float* x, const float* weight, float* out, uint32_t T, uint32_t H, float eps) {
    Dev xd((size_t)T * H * 4), wd((size_t)H * 4), od((size_t)T * H * 4);
    xd.up(x, (size_t)T * H * 4);
    wd.up(weight, (size_t)H * 4);
    check(hy_rms_norm_w(xd.as<float>(), wd.as<float>(), T, H, eps, od.as<float>(), nullptr));
    od.down(out, (size_t)T * H * 4);
}

// ------------------------------------------------------------------ hy::MoeStack
namespace hy {

MoeStack::MoeStack(const hy_moe_config& cfg) { check(hy_moe_create(&cfg, &ctx_)); }
MoeStack::~MoeStack() {
    if (ctx_) hy_moe_destroy(ctx_);
}
void MoeStack::upload_layer(uint32_t layer, const float* router, const void* sgu, const void* sdn, const void* gu,
                            const void* dn) {
    check(hy_moe_upload_layer(ctx_, layer, router, sgu, sdn, gu, dn));
}
void MoeStack::forward(uint32_t layer, const float* x, uint32_t T, float* out, void* stream) {
    check(hy_moe_forward(ctx_, layer, x, T, out, stream));
}
void MoeStack::stack_forward(uint32_t first, uint32_t n, const float* x, uint32_t T, float eps, float* out,
                             void* stream) {
    check(hy_moe_stack_forward(ctx_, first, n, x, T, eps, out, stream));
}

}  // namespace hy
