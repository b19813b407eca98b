// hunyuan_model_attn.cpp -- the reference's attention / decoder-layer / backbone C++
// API (include/hunyuan_model_attn.h) on top of the C ABI.  Host arrays in and out;
// the work runs on the GPU.
#include "../../include/hunyuan_model_attn.h"

#include <algorithm>
#include <cstring>

#include "../../include/hunyuan_moe_full.h"

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

hy_attn_config attn_config(const HunyuanConfig& cfg, uint32_t T) {
    hy_attn_config c{};
    c.hidden = cfg.hidden_size;
    c.n_heads = cfg.num_attention_heads;
    c.n_kv_heads = cfg.num_key_value_heads;
    c.head_dim = cfg.attention_head_dim;
    c.num_layers = 1;
    c.max_tokens = std::max<uint32_t>(T, 1);
    c.max_cache = 0;
    c.rms_norm_eps = cfg.rms_norm_eps;
    c.rope_theta = cfg.rope_theta;
    c.device = 0;
    return c;
}

// RAII attention context
class AttnCtx {
public:
    explicit AttnCtx(const hy_attn_config& c) { check(hy_attn_create(&c, &h_)); }
    ~AttnCtx() { hy_attn_destroy(h_); }
    AttnCtx(const AttnCtx&) = delete;
    AttnCtx& operator=(const AttnCtx&) = delete;
    hy_attn_ctx* get() const { return h_; }

private:
    hy_attn_ctx* h_ = nullptr;
};

void require_sizes(const AttentionWeights& w, const HunyuanConfig& cfg) {
    const size_t H = cfg.hidden_size, hd = cfg.attention_head_dim;
    const size_t nq = (size_t)cfg.num_attention_heads * hd, nk = (size_t)cfg.num_key_value_heads * hd;
    if (w.qkv_weight.size() != (nq + 2 * nk) * H || w.o_weight.size() != H * nq || w.q_norm_weight.size() != hd ||
        w.k_norm_weight.size() != hd)
        throw hy::Error(HY_ERR_INVALID, "AttentionWeights sizes do not match the config");
}

// stacked MoE weights of a MoEWeights in the C ABI's upload layout
struct StackedMoe {
    std::vector<float> gu, dn;
};
StackedMoe stack_experts(const MoEWeights& w, const HunyuanConfig& cfg) {
    const size_t H = cfg.hidden_size, I = cfg.moe_intermediate_size, E = w.num_experts;
    if (w.experts.size() < E) throw hy::Error(HY_ERR_INVALID, "MoEWeights has fewer experts than num_experts");
    StackedMoe s;
    s.gu.resize(E * 2 * I * H);
    s.dn.resize(E * H * I);
    for (size_t e = 0; e < E; e++) {
        std::memcpy(s.gu.data() + e * 2 * I * H, w.experts[e].gate_up.data(), 2 * I * H * 4);
        std::memcpy(s.dn.data() + e * H * I, w.experts[e].down.data(), H * I * 4);
    }
    return s;
}

}  // namespace

void rope_f32(float* q, float* k, uint32_t seq, uint32_t nh, uint32_t nkv, uint32_t hd, float theta,
              const int* positions) {
    if (seq == 0) return;
    Dev qd((size_t)seq * nh * hd * 4), kd((size_t)seq * nkv * hd * 4), pd((size_t)seq * 4);
    qd.up(q, (size_t)seq * nh * hd * 4);
    kd.up(k, (size_t)seq * nkv * hd * 4);
    if (positions) pd.up(positions, (size_t)seq * 4);
    const int32_t* p = positions ? pd.as<int32_t>() : nullptr;
    check(hy_rope_f32(qd.as<float>(), seq, nh, hd, theta, p, nullptr));
    check(hy_rope_f32(kd.as<float>(), seq, nkv, hd, theta, p, nullptr));
    qd.down(q, (size_t)seq * nh * hd * 4);
    kd.down(k, (size_t)seq * nkv * hd * 4);
}

void apply_rope_2d_f32(float* q, float* k, const float* cos, const float* sin, uint32_t T, uint32_t nh, uint32_t nkv,
                       uint32_t hd) {
    if (T == 0) return;
    Dev qd((size_t)T * nh * hd * 4), kd((size_t)T * nkv * hd * 4), cd((size_t)T * hd * 4), sd((size_t)T * hd * 4);
    qd.up(q, (size_t)T * nh * hd * 4);
    kd.up(k, (size_t)T * nkv * hd * 4);
    cd.up(cos, (size_t)T * hd * 4);
    sd.up(sin, (size_t)T * hd * 4);
    check(hy_rope_2d_f32(qd.as<float>(), T, nh, hd, cd.as<float>(), sd.as<float>(), nullptr));
    check(hy_rope_2d_f32(kd.as<float>(), T, nkv, hd, cd.as<float>(), sd.as<float>(), nullptr));
    qd.down(q, (size_t)T * nh * hd * 4);
    kd.down(k, (size_t)T * nkv * hd * 4);
}

void build_2d_rope(uint32_t seq, uint32_t n_elem, uint32_t text_len, uint32_t img_h, uint32_t img_w, float base,
                   float* cos_out, float* sin_out) {
    if (seq == 0) return;
    Dev cd((size_t)seq * n_elem * 4), sd((size_t)seq * n_elem * 4);
    check(hy_build_2d_rope(seq, n_elem, text_len, img_h, img_w, base, cd.as<float>(), sd.as<float>(), nullptr));
    cd.down(cos_out, (size_t)seq * n_elem * 4);
    sd.down(sin_out, (size_t)seq * n_elem * 4);
}

void attention_forward_cpu(const float* x, const AttentionWeights& w, uint32_t T, const HunyuanConfig& cfg,
                           const int* positions, float* out, float* dq, float* dk, float* dv) {
    if (T == 0) return;
    require_sizes(w, cfg);
    const size_t H = cfg.hidden_size, hd = cfg.attention_head_dim;
    const size_t nq = (size_t)cfg.num_attention_heads * hd, nk = (size_t)cfg.num_key_value_heads * hd;
    AttnCtx a(attn_config(cfg, T));
    check(hy_attn_upload(a.get(), 0, w.qkv_weight.data(), w.o_weight.data(), w.q_norm_weight.data(),
                         w.k_norm_weight.data()));
    Dev xd(T * H * 4), od(T * H * 4), pd((size_t)T * 4), qd(dq ? T * nq * 4 : 4), kd(dk ? T * nk * 4 : 4),
        vd(dv ? T * nk * 4 : 4);
    xd.up(x, T * H * 4);
    if (positions) pd.up(positions, (size_t)T * 4);
    check(hy_attn_forward(a.get(), 0, xd.as<float>(), T, positions ? pd.as<int32_t>() : nullptr, od.as<float>(),
                          dq ? qd.as<float>() : nullptr, dk ? kd.as<float>() : nullptr, dv ? vd.as<float>() : nullptr,
                          nullptr));
    od.down(out, T * H * 4);
    if (dq) qd.down(dq, T * nq * 4);
    if (dk) kd.down(dk, T * nk * 4);
    if (dv) vd.down(dv, T * nk * 4);
}

void decoder_layer_forward_cpu(const float* x, const DecoderLayerWeights& w, uint32_t T, const HunyuanConfig& cfg,
                               const int* positions, float* out) {
    if (T == 0) return;
    require_sizes(w.attn, cfg);
    const uint32_t H = cfg.hidden_size, I = cfg.moe_intermediate_size, E = w.moe.num_experts, K = cfg.moe_topk;
    if (w.input_ln_weight.size() != H || w.post_attn_ln_weight.size() != H)
        throw hy::Error(HY_ERR_INVALID, "layer norm weights must have hidden_size entries");
    AttnCtx a(attn_config(cfg, T));
    check(hy_attn_upload(a.get(), 0, w.attn.qkv_weight.data(), w.attn.o_weight.data(), w.attn.q_norm_weight.data(),
                         w.attn.k_norm_weight.data()));
    check(hy_attn_set_input_norm(a.get(), 0, w.input_ln_weight.data()));
    hy_moe_config mc{};
    mc.hidden = H;
    mc.intermediate = I;
    mc.num_experts = E;
    mc.topk = K;
    mc.num_layers = 1;
    mc.max_tokens = T;
    mc.wtype = HY_TYPE_F32;
    mc.has_shared = cfg.num_shared_expert > 0 ? 1 : 0;
    mc.norm_topk_prob = 1;
    mc.routed_scaling_factor = 1.0f;
    hy::MoeStack m(mc);
    const StackedMoe st = stack_experts(w.moe, cfg);
    m.upload_layer(0, w.moe.router_weight.data(), mc.has_shared ? w.moe.shared_gate_up.data() : nullptr,
                   mc.has_shared ? w.moe.shared_down.data() : nullptr, st.gu.data(), st.dn.data());
    check(hy_moe_set_ffn_norm(m.handle(), 0, w.post_attn_ln_weight.data()));
    Dev xd((size_t)T * H * 4), od((size_t)T * H * 4), pd((size_t)T * 4);
    xd.up(x, (size_t)T * H * 4);
    if (positions) pd.up(positions, (size_t)T * 4);
    check(hy_decoder_layer_forward(a.get(), 0, m.handle(), 0, xd.as<float>(), T,
                                   positions ? pd.as<int32_t>() : nullptr, od.as<float>(), nullptr, nullptr));
    od.down(out, (size_t)T * H * 4);
}

void embedding_lookup_f32(const int* ids, const float* table, float* out, uint32_t T, uint32_t H) {
    if (T == 0) return;
    // the reference's signature carries no vocabulary size: upload rows 0..max id
    int32_t hi = 0;
    for (uint32_t t = 0; t < T; t++) {
        if (ids[t] < 0) throw hy::Error(HY_ERR_INVALID, "negative token id");
        hi = std::max<int32_t>(hi, ids[t]);
    }
    const size_t rows = (size_t)hi + 1;
    Dev idd((size_t)T * 4), tb(rows * H * 4), od((size_t)T * H * 4);
    idd.up(ids, (size_t)T * 4);
    tb.up(table, rows * H * 4);
    check(hy_embedding_lookup_f32(idd.as<int32_t>(), tb.as<float>(), T, H, (uint32_t)rows, od.as<float>(), nullptr));
    od.down(out, (size_t)T * H * 4);
}

void lm_head_f32(const float* h, const float* w, float* logits, uint32_t T, uint32_t H, uint32_t V) {
    if (T == 0 || V == 0) return;
    Dev hd((size_t)T * H * 4), wd((size_t)V * H * 4), ld((size_t)T * V * 4);
    hd.up(h, (size_t)T * H * 4);
    wd.up(w, (size_t)V * H * 4);
    check(hy_lm_head_f32(hd.as<float>(), wd.as<float>(), nullptr, T, H, V, ld.as<float>(), nullptr));
    ld.down(logits, (size_t)T * V * 4);
}

// ------------------------------------------------------------------ hy::Backbone
namespace hy {

Backbone::Backbone(const hy_model_config& cfg) { check(hy_model_create(&cfg, &ctx_)); }
Backbone::~Backbone() { hy_model_destroy(ctx_); }

void Backbone::upload_globals(const float* embedding, const float* final_norm, const float* lm_head) {
    check(hy_model_upload_globals(ctx_, embedding, final_norm, lm_head));
}

void Backbone::upload_layer(uint32_t layer, const DecoderLayerWeights& w, const HunyuanConfig& cfg) {
    require_sizes(w.attn, cfg);
    check(hy_attn_upload(attn(), layer, w.attn.qkv_weight.data(), w.attn.o_weight.data(), w.attn.q_norm_weight.data(),
                         w.attn.k_norm_weight.data()));
    check(hy_attn_set_input_norm(attn(), layer, w.input_ln_weight.empty() ? nullptr : w.input_ln_weight.data()));
    const StackedMoe st = stack_experts(w.moe, cfg);
    const bool shared = !w.moe.shared_gate_up.empty() && !w.moe.shared_down.empty();
    check(hy_moe_upload_layer(moe(), layer, w.moe.router_weight.data(), shared ? w.moe.shared_gate_up.data() : nullptr,
                              shared ? w.moe.shared_down.data() : nullptr, st.gu.data(), st.dn.data()));
    check(hy_moe_set_ffn_norm(moe(), layer, w.post_attn_ln_weight.empty() ? nullptr : w.post_attn_ln_weight.data()));
}

void Backbone::forward(const int32_t* ids, uint32_t T, const int32_t* positions, float* logits, void* stream) {
    check(hy_model_forward(ctx_, ids, T, positions, logits, stream));
}

}  // namespace hy
