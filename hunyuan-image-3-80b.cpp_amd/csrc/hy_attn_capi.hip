// hy_attn_capi.hip -- the C ABI of the attention half (include/hy_attn.h): context,
// resident weights and key / value cache, forward orchestration, timing.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/hy_attn.h"
#include "hy_launch.hpp"

namespace hy {
int set_last_error(int code, const std::string& msg);  // hy_capi.hip
int moe_hidden(const hy_moe_ctx* c);                   // hy_capi.hip
int moe_device(const hy_moe_ctx* c);
}

namespace {

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return hy::set_last_error(code, buf);
}

#define HIP_TRY(expr)                                                                                    \
    do {                                                                                                 \
        hipError_t e_ = (expr);                                                                          \
        if (e_ != hipSuccess) return fail(HY_ERR_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_),   \
                                          __FILE__, __LINE__);                                           \
    } while (0)

#define HY_TRY(expr)                \
    do {                            \
        int r_ = (expr);            \
        if (r_ != HY_OK) return r_; \
    } while (0)

enum { AK_QKV = 0, AK_ROPE = 1, AK_ATTN = 2, AK_OPROJ = 3, AK_COUNT = 4 };

struct ProfRec {
    int kid;
    hipEvent_t a, b;
};

}  // namespace

struct hy_attn_ctx {
    hy_attn_config cfg{};
    int H = 0, nh = 0, nkv = 0, hd = 0, nqkv = 0, Tm = 0, Lc = 0;
    void* arena = nullptr;
    float* qkv_w = nullptr;   // [nqkv][H]
    float* o_w = nullptr;     // [H][nh*hd]
    float* q_norm = nullptr;  // [hd]
    float* k_norm = nullptr;
    float* qkv = nullptr;     // [Tm][nqkv]
    float* q = nullptr;       // [Tm][nh][hd]
    float* kf = nullptr;      // [nkv][Tm][hd] (forward without cache)
    float* vf = nullptr;
    float* kc = nullptr;      // [nkv][Lc][hd] cache
    float* vc = nullptr;
    float* merged = nullptr;  // [Tm][nh*hd]
    float* in_norm = nullptr; // input_layernorm weight [H] (used when has_in_norm)
    float* xn = nullptr;      // decoder layer: normed input [Tm][H]
    float* hres = nullptr;    // decoder layer: x + attention [Tm][H]
    uint32_t cache_len = 0;
    bool loaded = false;
    bool has_in_norm = false;
    bool prof = false;
    std::vector<ProfRec> pending;
    std::vector<hipEvent_t> free_events;
    uint64_t prof_n[AK_COUNT] = {};
    double prof_ms[AK_COUNT] = {};
};

namespace {

size_t al256(size_t b) { return (b + 255) / 256 * 256; }

int get_event(hy_attn_ctx* c, hipEvent_t* ev) {
    if (!c->free_events.empty()) {
        *ev = c->free_events.back();
        c->free_events.pop_back();
        return HY_OK;
    }
    HIP_TRY(hipEventCreate(ev));
    return HY_OK;
}

int drain_prof(hy_attn_ctx* c) {
    for (auto& r : c->pending) {
        HIP_TRY(hipEventSynchronize(r.b));
        float ms = 0.0f;
        HIP_TRY(hipEventElapsedTime(&ms, r.a, r.b));
        c->prof_n[r.kid]++;
        c->prof_ms[r.kid] += ms;
        c->free_events.push_back(r.a);
        c->free_events.push_back(r.b);
    }
    c->pending.clear();
    return HY_OK;
}

template <class F>
int timed(hy_attn_ctx* c, int kid, hipStream_t s, F&& launch) {
    hipEvent_t a = nullptr, b = nullptr;
    if (c->prof) {
        HY_TRY(get_event(c, &a));
        HY_TRY(get_event(c, &b));
        HIP_TRY(hipEventRecord(a, s));
    }
    const hipError_t e = launch();
    if (e != hipSuccess) return fail(HY_ERR_HIP, "attention kernel %d launch failed: %s", kid, hipGetErrorString(e));
    if (c->prof) {
        HIP_TRY(hipEventRecord(b, s));
        c->pending.push_back({kid, a, b});
        if (c->pending.size() > 4096) HY_TRY(drain_prof(c));
    }
    return HY_OK;
}

// projection, rotary + norm, attention, output projection for T tokens whose keys /
// values land in k / v ([nkv][L][hd]) at row pos0 + t
int run(hy_attn_ctx* c, const float* x, int T, int mode, const int32_t* positions, const float* cos_t,
        const float* sin_t, int norm_assoc, float* k, float* v, int L, int pos0, int kv_len, int causal, float* out,
        hipStream_t s, const float* resid = nullptr) {
    HY_TRY(timed(c, AK_QKV, s,
                 [&] { return hy::launch_gemm_nt_f32(x, c->qkv_w, nullptr, c->qkv, T, c->nqkv, c->H, s); }));
    hy::RopeNormArgs r{c->qkv, T, c->nh, c->nkv, c->hd, c->nqkv, mode, positions, c->cfg.rope_theta, cos_t, sin_t,
                       c->q_norm, c->k_norm, c->cfg.rms_norm_eps, norm_assoc, c->q, k, v, L, pos0};
    HY_TRY(timed(c, AK_ROPE, s, [&] { return hy::launch_rope_qknorm(r, s); }));
    hy::FlashArgs f{c->q, k, v, c->merged, T, c->nh, c->nkv, c->hd, L, kv_len, pos0, causal,
                    1.0f / sqrtf((float)c->hd)};
    HY_TRY(timed(c, AK_ATTN, s, [&] { return hy::launch_flash_attn(f, s); }));
    HY_TRY(timed(c, AK_OPROJ, s,
                 [&] { return hy::launch_gemm_nt_f32(c->merged, c->o_w, resid, out, T, c->H, c->nh * c->hd, s); }));
    return HY_OK;
}

}  // namespace

extern "C" {

int hy_attn_create(const hy_attn_config* cfg, hy_attn_ctx** out) {
    if (!out) return fail(HY_ERR_INVALID, "null out");
    *out = nullptr;
    if (!cfg) return fail(HY_ERR_INVALID, "null config");
    if (cfg->hidden == 0 || cfg->hidden % 16)
        return fail(HY_ERR_INVALID, "hidden=%u must be a positive multiple of 16", cfg->hidden);
    if (cfg->head_dim != 64 && cfg->head_dim != 128)
        return fail(HY_ERR_UNSUPPORTED, "head_dim=%u: the kernels take 64 or 128", cfg->head_dim);
    if (cfg->n_kv_heads == 0 || cfg->n_heads != 4 * cfg->n_kv_heads)
        return fail(HY_ERR_UNSUPPORTED, "n_heads=%u n_kv_heads=%u: the kernels take 4 query heads per kv head",
                    cfg->n_heads, cfg->n_kv_heads);
    if (cfg->max_tokens == 0 || cfg->max_tokens > 16384)
        return fail(HY_ERR_INVALID, "max_tokens=%u must be in 1..16384", cfg->max_tokens);
    if (cfg->max_cache > 1u << 20) return fail(HY_ERR_INVALID, "max_cache=%u too large", cfg->max_cache);
    HIP_TRY(hipSetDevice(cfg->device));
    hy_attn_ctx* c = new hy_attn_ctx();
    c->cfg = *cfg;
    c->H = (int)cfg->hidden;
    c->nh = (int)cfg->n_heads;
    c->nkv = (int)cfg->n_kv_heads;
    c->hd = (int)cfg->head_dim;
    c->nqkv = (c->nh + 2 * c->nkv) * c->hd;
    c->Tm = (int)cfg->max_tokens;
    c->Lc = (int)cfg->max_cache;
    const size_t H = c->H, nq = (size_t)c->nh * c->hd, nk = (size_t)c->nkv * c->hd, Tm = c->Tm, Lc = c->Lc;
    struct Part {
        float** p;
        size_t n;
    } parts[] = {{&c->qkv_w, (size_t)c->nqkv * H}, {&c->o_w, H * nq},        {&c->q_norm, (size_t)c->hd},
                 {&c->k_norm, (size_t)c->hd},      {&c->qkv, Tm * c->nqkv},  {&c->q, Tm * nq},
                 {&c->kf, Tm * nk},                {&c->vf, Tm * nk},        {&c->kc, Lc * nk},
                 {&c->vc, Lc * nk},                {&c->merged, Tm * nq},    {&c->in_norm, H},
                 {&c->xn, Tm * H},                 {&c->hres, Tm * H}};
    size_t total = 0;
    for (auto& p : parts) total += al256(p.n * 4);
    if (hipMalloc(&c->arena, total) != hipSuccess) {
        delete c;
        return fail(HY_ERR_NOMEM, "hipMalloc of %zu bytes for the attention context failed", total);
    }
    size_t o = 0;
    for (auto& p : parts) {
        *p.p = reinterpret_cast<float*>(static_cast<uint8_t*>(c->arena) + o);
        o += al256(p.n * 4);
    }
    if (hipMemset(c->arena, 0, total) != hipSuccess) {
        (void)hipFree(c->arena);
        delete c;
        return fail(HY_ERR_HIP, "hipMemset of the attention context failed");
    }
    *out = c;
    return HY_OK;
}

int hy_attn_destroy(hy_attn_ctx* c) {
    if (!c) return HY_OK;
    (void)hipSetDevice(c->cfg.device);
    (void)hipDeviceSynchronize();
    for (auto& r : c->pending) {
        (void)hipEventDestroy(r.a);
        (void)hipEventDestroy(r.b);
    }
    for (auto e : c->free_events) (void)hipEventDestroy(e);
    if (c->arena) (void)hipFree(c->arena);
    delete c;
    return HY_OK;
}

int hy_attn_upload(hy_attn_ctx* c, const float* qkv_w, const float* o_w, const float* qn, const float* kn) {
    if (!c || !qkv_w || !o_w || !qn || !kn) return fail(HY_ERR_INVALID, "null argument");
    HIP_TRY(hipSetDevice(c->cfg.device));
    const size_t nq = (size_t)c->nh * c->hd;
    HIP_TRY(hipMemcpy(c->qkv_w, qkv_w, (size_t)c->nqkv * c->H * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(c->o_w, o_w, (size_t)c->H * nq * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(c->q_norm, qn, (size_t)c->hd * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(c->k_norm, kn, (size_t)c->hd * 4, hipMemcpyHostToDevice));
    c->loaded = true;
    return HY_OK;
}

int hy_attn_forward(hy_attn_ctx* c, const float* x, uint32_t T, const int32_t* positions, float* out, float* dq,
                    float* dk, float* dv, void* stream) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    if (!c->loaded) return fail(HY_ERR_STATE, "attention weights not uploaded");
    if (!x || !out) return fail(HY_ERR_INVALID, "null x/out");
    if (T == 0 || T > (uint32_t)c->Tm) return fail(HY_ERR_INVALID, "T=%u must be in 1..max_tokens=%d", T, c->Tm);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int iT = (int)T;
    HY_TRY(run(c, x, iT, hy::ROPE_1D, positions, nullptr, nullptr, 0, c->kf, c->vf, c->Tm, 0, iT, 1, out, s));
    const size_t nq = (size_t)c->nh * c->hd;
    if (dq) HIP_TRY(hipMemcpyAsync(dq, c->q, (size_t)T * nq * 4, hipMemcpyDeviceToDevice, s));
    if (dk) HIP_TRY(hy::launch_gather_kv(c->kf, c->nkv, c->Tm, 0, iT, c->hd, dk, s));
    if (dv) HIP_TRY(hy::launch_gather_kv(c->vf, c->nkv, c->Tm, 0, iT, c->hd, dv, s));
    return HY_OK;
}

int hy_attn_forward_cached(hy_attn_ctx* c, const float* x, uint32_t T, const float* cos_t, const float* sin_t,
                           float* out, void* stream) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    if (!c->loaded) return fail(HY_ERR_STATE, "attention weights not uploaded");
    if (!x || !out) return fail(HY_ERR_INVALID, "null x/out");
    if (T == 0 || T > (uint32_t)c->Tm) return fail(HY_ERR_INVALID, "T=%u must be in 1..max_tokens=%d", T, c->Tm);
    if ((cos_t == nullptr) != (sin_t == nullptr)) return fail(HY_ERR_INVALID, "give both rotary tables or neither");
    if ((uint64_t)c->cache_len + T > (uint64_t)c->Lc)
        return fail(HY_ERR_INVALID, "cache overflow: %u cached + %u new > max_cache %d", c->cache_len, T, c->Lc);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int pos0 = (int)c->cache_len;
    HY_TRY(run(c, x, (int)T, cos_t ? hy::ROPE_TABLE : hy::ROPE_NONE, nullptr, cos_t, sin_t, 1, c->kc, c->vc, c->Lc,
               pos0, pos0 + (int)T, 0, out, s));
    c->cache_len += T;
    return HY_OK;
}

int hy_attn_set_input_norm(hy_attn_ctx* c, const float* w) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    if (!w) {
        c->has_in_norm = false;
        return HY_OK;
    }
    HIP_TRY(hipSetDevice(c->cfg.device));
    HIP_TRY(hipMemcpy(c->in_norm, w, (size_t)c->H * 4, hipMemcpyHostToDevice));
    c->has_in_norm = true;
    return HY_OK;
}

int hy_decoder_layer_forward(hy_attn_ctx* c, hy_moe_ctx* moe, uint32_t moe_layer, const float* x, uint32_t T,
                             const int32_t* positions, float* out, float* debug_h, void* stream) {
    if (!c || !moe) return fail(HY_ERR_INVALID, "null context");
    if (hy::moe_hidden(moe) != c->H || hy::moe_device(moe) != c->cfg.device)
        return fail(HY_ERR_INVALID, "the MoE context (hidden %d, device %d) does not match the attention context "
                    "(hidden %d, device %d)", hy::moe_hidden(moe), hy::moe_device(moe), c->H, c->cfg.device);
    if (!c->loaded) return fail(HY_ERR_STATE, "attention weights not uploaded");
    if (!x || !out) return fail(HY_ERR_INVALID, "null x/out");
    if (T == 0 || T > (uint32_t)c->Tm) return fail(HY_ERR_INVALID, "T=%u must be in 1..max_tokens=%d", T, c->Tm);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int iT = (int)T;
    const float eps = c->cfg.rms_norm_eps;
    // input_layernorm -> self-attention -> h = x + attention (in the output projection)
    HIP_TRY(c->has_in_norm ? hy::launch_rms_norm_w(x, c->in_norm, iT, c->H, eps, c->xn, s)
                           : hy::launch_rms_norm(x, iT, c->H, eps, c->xn, s));
    HY_TRY(run(c, c->xn, iT, hy::ROPE_1D, positions, nullptr, nullptr, 0, c->kf, c->vf, c->Tm, 0, iT, 1, c->hres, s,
               x));
    if (debug_h) HIP_TRY(hipMemcpyAsync(debug_h, c->hres, (size_t)T * c->H * 4, hipMemcpyDeviceToDevice, s));
    // post_attention_layernorm -> MoE -> out = h + MoE (the MoE context's layer and norm)
    return hy_moe_stack_forward(moe, moe_layer, 1, c->hres, T, eps, out, stream);
}

int hy_attn_cache_reset(hy_attn_ctx* c) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    c->cache_len = 0;
    return HY_OK;
}

int hy_attn_cache_len(const hy_attn_ctx* c, uint32_t* len) {
    if (!c || !len) return fail(HY_ERR_INVALID, "null argument");
    *len = c->cache_len;
    return HY_OK;
}

int hy_build_2d_rope(uint32_t seq, uint32_t n_elem, uint32_t text_len, uint32_t img_h, uint32_t img_w, float base,
                     float* cos_out, float* sin_out, void* stream) {
    if (!cos_out || !sin_out) return fail(HY_ERR_INVALID, "null table");
    if (seq == 0 || n_elem == 0 || n_elem % 2) return fail(HY_ERR_INVALID, "bad table shape");
    if (seq > text_len && (img_w == 0 || img_h == 0 || (uint64_t)text_len + (uint64_t)img_h * img_w < seq))
        return fail(HY_ERR_INVALID, "seq=%u exceeds text_len + img_h*img_w", seq);
    HIP_TRY(hy::launch_rope2d_table((int)seq, (int)n_elem, (int)text_len, (int)img_h, (int)img_w, base, cos_out,
                                    sin_out, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_attn_prof_enable(hy_attn_ctx* c, int32_t on) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    if (!on) HY_TRY(drain_prof(c));
    if (on) {
        for (int k = 0; k < AK_COUNT; k++) {
            c->prof_n[k] = 0;
            c->prof_ms[k] = 0.0;
        }
    }
    c->prof = on != 0;
    return HY_OK;
}

int hy_attn_prof_read(hy_attn_ctx* c, uint32_t kid, uint64_t* n, double* ms) {
    if (!c || !n || !ms || kid >= AK_COUNT) return fail(HY_ERR_INVALID, "bad argument");
    HY_TRY(drain_prof(c));
    *n = c->prof_n[kid];
    *ms = c->prof_ms[kid];
    return HY_OK;
}

}  // extern "C"
