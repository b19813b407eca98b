// hy_attn_capi.hip -- the C ABI of the attention half and of the resident backbone
// (include/hy_attn.h): per-layer attention weights and key / value caches, a work
// arena shared by the layers, forward orchestration, timing; the model context
// (embedding, decoder layers, final norm, lm_head).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/hy_attn.h"
#include "../host/hy_gguf.hpp"
#include "hy_device.hpp"
#include "hy_launch.hpp"

namespace hy {
int set_last_error(int code, const std::string& msg);  // hy_capi.hip
int moe_hidden(const hy_moe_ctx* c);                   // hy_capi.hip
int moe_device(const hy_moe_ctx* c);
const GgufFile& gguf_file(const hy_gguf* g);           // host/hy_gguf.cpp
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

// stream-K scratch of the stand-alone lm_head GEMM (one per device)
struct LmScratch {
    float* ws = nullptr;
    hipEvent_t done = nullptr;
};

struct ProfRec {
    int kid;
    hipEvent_t a, b;
};

struct AttnLayer {
    void* base = nullptr;      // one allocation: weights, norms, cache
    float* qkv_w = nullptr;    // [nqkv][H]
    float* o_w = nullptr;      // [H][nh*hd]
    float* q_norm = nullptr;   // [hd]
    float* k_norm = nullptr;
    float* in_norm = nullptr;  // input_layernorm [H] (used when has_in_norm)
    float* kc = nullptr;       // [nkv][Lc][hd]
    float* vc = nullptr;
    uint32_t cache_len = 0;
    bool loaded = false;
    bool has_in_norm = false;
};

size_t al256(size_t b) { return (b + 255) / 256 * 256; }

}  // namespace

struct hy_attn_ctx {
    hy_attn_config cfg{};
    int H = 0, nh = 0, nkv = 0, hd = 0, nqkv = 0, Tm = 0, Lc = 0;
    std::vector<AttnLayer> layers;
    void* arena = nullptr;     // work buffers shared by the layers
    float* qkv = nullptr;      // [Tm][nqkv]
    float* q = nullptr;        // [Tm][nh][hd]
    float* kf = nullptr;       // [nkv][Tm][hd] (forward without cache)
    float* vf = nullptr;
    float* merged = nullptr;   // [Tm][nh*hd]
    float* gemm_ws = nullptr;  // stream-K partial tiles of the projections' GEMM
    float* fa_ws = nullptr;    // partial tiles of the attention split over the keys
    int fa_slots = 0;
    int decode_waves = 0;      // cap on the decode attention's waves (0: resident count)
    float* xn = nullptr;       // decoder layer: normed input [Tm][H]
    float* hres = nullptr;     // decoder layer: x + attention [Tm][H]
    bool prof = false;
    std::vector<ProfRec> pending;
    std::vector<hipEvent_t> free_events;
    uint64_t prof_n[AK_COUNT] = {};
    double prof_ms[AK_COUNT] = {};
};

struct hy_model_ctx {
    hy_model_config cfg{};
    hy_attn_ctx* attn = nullptr;
    hy_moe_ctx* moe = nullptr;
    int H = 0, V = 0, Tm = 0, L = 0;
    void* arena = nullptr;
    float* embed = nullptr;    // [V][H]
    float* fnorm = nullptr;    // [H]
    float* lm_head = nullptr;  // [V][H]
    float* ha = nullptr;       // hidden ping-pong [Tm][H]
    float* hb = nullptr;
    float* normed = nullptr;   // [Tm][H]
};

namespace {

int get_event(hy_attn_ctx* c, hipEvent_t* ev) {
    if (!c->free_events.empty()) {
        *ev = c->free_events.back();
        c->free_events.pop_back();
        return HY_OK;
    }
    // timing-only events: no system-scope fence (cache writeback / invalidate) when
    // they are recorded, which would otherwise be counted in the kernel's time
    HIP_TRY(hipEventCreateWithFlags(ev, hipEventDisableSystemFence));
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

int check_layer(const hy_attn_ctx* c, uint32_t layer, bool need_loaded) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    if (layer >= c->layers.size()) return fail(HY_ERR_INVALID, "layer %u out of range", layer);
    if (need_loaded && !c->layers[layer].loaded) return fail(HY_ERR_STATE, "attention layer %u not uploaded", layer);
    return HY_OK;
}

int alloc_layer(hy_attn_ctx* c, AttnLayer& L) {
    if (L.base) return HY_OK;
    const size_t H = c->H, nq = (size_t)c->nh * c->hd, nk = (size_t)c->nkv * c->hd;
    const size_t parts[] = {(size_t)c->nqkv * H, H * nq, (size_t)c->hd, (size_t)c->hd, H, (size_t)c->Lc * nk,
                            (size_t)c->Lc * nk};
    float** ptrs[] = {&L.qkv_w, &L.o_w, &L.q_norm, &L.k_norm, &L.in_norm, &L.kc, &L.vc};
    size_t total = 0;
    for (size_t n : parts) total += al256(n * 4);
    if (hipMalloc(&L.base, total) != hipSuccess) {
        L.base = nullptr;
        return fail(HY_ERR_NOMEM, "hipMalloc of %zu bytes for an attention layer failed", total);
    }
    size_t o = 0;
    for (int i = 0; i < 7; i++) {
        *ptrs[i] = reinterpret_cast<float*>(static_cast<uint8_t*>(L.base) + o);
        o += al256(parts[i] * 4);
    }
    return HY_OK;
}

// projection, rotary + norm, attention, output projection for T tokens whose keys /
// values land in k / v ([nkv][Lrows][hd]) at row pos0 + t; resid (nullable) is added
// in the output projection
int run(hy_attn_ctx* c, const AttnLayer& W, const float* x, int T, int mode, const int32_t* positions,
        const float* cos_t, const float* sin_t, int norm_assoc, float* k, float* v, int Lrows, int pos0, int kv_len,
        int causal, float* out, hipStream_t s, const float* resid = nullptr) {
    HY_TRY(timed(c, AK_QKV, s,
                 [&] { return hy::launch_gemm_nt_f32(x, W.qkv_w, nullptr, c->qkv, T, c->nqkv, c->H, s, c->gemm_ws); }));
    hy::RopeNormArgs r{c->qkv, T, c->nh, c->nkv, c->hd, c->nqkv, mode, positions, c->cfg.rope_theta, cos_t, sin_t,
                       W.q_norm, W.k_norm, c->cfg.rms_norm_eps, norm_assoc, c->q, k, v, Lrows, pos0};
    HY_TRY(timed(c, AK_ROPE, s, [&] { return hy::launch_rope_qknorm(r, s); }));
    hy::FlashArgs f{c->q, k, v, c->merged, T, c->nh, c->nkv, c->hd, Lrows, kv_len, pos0, causal,
                    1.0f / sqrtf((float)c->hd)};
    HY_TRY(timed(c, AK_ATTN, s, [&] { return hy::launch_flash_attn(f, s, c->fa_ws, c->fa_slots, c->decode_waves); }));
    HY_TRY(timed(c, AK_OPROJ, s,
                 [&] {
                     return hy::launch_gemm_nt_f32(c->merged, W.o_w, resid, out, T, c->H, c->nh * c->hd, s,
                                                   c->gemm_ws);
                 }));
    return HY_OK;
}

// GGUF tensor -> f32 host copy (row-major as stored: ne0 innermost): F32, F16, BF16,
// Q8_0 or Q4_0, as the reference loader's read_tensor_data takes every tensor
// (src/hunyuan_gguf_loader.cpp:167-222)
int gguf_f32(const hy::GgufFile& f, const std::string& name, uint64_t ne0, uint64_t ne1, bool optional,
             std::vector<float>& out, bool* present) {
    const hy::GgufTensor* t = f.find(name);
    if (present) *present = t != nullptr;
    if (!t) return optional ? HY_OK : fail(HY_ERR_INVALID, "GGUF file has no tensor %s", name.c_str());
    const uint32_t want_dims = ne1 > 1 ? 2u : 1u;
    if (t->n_dims != want_dims || t->ne[0] != ne0 || (want_dims == 2 && t->ne[1] != ne1))
        return fail(HY_ERR_INVALID, "%s has shape [%llu, %llu], want [%llu, %llu]", name.c_str(),
                    (unsigned long long)t->ne[0], (unsigned long long)t->ne[1], (unsigned long long)ne0,
                    (unsigned long long)ne1);
    out.resize((size_t)ne0 * ne1);
    if (!hy::tensor_to_f32(*t, out.data()))
        return fail(HY_ERR_UNSUPPORTED, "%s has ggml type %d; F32, F16, BF16, Q8_0 or Q4_0 expected", name.c_str(),
                    t->type);
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
    if (cfg->num_layers == 0 || cfg->num_layers > 4096)
        return fail(HY_ERR_INVALID, "num_layers=%u must be in 1..4096", cfg->num_layers);
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
    c->layers.resize(cfg->num_layers);
    const size_t H = c->H, nq = (size_t)c->nh * c->hd, nk = (size_t)c->nkv * c->hd, Tm = c->Tm;
    c->fa_slots = hy::flash_attn_ws_slots(c->Tm, c->Tm > c->Lc ? c->Tm : c->Lc, c->nkv);
    struct Part {
        float** p;
        size_t n;
    } parts[] = {{&c->qkv, Tm * c->nqkv}, {&c->q, Tm * nq},  {&c->kf, Tm * nk},   {&c->vf, Tm * nk},
                 {&c->merged, Tm * nq},   {&c->xn, Tm * H}, {&c->hres, Tm * H},
                 {&c->gemm_ws, hy::gemm_nt_f32_ws_bytes() / 4},
                 {&c->fa_ws, hy::flash_attn_ws_floats(c->hd, c->fa_slots)}};
    size_t total = 0;
    for (auto& p : parts) total += al256(p.n * 4);
    if (hipMalloc(&c->arena, total) != hipSuccess) {
        delete c;
        return fail(HY_ERR_NOMEM, "hipMalloc of %zu bytes for the attention work arena failed", total);
    }
    size_t o = 0;
    for (auto& p : parts) {
        *p.p = reinterpret_cast<float*>(static_cast<uint8_t*>(c->arena) + o);
        o += al256(p.n * 4);
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
    for (auto& L : c->layers)
        if (L.base) (void)hipFree(L.base);
    if (c->arena) (void)hipFree(c->arena);
    delete c;
    return HY_OK;
}

int hy_attn_upload(hy_attn_ctx* c, uint32_t layer, const float* qkv_w, const float* o_w, const float* qn,
                   const float* kn) {
    HY_TRY(check_layer(c, layer, false));
    if (!qkv_w || !o_w || !qn || !kn) return fail(HY_ERR_INVALID, "null weight");
    HIP_TRY(hipSetDevice(c->cfg.device));
    AttnLayer& L = c->layers[layer];
    HY_TRY(alloc_layer(c, L));
    const size_t nq = (size_t)c->nh * c->hd;
    HIP_TRY(hipMemcpy(L.qkv_w, qkv_w, (size_t)c->nqkv * c->H * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(L.o_w, o_w, (size_t)c->H * nq * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(L.q_norm, qn, (size_t)c->hd * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(L.k_norm, kn, (size_t)c->hd * 4, hipMemcpyHostToDevice));
    L.loaded = true;
    return HY_OK;
}

int hy_attn_upload_gguf(hy_attn_ctx* c, uint32_t layer, const hy_gguf* g, uint32_t block) {
    HY_TRY(check_layer(c, layer, false));
    if (!g) return fail(HY_ERR_INVALID, "null file");
    const hy::GgufFile& f = hy::gguf_file(g);
    const std::string p = "blk." + std::to_string(block) + ".";
    const uint64_t H = c->H, nq = (uint64_t)c->nh * c->hd, hd = c->hd;
    std::vector<float> qkv, o, qn, kn, in;
    bool has_in = false;
    // every tensor first: nothing is uploaded from an incomplete or mismatched file
    HY_TRY(gguf_f32(f, p + "attn_qkv.weight", H, (uint64_t)c->nqkv, false, qkv, nullptr));
    HY_TRY(gguf_f32(f, p + "attn_output.weight", nq, H, false, o, nullptr));
    HY_TRY(gguf_f32(f, p + "attn_q_norm.weight", hd, 1, false, qn, nullptr));
    HY_TRY(gguf_f32(f, p + "attn_k_norm.weight", hd, 1, false, kn, nullptr));
    HY_TRY(gguf_f32(f, p + "attn_norm.weight", H, 1, true, in, &has_in));
    HY_TRY(hy_attn_upload(c, layer, qkv.data(), o.data(), qn.data(), kn.data()));
    return hy_attn_set_input_norm(c, layer, has_in ? in.data() : nullptr);
}

int hy_attn_synth_layer(hy_attn_ctx* c, uint32_t layer, uint64_t seed, float std) {
    HY_TRY(check_layer(c, layer, false));
    HIP_TRY(hipSetDevice(c->cfg.device));
    AttnLayer& L = c->layers[layer];
    HY_TRY(alloc_layer(c, L));
    const float scale = std * hy::NORM_SCALE;
    const size_t nq = (size_t)c->nh * c->hd;
    HIP_TRY(hy::launch_synth_fill(L.qkv_w, (size_t)c->nqkv * c->H, hy::stream_key(seed, layer, hy::TENSOR_QKV, 0),
                                  scale, nullptr));
    HIP_TRY(hy::launch_synth_fill(L.o_w, (size_t)c->H * nq, hy::stream_key(seed, layer, hy::TENSOR_O, 0), scale,
                                  nullptr));
    HIP_TRY(hy::launch_fill_f32(L.q_norm, (size_t)c->hd, 1.0f, nullptr));
    HIP_TRY(hy::launch_fill_f32(L.k_norm, (size_t)c->hd, 1.0f, nullptr));
    HIP_TRY(hipDeviceSynchronize());
    L.loaded = true;
    L.has_in_norm = false;
    return HY_OK;
}

int hy_attn_set_input_norm(hy_attn_ctx* c, uint32_t layer, const float* w) {
    HY_TRY(check_layer(c, layer, false));
    AttnLayer& L = c->layers[layer];
    if (!w) {
        L.has_in_norm = false;
        return HY_OK;
    }
    HIP_TRY(hipSetDevice(c->cfg.device));
    HY_TRY(alloc_layer(c, L));
    HIP_TRY(hipMemcpy(L.in_norm, w, (size_t)c->H * 4, hipMemcpyHostToDevice));
    L.has_in_norm = true;
    return HY_OK;
}

int hy_attn_forward(hy_attn_ctx* c, uint32_t layer, const float* x, uint32_t T, const int32_t* positions, float* out,
                    float* dq, float* dk, float* dv, void* stream) {
    HY_TRY(check_layer(c, layer, true));
    if (!x || !out) return fail(HY_ERR_INVALID, "null x/out");
    if (T == 0 || T > (uint32_t)c->Tm) return fail(HY_ERR_INVALID, "T=%u must be in 1..max_tokens=%d", T, c->Tm);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int iT = (int)T;
    HY_TRY(run(c, c->layers[layer], x, iT, hy::ROPE_1D, positions, nullptr, nullptr, 0, c->kf, c->vf, c->Tm, 0, iT,
               1, out, s));
    const size_t nq = (size_t)c->nh * c->hd;
    if (dq) HIP_TRY(hipMemcpyAsync(dq, c->q, (size_t)T * nq * 4, hipMemcpyDeviceToDevice, s));
    if (dk) HIP_TRY(hy::launch_gather_kv(c->kf, c->nkv, c->Tm, 0, iT, c->hd, dk, s));
    if (dv) HIP_TRY(hy::launch_gather_kv(c->vf, c->nkv, c->Tm, 0, iT, c->hd, dv, s));
    return HY_OK;
}

int hy_attn_forward_cached(hy_attn_ctx* c, uint32_t layer, const float* x, uint32_t T, const float* cos_t,
                           const float* sin_t, float* out, void* stream) {
    HY_TRY(check_layer(c, layer, true));
    if (!x || !out) return fail(HY_ERR_INVALID, "null x/out");
    if (T == 0 || T > (uint32_t)c->Tm) return fail(HY_ERR_INVALID, "T=%u must be in 1..max_tokens=%d", T, c->Tm);
    if ((cos_t == nullptr) != (sin_t == nullptr)) return fail(HY_ERR_INVALID, "give both rotary tables or neither");
    AttnLayer& L = c->layers[layer];
    if ((uint64_t)L.cache_len + T > (uint64_t)c->Lc)
        return fail(HY_ERR_INVALID, "cache overflow: %u cached + %u new > max_cache %d", L.cache_len, T, c->Lc);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int pos0 = (int)L.cache_len;
    HY_TRY(run(c, L, x, (int)T, cos_t ? hy::ROPE_TABLE : hy::ROPE_NONE, nullptr, cos_t, sin_t, 1, L.kc, L.vc, c->Lc,
               pos0, pos0 + (int)T, 0, out, s));
    L.cache_len += T;
    return HY_OK;
}

int hy_attn_cache_reset(hy_attn_ctx* c) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    for (auto& L : c->layers) L.cache_len = 0;
    return HY_OK;
}

int hy_attn_cache_len(const hy_attn_ctx* c, uint32_t layer, uint32_t* len) {
    HY_TRY(check_layer(c, layer, false));
    if (!len) return fail(HY_ERR_INVALID, "null len");
    *len = c->layers[layer].cache_len;
    return HY_OK;
}

int hy_decoder_layer_forward(hy_attn_ctx* c, uint32_t attn_layer, hy_moe_ctx* moe, uint32_t moe_layer,
                             const float* x, uint32_t T, const int32_t* positions, float* out, float* debug_h,
                             void* stream) {
    HY_TRY(check_layer(c, attn_layer, true));
    if (!moe) return fail(HY_ERR_INVALID, "null MoE context");
    if (hy::moe_hidden(moe) != c->H || hy::moe_device(moe) != c->cfg.device)
        return fail(HY_ERR_INVALID,
                    "the MoE context (hidden %d, device %d) does not match the attention context (hidden %d, device %d)",
                    hy::moe_hidden(moe), hy::moe_device(moe), c->H, c->cfg.device);
    if (!x || !out) return fail(HY_ERR_INVALID, "null x/out");
    if (T == 0 || T > (uint32_t)c->Tm) return fail(HY_ERR_INVALID, "T=%u must be in 1..max_tokens=%d", T, c->Tm);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int iT = (int)T;
    const float eps = c->cfg.rms_norm_eps;
    const AttnLayer& L = c->layers[attn_layer];
    // input_layernorm -> self-attention -> h = x + attention (in the output projection)
    HIP_TRY(L.has_in_norm ? hy::launch_rms_norm_w(x, L.in_norm, iT, c->H, eps, c->xn, s)
                          : hy::launch_rms_norm(x, iT, c->H, eps, c->xn, s));
    HY_TRY(run(c, L, c->xn, iT, hy::ROPE_1D, positions, nullptr, nullptr, 0, c->kf, c->vf, c->Tm, 0, iT, 1, c->hres,
               s, x));
    if (debug_h) HIP_TRY(hipMemcpyAsync(debug_h, c->hres, (size_t)T * c->H * 4, hipMemcpyDeviceToDevice, s));
    // post_attention_layernorm -> MoE -> out = h + MoE (the MoE context's layer and norm)
    return hy_moe_stack_forward(moe, moe_layer, 1, c->hres, T, eps, out, stream);
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

int hy_lm_head_f32(const float* x, const float* w, const float* resid, uint32_t T, uint32_t hidden, uint32_t vocab,
                   float* out, void* stream) {
    if (!x || !w || !out) return fail(HY_ERR_INVALID, "null pointer");
    if (T == 0 || vocab == 0 || hidden == 0 || hidden % 16)
        return fail(HY_ERR_INVALID, "bad GEMM shape T=%u hidden=%u vocab=%u (hidden a multiple of 16)", T, hidden,
                    vocab);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!hy::gemm_nt_f32_uses_ws((int)T, (int)vocab, (int)hidden)) {
        HIP_TRY(hy::launch_gemm_nt_f32(x, w, resid, out, (int)T, (int)vocab, (int)hidden, s, nullptr));
        return HY_OK;
    }
    // mid-size grids take the stream-K split, which needs a scratch of partial tiles:
    // one per device, allocated on the first such call and kept for the process.  A
    // call waits (on the device) for the previous call's use of it to finish, so calls
    // on different streams stay ordered.  That ordering is an event recorded by eager
    // calls, which a captured graph's replays would not follow: such a shape is refused
    // under stream capture (graph users run the lm_head through hy_model_forward, whose
    // context owns its scratch).
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(s, &cap));
    if (cap != hipStreamCaptureStatusNone)
        return fail(HY_ERR_UNSUPPORTED,
                    "hy_lm_head_f32 with T=%u vocab=%u uses a shared scratch and cannot be captured into a graph",
                    T, vocab);
    static std::mutex mu;
    static std::vector<LmScratch> per_dev;
    std::lock_guard<std::mutex> lock(mu);
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if ((int)per_dev.size() <= dev) per_dev.resize(dev + 1);
    LmScratch& sc = per_dev[dev];
    if (!sc.ws) {
        // both resources exist before the scratch is published; a failure leaves none
        hipEvent_t ev = nullptr;
        HIP_TRY(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
        float* ws = nullptr;
        if (hipMalloc(reinterpret_cast<void**>(&ws), hy::gemm_nt_f32_ws_bytes()) != hipSuccess) {
            (void)hipEventDestroy(ev);
            return fail(HY_ERR_NOMEM, "GEMM scratch allocation failed");
        }
        sc.done = ev;
        sc.ws = ws;
    } else {
        HIP_TRY(hipStreamWaitEvent(s, sc.done, 0));
    }
    HIP_TRY(hy::launch_gemm_nt_f32(x, w, resid, out, (int)T, (int)vocab, (int)hidden, s, sc.ws));
    HIP_TRY(hipEventRecord(sc.done, s));
    return HY_OK;
}

int hy_rope_f32(float* x, uint32_t T, uint32_t heads, uint32_t hd, float theta, const int32_t* positions,
                void* stream) {
    if (!x) return fail(HY_ERR_INVALID, "null x");
    if (hd == 0 || hd % 2) return fail(HY_ERR_INVALID, "head_dim=%u must be even", hd);
    HIP_TRY(hy::launch_rope_apply(x, (int)T, (int)heads, (int)hd, hy::ROPE_1D, positions, theta, nullptr, nullptr,
                                  static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_rope_2d_f32(float* x, uint32_t T, uint32_t heads, uint32_t hd, const float* cos_t, const float* sin_t,
                   void* stream) {
    if (!x || !cos_t || !sin_t) return fail(HY_ERR_INVALID, "null pointer");
    if (hd == 0 || hd % 2) return fail(HY_ERR_INVALID, "head_dim=%u must be even", hd);
    HIP_TRY(hy::launch_rope_apply(x, (int)T, (int)heads, (int)hd, hy::ROPE_TABLE, nullptr, 0.0f, cos_t, sin_t,
                                  static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_embedding_lookup_f32(const int32_t* ids, const float* table, uint32_t T, uint32_t hidden, uint32_t vocab,
                            float* out, void* stream) {
    if (!ids || !table || !out) return fail(HY_ERR_INVALID, "null pointer");
    if (hidden == 0 || hidden % 4) return fail(HY_ERR_INVALID, "hidden=%u must be a multiple of 4", hidden);
    HIP_TRY(hy::launch_embed(ids, table, (int)T, (int)hidden, (int)vocab, out, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_attn_set_decode_waves(hy_attn_ctx* c, uint32_t max_waves) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    if (max_waves > (1u << 20)) return fail(HY_ERR_INVALID, "max_waves=%u out of range", max_waves);
    c->decode_waves = (int)max_waves;
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

// ------------------------------------------------------------------ the backbone

int hy_model_create(const hy_model_config* cfg, hy_model_ctx** out) {
    if (!out) return fail(HY_ERR_INVALID, "null out");
    *out = nullptr;
    if (!cfg) return fail(HY_ERR_INVALID, "null config");
    if (cfg->moe.hidden != cfg->attn.hidden || cfg->moe.num_layers != cfg->attn.num_layers ||
        cfg->moe.max_tokens != cfg->attn.max_tokens || cfg->moe.device != cfg->attn.device)
        return fail(HY_ERR_INVALID, "the MoE and attention configs must agree on hidden, num_layers, max_tokens "
                                    "and device");
    if (cfg->vocab == 0 || cfg->vocab > (1u << 22)) return fail(HY_ERR_INVALID, "vocab=%u out of range", cfg->vocab);
    if (cfg->attn.hidden % 4) return fail(HY_ERR_INVALID, "hidden must be a multiple of 4");
    hy_model_ctx* m = new hy_model_ctx();
    m->cfg = *cfg;
    int rc = hy_attn_create(&cfg->attn, &m->attn);
    if (rc == HY_OK) rc = hy_moe_create(&cfg->moe, &m->moe);
    if (rc != HY_OK) {
        hy_attn_destroy(m->attn);
        delete m;
        return rc;
    }
    m->H = (int)cfg->attn.hidden;
    m->V = (int)cfg->vocab;
    m->Tm = (int)cfg->attn.max_tokens;
    m->L = (int)cfg->attn.num_layers;
    const size_t H = m->H, V = m->V, Tm = m->Tm;
    struct Part {
        float** p;
        size_t n;
    } parts[] = {{&m->embed, V * H}, {&m->fnorm, H}, {&m->lm_head, V * H},
                 {&m->ha, Tm * H},   {&m->hb, Tm * H}, {&m->normed, Tm * H}};
    size_t total = 0;
    for (auto& p : parts) total += al256(p.n * 4);
    if (hipMalloc(&m->arena, total) != hipSuccess) {
        hy_moe_destroy(m->moe);
        hy_attn_destroy(m->attn);
        delete m;
        return fail(HY_ERR_NOMEM, "hipMalloc of %zu bytes for the model's global weights failed", total);
    }
    size_t o = 0;
    for (auto& p : parts) {
        *p.p = reinterpret_cast<float*>(static_cast<uint8_t*>(m->arena) + o);
        o += al256(p.n * 4);
    }
    if (hy::launch_fill_f32(m->fnorm, H, 1.0f, nullptr) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        hy_model_destroy(m);
        return fail(HY_ERR_HIP, "initialising the final norm failed");
    }
    *out = m;
    return HY_OK;
}

int hy_model_destroy(hy_model_ctx* m) {
    if (!m) return HY_OK;
    (void)hipSetDevice(m->cfg.attn.device);
    (void)hipDeviceSynchronize();
    hy_attn_destroy(m->attn);
    hy_moe_destroy(m->moe);
    if (m->arena) (void)hipFree(m->arena);
    delete m;
    return HY_OK;
}

hy_attn_ctx* hy_model_attn(hy_model_ctx* m) { return m ? m->attn : nullptr; }
hy_moe_ctx* hy_model_moe(hy_model_ctx* m) { return m ? m->moe : nullptr; }

int hy_model_upload_globals(hy_model_ctx* m, const float* embedding, const float* final_norm, const float* lm_head) {
    if (!m) return fail(HY_ERR_INVALID, "null ctx");
    HIP_TRY(hipSetDevice(m->cfg.attn.device));
    const size_t VH = (size_t)m->V * m->H;
    if (embedding) HIP_TRY(hipMemcpy(m->embed, embedding, VH * 4, hipMemcpyHostToDevice));
    if (final_norm) HIP_TRY(hipMemcpy(m->fnorm, final_norm, (size_t)m->H * 4, hipMemcpyHostToDevice));
    if (lm_head) HIP_TRY(hipMemcpy(m->lm_head, lm_head, VH * 4, hipMemcpyHostToDevice));
    return HY_OK;
}

int hy_model_upload_globals_gguf(hy_model_ctx* m, const hy_gguf* g) {
    if (!m || !g) return fail(HY_ERR_INVALID, "null argument");
    const hy::GgufFile& f = hy::gguf_file(g);
    std::vector<float> emb, fn, lm;
    HY_TRY(gguf_f32(f, "token_embd.weight", (uint64_t)m->H, (uint64_t)m->V, false, emb, nullptr));
    HY_TRY(gguf_f32(f, "output_norm.weight", (uint64_t)m->H, 1, false, fn, nullptr));
    HY_TRY(gguf_f32(f, "output.weight", (uint64_t)m->H, (uint64_t)m->V, false, lm, nullptr));
    return hy_model_upload_globals(m, emb.data(), fn.data(), lm.data());
}

int hy_model_synth_globals(hy_model_ctx* m, uint64_t seed, float std) {
    if (!m) return fail(HY_ERR_INVALID, "null ctx");
    HIP_TRY(hipSetDevice(m->cfg.attn.device));
    const size_t VH = (size_t)m->V * m->H;
    const float scale = std * hy::NORM_SCALE;
    HIP_TRY(hy::launch_synth_fill(m->embed, VH, hy::stream_key(seed, 0, hy::TENSOR_EMBED, 0), scale, nullptr));
    HIP_TRY(hy::launch_synth_fill(m->lm_head, VH, hy::stream_key(seed, 0, hy::TENSOR_LM_HEAD, 0), scale, nullptr));
    HIP_TRY(hy::launch_fill_f32(m->fnorm, (size_t)m->H, 1.0f, nullptr));
    HIP_TRY(hipDeviceSynchronize());
    return HY_OK;
}

}  // extern "C"

namespace {
// layers 0..n-1 from `in` (not modified); *result is the buffer holding the output
int run_layers(hy_model_ctx* m, const float* in, uint32_t T, const int32_t* positions, uint32_t n, hipStream_t s,
               const float** result) {
    const float* cur = in;
    for (uint32_t l = 0; l < n; l++) {
        float* dst = (cur == m->ha) ? m->hb : m->ha;
        HY_TRY(hy_decoder_layer_forward(m->attn, l, m->moe, l, cur, T, positions, dst, nullptr, s));
        cur = dst;
    }
    *result = cur;
    return HY_OK;
}
}  // namespace

extern "C" {

int hy_model_forward(hy_model_ctx* m, const int32_t* ids, uint32_t T, const int32_t* positions, float* logits,
                     void* stream) {
    if (!m) return fail(HY_ERR_INVALID, "null ctx");
    if (!ids || !logits) return fail(HY_ERR_INVALID, "null ids/logits");
    if (T == 0 || T > (uint32_t)m->Tm) return fail(HY_ERR_INVALID, "T=%u must be in 1..max_tokens=%d", T, m->Tm);
    hipStream_t s = static_cast<hipStream_t>(stream);
    HIP_TRY(hy::launch_embed(ids, m->embed, (int)T, m->H, m->V, m->hb, s));
    const float* h = nullptr;
    HY_TRY(run_layers(m, m->hb, T, positions, (uint32_t)m->L, s, &h));
    HIP_TRY(hy::launch_rms_norm_w(h, m->fnorm, (int)T, m->H, m->cfg.attn.rms_norm_eps, m->normed, s));
    HIP_TRY(hy::launch_gemm_nt_f32(m->normed, m->lm_head, nullptr, logits, (int)T, m->V, m->H, s, m->attn->gemm_ws));
    return HY_OK;
}

int hy_model_forward_hidden(hy_model_ctx* m, const float* embeds, uint32_t T, const int32_t* positions,
                            uint32_t n_layers, float* hidden, void* stream) {
    if (!m) return fail(HY_ERR_INVALID, "null ctx");
    if (!embeds || !hidden) return fail(HY_ERR_INVALID, "null embeds/hidden");
    if (T == 0 || T > (uint32_t)m->Tm) return fail(HY_ERR_INVALID, "T=%u must be in 1..max_tokens=%d", T, m->Tm);
    if (n_layers > (uint32_t)m->L) return fail(HY_ERR_INVALID, "n_layers=%u > %d layers", n_layers, m->L);
    const uint32_t n = n_layers ? n_layers : (uint32_t)m->L;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const float* h = nullptr;
    HY_TRY(run_layers(m, embeds, T, positions, n, s, &h));
    HIP_TRY(hipMemcpyAsync(hidden, h, (size_t)T * m->H * 4, hipMemcpyDeviceToDevice, s));
    return HY_OK;
}

}  // extern "C"
