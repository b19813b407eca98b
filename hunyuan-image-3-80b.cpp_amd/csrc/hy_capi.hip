// hy_capi.hip -- the C ABI (include/hy_moe.h): context, resident weights, work
// arena, forward orchestration, timing.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/hy_moe.h"
#include "hy_device.hpp"
#include "hy_launch.hpp"
#include "hy_layout.hpp"
#include "../host/hy_gguf.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

#define HIP_TRY(expr)                                                                                    \
    do {                                                                                                 \
        hipError_t e_ = (expr);                                                                          \
        if (e_ != hipSuccess) return fail(HY_ERR_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_),   \
                                          __FILE__, __LINE__);                                           \
    } while (0)

#define HY_TRY(expr)              \
    do {                          \
        int r_ = (expr);          \
        if (r_ != HY_OK) return r_; \
    } while (0)

size_t row_bytes(int wtype, int cols) {
    switch (wtype) {
    case HY_TYPE_F32: return (size_t)cols * 4;
    case HY_TYPE_Q8_0: return (size_t)cols;       // resident int8 plane
    case HY_TYPE_Q4_0: return (size_t)cols / 2;   // resident nibble plane
    default: return 0;
    }
}
size_t gguf_row_bytes(int wtype, int cols) {
    switch (wtype) {
    case HY_TYPE_F32: return (size_t)cols * 4;
    case HY_TYPE_Q8_0: return (size_t)cols / 32 * 34;
    case HY_TYPE_Q4_0: return (size_t)cols / 32 * 18;
    default: return 0;
    }
}
size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

struct LayerW {
    uint8_t* base = nullptr;
    float* router = nullptr;
    uint8_t* gu_qs = nullptr;
    uint16_t* gu_sc = nullptr;
    uint8_t* dn_qs = nullptr;
    uint16_t* dn_sc = nullptr;
    float* ffn_norm = nullptr;  // post-attention RMSNorm weight [H] (used when has_norm)
    bool loaded = false;
    bool has_norm = false;
};

struct ProfRec {
    int kid;
    hipEvent_t a, b;
};

}  // namespace

struct hy_moe_ctx {
    hy_moe_config cfg{};
    int H = 0, I = 0, E = 0, K = 0, X = 0;  // X = experts incl. shared slot
    size_t gu_qs_stride = 0, gu_sc_stride = 0, dn_qs_stride = 0, dn_sc_stride = 0;
    size_t layer_bytes = 0;
    std::vector<LayerW> layers;

    // arena
    void* arena = nullptr;
    int8_t* xq = nullptr;
    float* xd = nullptr;
    int* xs = nullptr;
    float* logits = nullptr;
    float* topw = nullptr;
    int* topi = nullptr;
    int *cnt = nullptr, *off = nullptr, *srt_tok = nullptr, *pair_pos = nullptr, *comb_pos = nullptr;
    float* comb_w = nullptr;
    int *tile_e = nullptr, *tile_start = nullptr, *tile_n = nullptr, *meta = nullptr;
    int* dsp_scratch = nullptr;  // per-block counts of the dispatch
    int8_t* hq = nullptr;  // h, block-major in slot order [I/32][T*K+T][32]
    float* hd = nullptr;
    int* hs = nullptr;
    int8_t* xg = nullptr;  // the grouped GEMM's gathered x, block-major in slot order [H/32][T*K+T][32]
    float* xgd = nullptr;
    int* mm_ctr = nullptr;  // the grouped GEMM's work counters (zeroed by the gather before each use)
    float* hf = nullptr;
    float* y = nullptr;
    float* xn = nullptr;
    float* cur = nullptr;
    float* gates = nullptr;  // [max_tokens][E]: the gates the aux loss averages
    float* aux = nullptr;    // the last forward's aux loss
    int max_tiles = 0;

    // routing options beyond the default (resolved from the config)
    int n_group = 0, topk_group = 0;  // group-limited greedy when n_group > 0

    // timing
    bool prof = false;
    std::vector<ProfRec> pending;
    std::vector<hipEvent_t> pool;
    uint64_t prof_n[hy::KID_COUNT] = {};
    double prof_ms[hy::KID_COUNT] = {};

    hipStream_t last_stream = nullptr;
    int path = 0;  // HY_PATH_AUTO / _VALU / _MFMA
};

namespace {

const char* kKernelNames[hy::KID_COUNT] = {"quant_q8_0", "router",  "dispatch", "ffn_up",
                                           "ffn_down",   "combine", "rms_norm", "aux_loss"};

int get_event(hy_moe_ctx* c, hipEvent_t* ev) {
    if (!c->pool.empty()) {
        *ev = c->pool.back();
        c->pool.pop_back();
        return HY_OK;
    }
    // timing-only events: no system-scope fence (cache writeback / invalidate) when
    // they are recorded, which would otherwise be counted in the kernel's time
    HIP_TRY(hipEventCreateWithFlags(ev, hipEventDisableSystemFence));
    return HY_OK;
}

int drain_prof(hy_moe_ctx* c) {
    for (auto& r : c->pending) {
        HIP_TRY(hipEventSynchronize(r.b));
        float ms = 0.f;
        HIP_TRY(hipEventElapsedTime(&ms, r.a, r.b));
        c->prof_n[r.kid]++;
        c->prof_ms[r.kid] += ms;
        c->pool.push_back(r.a);
        c->pool.push_back(r.b);
    }
    c->pending.clear();
    return HY_OK;
}

// Launch wrapper: brackets a launch with events when timing is on.
template <typename F>
int timed(hy_moe_ctx* c, int kid, hipStream_t s, F&& launch) {
    hipEvent_t a = nullptr, b = nullptr;
    if (c->prof) {
        HY_TRY(get_event(c, &a));
        HY_TRY(get_event(c, &b));
        HIP_TRY(hipEventRecord(a, s));
    }
    hipError_t e = launch();
    if (e != hipSuccess)
        return fail(HY_ERR_HIP, "launch of %s failed: %s", kKernelNames[kid], hipGetErrorString(e));
    if (c->prof) {
        HIP_TRY(hipEventRecord(b, s));
        c->pending.push_back({kid, a, b});
        if (c->pending.size() > 4096) HY_TRY(drain_prof(c));
    }
    return HY_OK;
}

// Upper bound on routed tiles of at most NT pairs: an expert with c pairs takes
// ceil(c / NT) tiles, at most min(E, T*K) experts are hit, and a tile holds >= 1 pair.
int tile_bound_routed(int T, int K, int E, int NT) {
    const int pairs = T * K;
    const int hit = E < pairs ? E : pairs;
    const int b = (pairs + hit * (NT - 1)) / NT;
    return b < pairs ? b : pairs;
}

// Renormalise the selected weights?  HY_NORM_TOPK follows topkgating_full
// (src/hunyuan_moe_full.cpp:230: `norm_topk_prob && K > 1`, so one expert keeps
// p * routed_scaling_factor); HY_NORM_ALWAYS follows topkgating_easy and
// moe_forward_cpu (src/attention.cpp:268-275), which renormalise at every K.
int renorm_rule(int32_t norm, uint32_t K) { return (norm == HY_NORM_ALWAYS || (norm != HY_NORM_OFF && K > 1)) ? 1 : 0; }

// largest batch the one-launch decode routing takes; the decode GEMV takes at least
// these in AUTO mode
constexpr uint32_t kGemvMaxTokens = 16;

// AUTO mode: the decode GEMV or the MFMA grouped GEMM.  Measured crossover on one MI355X
// (H 4096, I 3072, E 64, K 8, layer steps over rotating weight sets): Q4_0 GEMV 374 vs
// MFMA 423 us at T=32, 515 vs 478 at T=48 (up to ~5 pairs per expert); Q8_0 452 vs 464
// us at T=20, 512 vs 474 at T=24 (up to ~2.5 pairs per expert).
bool gemv_batch(int wt, uint32_t T, int K, int E) {
    if (T <= kGemvMaxTokens) return true;
    const uint64_t pairs = (uint64_t)T * (uint64_t)K;
    if (wt == HY_TYPE_Q4_0) return pairs <= 5ull * (uint64_t)E;
    if (wt == HY_TYPE_Q8_0) return 2 * pairs <= 5ull * (uint64_t)E;
    return false;
}

int check_cfg(const hy_moe_config* c) {
    if (!c) return fail(HY_ERR_INVALID, "null config");
    if (c->hidden == 0 || c->hidden % 64)
        return fail(HY_ERR_INVALID, "hidden=%u must be a positive multiple of 64", c->hidden);
    if (c->intermediate == 0 || c->intermediate % 32)
        return fail(HY_ERR_INVALID, "intermediate=%u must be a positive multiple of 32", c->intermediate);
    if (c->num_experts == 0 || c->num_experts > hy::MAX_E)
        return fail(HY_ERR_INVALID, "num_experts=%u must be in 1..%d", c->num_experts, hy::MAX_E);
    if (c->topk == 0 || c->topk > c->num_experts || c->topk > (uint32_t)hy::MAX_K)
        return fail(HY_ERR_INVALID, "topk=%u must be in 1..min(num_experts, %d)", c->topk, hy::MAX_K);
    if (c->num_layers == 0) return fail(HY_ERR_INVALID, "num_layers must be >= 1");
    if (c->max_tokens == 0 || c->max_tokens > 16384)
        return fail(HY_ERR_INVALID, "max_tokens=%u must be in 1..16384", c->max_tokens);
    if (c->wtype != HY_TYPE_F32 && c->wtype != HY_TYPE_Q8_0 && c->wtype != HY_TYPE_Q4_0)
        return fail(HY_ERR_UNSUPPORTED, "weight type %d not supported (F32=0, Q4_0=2, Q8_0=8)", c->wtype);
    if (c->group_limited_greedy && c->n_group > 0 && c->topk_group > 64)
        return fail(HY_ERR_INVALID, "topk_group=%u must be <= 64 (topk_f32's bound)", c->topk_group);
    if (c->drop_tokens) {
        // the capacity rule converts capacity_factor * K * T / E to uint32
        const float most = c->capacity_factor * (float)c->topk * (float)c->max_tokens / (float)c->num_experts;
        if (!(c->capacity_factor >= 0.0f) || !(most < 4294967040.0f))
            return fail(HY_ERR_INVALID, "capacity_factor=%g gives no capacity in uint32 range", (double)c->capacity_factor);
    }
    return HY_OK;
}

// Expert capacity under token dropping (src/hunyuan_moe_full.cpp:210-214): float
// arithmetic left to right, truncated, at least K, at least min_capacity.
uint32_t drop_capacity(const hy_moe_config& c, uint32_t T) {
    uint32_t cap = (uint32_t)(c.capacity_factor * c.topk * T / c.num_experts);
    if (cap < c.topk) cap = c.topk;
    if (cap < c.min_capacity) cap = c.min_capacity;
    return cap;
}

hy::MatView gu_view(const hy_moe_ctx* c, const LayerW& L) {
    return {L.gu_qs, L.gu_sc, c->gu_qs_stride, c->gu_sc_stride, 2 * c->I, c->H, c->X};
}
hy::MatView dn_view(const hy_moe_ctx* c, const LayerW& L) {
    return {L.dn_qs, L.dn_sc, c->dn_qs_stride, c->dn_sc_stride, c->H, c->I, c->X};
}
hy::Routing routing(const hy_moe_ctx* c) {
    return {c->topi, c->topw, c->cnt, c->off, c->srt_tok, c->comb_pos, c->comb_w, c->tile_e, c->tile_start,
            c->tile_n, c->meta};
}

int alloc_layer(hy_moe_ctx* c, LayerW& L) {
    if (L.base) return HY_OK;
    void* p = nullptr;
    if (hipMalloc(&p, c->layer_bytes) != hipSuccess)
        return fail(HY_ERR_NOMEM, "hipMalloc of %zu bytes for a layer failed", c->layer_bytes);
    uint8_t* b = static_cast<uint8_t*>(p);
    size_t o = 0;
    L.base = b;
    L.router = reinterpret_cast<float*>(b + o);
    o += align256((size_t)c->E * c->H * 4);
    L.gu_qs = b + o;
    o += align256(c->gu_qs_stride * c->X);
    L.gu_sc = reinterpret_cast<uint16_t*>(b + o);
    o += align256(c->gu_sc_stride * 2 * c->X);
    L.dn_qs = b + o;
    o += align256(c->dn_qs_stride * c->X);
    L.dn_sc = reinterpret_cast<uint16_t*>(b + o);
    o += align256(c->dn_sc_stride * 2 * c->X);
    L.ffn_norm = reinterpret_cast<float*>(b + o);
    return HY_OK;
}

// forward of one layer; resid may be null.  prequant: c->xq/xd/xs already hold the
// Q8_0 form of x (the stack's fused RMSNorm + quantization wrote them).
int forward_impl(hy_moe_ctx* c, uint32_t layer, const float* x, uint32_t T, float* out, const float* resid,
                 hipStream_t s, bool prequant = false) {
    if (layer >= c->layers.size()) return fail(HY_ERR_INVALID, "layer %u out of range", layer);
    const LayerW& L = c->layers[layer];
    if (!L.loaded) return fail(HY_ERR_STATE, "layer %u has no weights", layer);
    if (T == 0 || T > c->cfg.max_tokens)
        return fail(HY_ERR_INVALID, "T=%u must be in 1..max_tokens=%u", T, c->cfg.max_tokens);
    if (!x || !out) return fail(HY_ERR_INVALID, "null x/out");
    c->last_stream = s;
    const int H = c->H, I = c->I, E = c->E, K = c->K, wt = c->cfg.wtype;
    const int iT = (int)T;
    const int has_shared = c->cfg.has_shared ? 1 : 0;
    const int renorm = renorm_rule(c->cfg.norm_topk_prob, c->cfg.topk);
    // expert products: int8 MFMA grouped GEMM for batches, dequant-GEMV for decode.  The
    // grouped GEMM addresses its slot-ordered operands with 32-bit offsets: the gathered
    // x (T*(K+1) x H bytes) and h (T*(K+1) x I bytes) must stay below 2^32 (at H = 4096
    // any T <= 16384 with K <= 62); beyond that the GEMV, which computes the same bits, runs.
    const bool mfma_fits = (uint64_t)T * (uint64_t)(K + 1) * (uint64_t)H < (1ull << 32) &&
                           (uint64_t)T * (uint64_t)(K + 1) * (uint64_t)I < (1ull << 32);
    const bool mfma = c->path != HY_PATH_VALU && hy::mfma_path_ok(wt, H, I) && mfma_fits &&
                      (c->path == HY_PATH_MFMA || !gemv_batch(wt, T, K, E));
    const int shape = mfma ? hy::mfma_shape(iT, K, E, H, I) : -1;
    const int NT = mfma ? hy::mfma_shape_tokens(shape) : hy::gemv_tile_tokens();
    // group-limited greedy, dropping and the aux loss take the general routing path
    const bool ext = c->n_group > 0 || c->cfg.drop_tokens || c->cfg.compute_aux_loss;
    // one token: the router logits and the Q8_0 of x in one launch; the gate/up GEMV's
    // own waves then select the top-k and write the dispatch lists (the selection pass
    // and its kernel boundary go away)
    const bool route1 = !ext && !mfma && iT == 1 && hy::gemv_route1_ok(wt, H);
    if (route1) {
        HY_TRY(timed(c, hy::KID_ROUTER, s, [&] {
            return hy::launch_decode_logits(x, L.router, H, E, c->logits, prequant ? nullptr : c->xq, c->xd, c->xs, s);
        }));
    } else if (!ext && !mfma && wt != HY_TYPE_F32 && T <= kGemvMaxTokens && iT * K <= hy::MAX_DECODE_PAIRS) {
        // decode: router logits, then top-k, dispatch lists and Q8_0 of x in one launch
        HY_TRY(timed(c, hy::KID_ROUTER, s, [&] {
            return hy::launch_route_decode(x, L.router, iT, H, E, K, renorm,
                                           c->cfg.routed_scaling_factor, c->logits, c->topw, c->topi,
                                           prequant ? nullptr : c->xq, c->xd, c->xs, NT, has_shared, c->cnt, c->off, c->srt_tok, c->pair_pos,
                                           c->comb_pos, c->comb_w, c->tile_e, c->tile_start, c->tile_n, c->meta, s);
        }));
    } else {
        // small batches quantize the activations inside the selection pass, large ones
        // in a bandwidth-shaped kernel of their own
        const bool fuse_quant = wt != HY_TYPE_F32 && T <= 32 && !prequant;
        if (wt != HY_TYPE_F32 && !fuse_quant && !prequant)
            HY_TRY(timed(c, hy::KID_QUANT, s, [&] {
                return hy::launch_quant_q8_0(x, (size_t)T * H, c->xq, c->xd, c->xs, nullptr, s);
            }));
        hy::RouteOpts opt;
        opt.n_group = c->n_group;
        opt.topk_group = c->topk_group;
        opt.probs = c->cfg.compute_aux_loss ? c->gates : nullptr;
        HY_TRY(timed(c, hy::KID_ROUTER, s, [&] {
            return hy::launch_router_q(x, L.router, iT, H, E, K, renorm,
                                       c->cfg.routed_scaling_factor, c->logits, c->topw, c->topi,
                                       fuse_quant ? c->xq : nullptr, c->xd, c->xs, s, false, opt);
        }));
        const int cap = c->cfg.drop_tokens ? (int)std::min<uint32_t>(drop_capacity(c->cfg, T), 0x7fffffffu)
                                           : 0x7fffffff;
        HY_TRY(timed(c, hy::KID_DISPATCH, s, [&] {
            return hy::launch_dispatch(c->topi, c->topw, iT, K, E, NT, has_shared, c->cnt, c->off, c->srt_tok,
                                       c->pair_pos, c->comb_pos, c->comb_w, c->tile_e, c->tile_start, c->tile_n,
                                       c->meta, c->dsp_scratch, s, cap);
        }));
        if (c->cfg.compute_aux_loss)
            HY_TRY(timed(c, hy::KID_AUX, s, [&] { return hy::launch_aux_loss(c->gates, c->cnt, iT, E, c->aux, s); }));
    }
    const hy::Routing R = routing(c);
    const hy::ActQ X{c->xq, c->xd, c->xs, H};
    const int routed_bound = tile_bound_routed(iT, K, E, NT);
    const int shared_tiles = has_shared ? (iT + NT - 1) / NT : 0;
    if (mfma) {
        // the dispatched activations: x's Q8_0 rows copied into slot order, block-major
        HY_TRY(timed(c, hy::KID_DISPATCH, s, [&] { return hy::launch_gather_act(X, R, iT, K, H, c->xg, c->xgd, c->mm_ctr, s); }));
        const hy::ActQ XG{c->xg, c->xgd, nullptr, H};
        HY_TRY(timed(c, hy::KID_UP, s, [&] {
            return hy::launch_ffn_up_mfma(wt, shape, routed_bound + shared_tiles, gu_view(c, L), R, XG, iT, H, I, E, K,
                                          c->hq, c->hd, c->hs, c->mm_ctr, s);
        }));
        // routed and shared down products in one launch (y rows for every slot), then
        // the combine
        HY_TRY(timed(c, hy::KID_DOWN, s, [&] {
            return hy::launch_ffn_down_mfma(wt, shape, routed_bound + shared_tiles, dn_view(c, L), R, c->hq, c->hd, iT, H,
                                            I, E, K, c->y, c->mm_ctr, s);
        }));
        HY_TRY(timed(c, hy::KID_COMBINE, s, [&] {
            return hy::launch_combine(R, c->y, iT, H, K, has_shared, resid, out, s);
        }));
        return HY_OK;
    }
    if (route1) {
        const hy::Route1Out r1{c->logits, renorm, c->cfg.routed_scaling_factor, has_shared, c->topw, c->topi, c->cnt,
                               c->off, c->srt_tok, c->pair_pos, c->comb_pos, c->comb_w, c->tile_e, c->tile_start,
                               c->tile_n, c->meta};
        HY_TRY(timed(c, hy::KID_UP, s, [&] {
            return hy::launch_gemv_up_route1(wt, gu_view(c, L), r1, X, H, I, E, K, c->hq, c->hd, c->hs, s);
        }));
    } else {
        HY_TRY(timed(c, hy::KID_UP, s, [&] {
            return hy::launch_gemv_up(wt, routed_bound + shared_tiles, gu_view(c, L), R, X, x, iT, H, I, E, K, c->hq,
                                      c->hd, c->hs, c->hf, s);
        }));
    }
    // decode: routed and shared down products in one launch (the shared expert's rows
    // no longer wait behind the routed ones), then the combine.  (Folding the combine
    // into the down launch through per-row-group completion counters made it slower:
    // several times with an agent-scope release per work group, which writes back the
    // XCD's L2; 21.2 against 16.3 + 4.5 us at T=1 with write-through y stores.)
    HY_TRY(timed(c, hy::KID_DOWN, s, [&] {
        return hy::launch_gemv_down(wt, routed_bound + shared_tiles, dn_view(c, L), R, c->hq, c->hd, c->hs, c->hf, iT,
                                    H, I, E, K, c->y, s);
    }));
    HY_TRY(timed(c, hy::KID_COMBINE, s, [&] {
        return hy::launch_combine(R, c->y, iT, H, K, has_shared, resid, out, s);
    }));
    return HY_OK;
}

// ---- token -> expert dispatch of caller-given top-k pairs (hy_dispatch_pairs*)

int check_dispatch_args(const int32_t* topi, const float* topw, uint32_t T, uint32_t K, uint32_t E,
                        const int32_t* counts, const int32_t* offsets, const int32_t* pos) {
    if (!topi || !topw || !counts || !offsets || !pos) return fail(HY_ERR_INVALID, "null pointer");
    if (T == 0 || T > 16384 || K == 0 || K > (uint32_t)hy::MAX_K || E == 0 || E > (uint32_t)hy::MAX_E || K > E)
        return fail(HY_ERR_INVALID, "bad dispatch shape T=%u K=%u E=%u", T, K, E);
    return HY_OK;
}

int dispatch_max_tiles(uint32_t T, uint32_t K, uint32_t E) { return (int)(((size_t)T * K + E * 7) / 8 + 1); }

// sorted tokens, combine positions and weights, three tile arrays, meta, per-block counts
size_t dispatch_ws_bytes(uint32_t T, uint32_t K, uint32_t E) {
    const size_t pairs = (size_t)T * K;
    return pairs * 4 * 3 + (size_t)dispatch_max_tiles(T, K, E) * 4 * 3 + (size_t)hy::META_INTS * 4 +
           hy::dispatch_scratch_bytes((int)T, (int)K, (int)E);
}

// The three dispatch kernels over a workspace of dispatch_ws_bytes: every word of it
// they read was written earlier in the same call, so it needs no clearing.
hipError_t launch_dispatch_ws(const int32_t* topi, const float* topw, uint32_t T, uint32_t K, uint32_t E,
                              int32_t* counts, int32_t* offsets, int32_t* pos, void* ws, hipStream_t s) {
    const size_t pairs = (size_t)T * K;
    const int max_tiles = dispatch_max_tiles(T, K, E);
    int* srt = static_cast<int*>(ws);
    int* cpos = srt + pairs;
    float* cw = reinterpret_cast<float*>(cpos + pairs);
    int* te = reinterpret_cast<int*>(cw + pairs);
    int* ts = te + max_tiles;
    int* tn = ts + max_tiles;
    int* meta = tn + max_tiles;
    int* dscr = meta + hy::META_INTS;
    return hy::launch_dispatch(topi, topw, (int)T, (int)K, (int)E, 8, 0, counts, offsets, srt, pos, cpos, cw, te, ts,
                               tn, meta, dscr, s);
}

// Scratch of hy_dispatch_pairs_noalloc: a file-scope device array, one copy on every
// GPU the library runs on, held until the process ends (4 MiB covers every call with
// T*K <= 262,144 pairs, e.g. T = 16384 at K = 16 with E = 64: about 3.6 MB; larger
// needs are rejected).  Host
// code never passes the array's name to a kernel: that name is a host-side stand-in,
// not a device address.  The device address comes from hipGetSymbolAddress, taken
// once per device with that device current.
constexpr size_t kDispatchScratchMax = (size_t)4 << 20;
__device__ __align__(256) uint8_t scratch[kDispatchScratchMax];

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // per device ordinal

int scratch_of_device(void** out) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(HY_ERR_HIP, "hipGetSymbolAddress of the dispatch scratch failed: %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return HY_OK;
}

}  // namespace

namespace hy {
int set_last_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}
int moe_hidden(const hy_moe_ctx* c) { return c ? c->H : 0; }
int moe_device(const hy_moe_ctx* c) { return c ? c->cfg.device : -1; }
const GgufFile& gguf_file(const hy_gguf* g);  // host/hy_gguf.cpp
}  // namespace hy

// =====================================================================================
extern "C" {

const char* hy_last_error(void) { return g_last_error.c_str(); }

int hy_moe_create(const hy_moe_config* cfg, hy_moe_ctx** out) {
    if (!out) return fail(HY_ERR_INVALID, "null out");
    *out = nullptr;
    HY_TRY(check_cfg(cfg));
    HIP_TRY(hipSetDevice(cfg->device));
    hy_moe_ctx* c = new hy_moe_ctx();
    c->cfg = *cfg;
    c->H = (int)cfg->hidden;
    c->I = (int)cfg->intermediate;
    c->E = (int)cfg->num_experts;
    c->K = (int)cfg->topk;
    c->X = c->E + (cfg->has_shared ? 1 : 0);
    if (cfg->group_limited_greedy && cfg->n_group > 0 && cfg->topk_group > 0) {
        // n_group > E leaves every group empty (E / n_group == 0): E + 1 means the same
        c->n_group = (int)std::min<uint32_t>(cfg->n_group, cfg->num_experts + 1);
        c->topk_group = (int)cfg->topk_group;
    }
    const int wt = cfg->wtype;
    c->gu_qs_stride = align256(row_bytes(wt, c->H) * 2 * c->I);
    c->gu_sc_stride = wt == HY_TYPE_F32 ? 0 : (size_t)2 * c->I * (c->H / 32);
    c->dn_qs_stride = align256(row_bytes(wt, c->I) * c->H);
    c->dn_sc_stride = wt == HY_TYPE_F32 ? 0 : (size_t)c->H * (c->I / 32);
    c->layer_bytes = align256((size_t)c->E * c->H * 4) + align256(c->gu_qs_stride * c->X) +
                     align256(c->gu_sc_stride * 2 * c->X) + align256(c->dn_qs_stride * c->X) +
                     align256(c->dn_sc_stride * 2 * c->X) + align256((size_t)c->H * 4);
    c->layers.resize(cfg->num_layers);

    // work arena
    const size_t Tm = cfg->max_tokens, H = c->H, I = c->I, E = c->E, K = c->K;
    const size_t pairs = Tm * K, slots = Tm * (K + 1);
    // tiles of the smallest tile size any path uses (the decode GEMV's)
    const int nt_min = hy::GEMV_NT;
    c->max_tiles = tile_bound_routed((int)Tm, (int)K, (int)E, nt_min) + (int)((Tm + nt_min - 1) / nt_min) + 1;
    struct Part {
        void** p;
        size_t bytes;
    };
    std::vector<Part> parts = {
        {(void**)&c->xq, Tm * H},          {(void**)&c->xd, Tm * (H / 32) * 4},
        {(void**)&c->xs, Tm * (H / 32) * 4}, {(void**)&c->logits, Tm * E * 4},
        {(void**)&c->topw, pairs * 4},     {(void**)&c->topi, pairs * 4},
        {(void**)&c->cnt, E * 4},          {(void**)&c->off, (E + 1) * 4},
        {(void**)&c->srt_tok, pairs * 4},  {(void**)&c->pair_pos, pairs * 4},
        {(void**)&c->comb_pos, pairs * 4}, {(void**)&c->comb_w, pairs * 4},
        {(void**)&c->tile_e, (size_t)c->max_tiles * 4}, {(void**)&c->tile_start, (size_t)c->max_tiles * 4},
        {(void**)&c->tile_n, (size_t)c->max_tiles * 4}, {(void**)&c->meta, (size_t)hy::META_INTS * 4},
        {(void**)&c->hq, slots * I},       {(void**)&c->hd, slots * (I / 32) * 4},
        {(void**)&c->hs, slots * (I / 32) * 4},
        {(void**)&c->xg, wt == HY_TYPE_F32 ? 16 : slots * H}, {(void**)&c->xgd, wt == HY_TYPE_F32 ? 16 : slots * (H / 32) * 4},
        {(void**)&c->mm_ctr, (size_t)hy::mfma_counter_ints() * 4},
        {(void**)&c->hf, wt == HY_TYPE_F32 ? slots * I * 4 : 16},
        {(void**)&c->y, slots * H * 4},    {(void**)&c->xn, Tm * H * 4},
        {(void**)&c->cur, Tm * H * 4},
        {(void**)&c->dsp_scratch, hy::dispatch_scratch_bytes((int)Tm, (int)K, (int)E)},
        {(void**)&c->gates, cfg->compute_aux_loss ? Tm * E * 4 : 16}, {(void**)&c->aux, 16},
    };
    size_t total = 0;
    for (auto& p : parts) total += align256(p.bytes);
    if (hipMalloc(&c->arena, total) != hipSuccess) {
        delete c;
        return fail(HY_ERR_NOMEM, "hipMalloc of a %zu-byte work arena failed", total);
    }
    size_t o = 0;
    for (auto& p : parts) {
        *p.p = static_cast<uint8_t*>(c->arena) + o;
        o += align256(p.bytes);
    }
    if (hipMemset(c->arena, 0, total) != hipSuccess) {
        (void)hipFree(c->arena);
        delete c;
        return fail(HY_ERR_HIP, "hipMemset of the work arena failed");
    }
    *out = c;
    return HY_OK;
}

int hy_moe_destroy(hy_moe_ctx* c) {
    if (!c) return HY_OK;
    (void)hipDeviceSynchronize();
    for (auto& L : c->layers)
        if (L.base) (void)hipFree(L.base);
    if (c->arena) (void)hipFree(c->arena);
    for (auto& r : c->pending) {
        (void)hipEventDestroy(r.a);
        (void)hipEventDestroy(r.b);
    }
    for (auto e : c->pool) (void)hipEventDestroy(e);
    delete c;
    return HY_OK;
}

size_t hy_moe_layer_bytes(const hy_moe_ctx* c) { return c ? c->layer_bytes : 0; }

extern "C++" {
namespace {

// Upload one layer: the router (f32 [E][H]) and, for every resident matrix e
// (routed experts, then the shared one), gate_up [2I][H] and down [H][I] in ggml
// layout from host memory; each is staged on the device and repacked.
template <class GU, class DN>
int upload_layer(hy_moe_ctx* c, uint32_t layer, const float* router, GU gu_of, DN dn_of) {
    HIP_TRY(hipSetDevice(c->cfg.device));
    LayerW& L = c->layers[layer];
    HY_TRY(alloc_layer(c, L));
    const int wt = c->cfg.wtype, H = c->H, I = c->I, E = c->E;
    const size_t gu_b = gguf_row_bytes(wt, H) * 2 * I, dn_b = gguf_row_bytes(wt, I) * H;
    void* staging = nullptr;
    if (hipMalloc(&staging, gu_b > dn_b ? gu_b : dn_b) != hipSuccess)
        return fail(HY_ERR_NOMEM, "staging allocation failed");
    int rc = HY_OK;
    auto up = [&](const void* src, size_t bytes, int rows, int cols, int guI, uint8_t* qs, uint16_t* sc) -> int {
        HIP_TRY(hipMemcpy(staging, src, bytes, hipMemcpyHostToDevice));
        HIP_TRY(hy::launch_repack(wt, static_cast<uint8_t*>(staging), rows, cols, guI, qs, sc, nullptr));
        return HY_OK;
    };
    for (int e = 0; e < c->X && rc == HY_OK; e++) {
        rc = up(gu_of(e), gu_b, 2 * I, H, I, L.gu_qs + (size_t)e * c->gu_qs_stride,
                L.gu_sc ? L.gu_sc + (size_t)e * c->gu_sc_stride : nullptr);
        if (rc == HY_OK)
            rc = up(dn_of(e), dn_b, H, I, 0, L.dn_qs + (size_t)e * c->dn_qs_stride,
                    L.dn_sc ? L.dn_sc + (size_t)e * c->dn_sc_stride : nullptr);
    }
    if (rc == HY_OK && hipMemcpy(L.router, router, (size_t)E * H * 4, hipMemcpyHostToDevice) != hipSuccess)
        rc = fail(HY_ERR_HIP, "router upload failed");
    if (rc == HY_OK && hipDeviceSynchronize() != hipSuccess) rc = fail(HY_ERR_HIP, "repack failed");
    (void)hipFree(staging);
    if (rc == HY_OK) L.loaded = true;
    return rc;
}

}  // namespace
}  // extern "C++"

int hy_moe_upload_layer(hy_moe_ctx* c, uint32_t layer, const float* router, const void* sgu, const void* sdn,
                        const void* gu, const void* dn) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    if (layer >= c->layers.size()) return fail(HY_ERR_INVALID, "layer %u out of range", layer);
    if (!router || !gu || !dn) return fail(HY_ERR_INVALID, "null router/gu/dn");
    if (c->cfg.has_shared && (!sgu || !sdn)) return fail(HY_ERR_INVALID, "config has a shared expert: pass it");
    const int wt = c->cfg.wtype, H = c->H, I = c->I, E = c->E;
    const size_t gu_b = gguf_row_bytes(wt, H) * 2 * I, dn_b = gguf_row_bytes(wt, I) * H;
    return upload_layer(
        c, layer, router,
        [&](int e) -> const void* { return e < E ? static_cast<const uint8_t*>(gu) + (size_t)e * gu_b : sgu; },
        [&](int e) -> const void* { return e < E ? static_cast<const uint8_t*>(dn) + (size_t)e * dn_b : sdn; });
}

int hy_moe_upload_layer_gguf(hy_moe_ctx* c, uint32_t layer, const hy_gguf* g, uint32_t block) {
    if (!c || !g) return fail(HY_ERR_INVALID, "null ctx/file");
    if (layer >= c->layers.size()) return fail(HY_ERR_INVALID, "layer %u out of range", layer);
    const hy::GgufFile& f = hy::gguf_file(g);
    const int wt = c->cfg.wtype, H = c->H, I = c->I, E = c->E;
    // metadata the converter writes, when present, must describe this context
    const struct {
        const char* key;
        uint32_t want;
    } meta[] = {{"hunyuan.hidden_size", (uint32_t)H},
                {"hunyuan.moe_intermediate_size", (uint32_t)I},
                {"hunyuan.num_experts", (uint32_t)E},
                {"hunyuan.moe_topk", (uint32_t)c->K}};
    for (const auto& m : meta) {
        const hy::GgufValue* v = f.kv(m.key);
        if (v && (v->type == hy::GGUF_U32 || v->type == hy::GGUF_U64) && v->u != m.want)
            return fail(HY_ERR_INVALID, "%s = %llu in the file, the context has %u", m.key, (unsigned long long)v->u,
                        m.want);
    }
    // every tensor first: nothing is uploaded from an incomplete or mismatched file
    auto find2 = [&](const std::string& name, uint64_t ne0, uint64_t ne1, const hy::GgufTensor** out) -> int {
        const hy::GgufTensor* t = f.find(name);
        if (!t) return fail(HY_ERR_INVALID, "GGUF file has no tensor %s", name.c_str());
        if (t->n_dims != 2 || t->ne[0] != ne0 || t->ne[1] != ne1)
            return fail(HY_ERR_INVALID, "%s has shape [%llu, %llu], the context wants [%llu, %llu]", name.c_str(),
                        (unsigned long long)t->ne[0], (unsigned long long)t->ne[1], (unsigned long long)ne0,
                        (unsigned long long)ne1);
        *out = t;
        return HY_OK;
    };
    auto convertible = [](int type) {
        return type == hy::GGML_F32 || type == hy::GGML_F16 || type == hy::GGML_BF16 || type == hy::GGML_Q8_0 ||
               type == hy::GGML_Q4_0;
    };
    // expert matrices: as stored when of the context's type; into an F32 context any
    // convertible type becomes f32; Q4_0 into a Q8_0 context is re-encoded exactly
    auto expert_ok = [&](const hy::GgufTensor* t) -> int {
        if (t->type == wt || (wt == HY_TYPE_F32 && convertible(t->type)) ||
            (wt == HY_TYPE_Q8_0 && t->type == hy::GGML_Q4_0))
            return HY_OK;
        if (!convertible(t->type))
            return fail(HY_ERR_INVALID, "%s has ggml type %d, the context wants %d", t->name.c_str(), t->type, wt);
        return fail(HY_ERR_UNSUPPORTED,
                    "%s has ggml type %d: turning it into the context's type %d would change the weights "
                    "(create the context with wtype F32, or use a file of type %d)",
                    t->name.c_str(), t->type, wt, wt);
    };
    const std::string pfx = "blk." + std::to_string(block) + ".";
    const hy::GgufTensor* router_t = nullptr;
    HY_TRY(find2(pfx + "ffn_gate.weight", (uint64_t)H, (uint64_t)E, &router_t));
    if (!convertible(router_t->type))
        return fail(HY_ERR_UNSUPPORTED, "%sffn_gate.weight has ggml type %d; F32, F16, BF16, Q8_0 or Q4_0 expected",
                    pfx.c_str(), router_t->type);
    std::vector<const hy::GgufTensor*> gus(c->X), dns(c->X);
    for (int e = 0; e < c->X; e++) {
        const std::string base = e < E ? pfx + "ffn_expert_" + std::to_string(e) + "_" : pfx + "ffn_shared_";
        HY_TRY(find2(base + "gate_up.weight", (uint64_t)H, (uint64_t)2 * I, &gus[e]));
        HY_TRY(expert_ok(gus[e]));
        HY_TRY(find2(base + "down.weight", (uint64_t)I, (uint64_t)H, &dns[e]));
        HY_TRY(expert_ok(dns[e]));
    }
    // the post-attention RMSNorm weight (post_attention_layernorm -> ffn_norm), [H];
    // optional: a file without it leaves the layer at unit weight
    const hy::GgufTensor* norm_t = f.find(pfx + "ffn_norm.weight");
    if (norm_t && (!convertible(norm_t->type) || norm_t->n_dims != 1 || norm_t->ne[0] != (uint64_t)H))
        return fail(HY_ERR_INVALID, "%sffn_norm.weight must be [%d] of F32/F16/BF16/Q8_0/Q4_0 (type %d, %u dims, ne0 %llu)",
                    pfx.c_str(), H, norm_t->type, norm_t->n_dims, (unsigned long long)norm_t->ne[0]);
    std::vector<float> router((size_t)E * H), norm(norm_t ? (size_t)H : 0);
    hy::tensor_to_f32(*router_t, router.data());
    if (norm_t) hy::tensor_to_f32(*norm_t, norm.data());
    // one conversion buffer per matrix kind: upload_layer takes expert e's gate_up,
    // then its down, before asking for expert e + 1
    std::vector<uint8_t> gu_buf, dn_buf;
    auto as_ctx = [&](const hy::GgufTensor* t, std::vector<uint8_t>& buf) -> const void* {
        if (t->type == wt) return t->data;
        const uint64_t n = t->ne[0] * t->ne[1];
        if (wt == HY_TYPE_F32) {
            buf.resize(n * 4);
            hy::tensor_to_f32(*t, reinterpret_cast<float*>(buf.data()));
        } else {  // Q4_0 -> Q8_0
            buf.resize(n / 32 * 34);
            hy::q4_0_to_q8_0(t->data, buf.data(), n / 32);
        }
        return buf.data();
    };
    HY_TRY(upload_layer(
        c, layer, router.data(), [&](int e) -> const void* { return as_ctx(gus[e], gu_buf); },
        [&](int e) -> const void* { return as_ctx(dns[e], dn_buf); }));
    return hy_moe_set_ffn_norm(c, layer, norm_t ? norm.data() : nullptr);
}

int hy_moe_synth_layer(hy_moe_ctx* c, uint32_t layer, uint64_t seed, float std, const float* bias) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    if (layer >= c->layers.size()) return fail(HY_ERR_INVALID, "layer %u out of range", layer);
    HIP_TRY(hipSetDevice(c->cfg.device));
    LayerW& L = c->layers[layer];
    HY_TRY(alloc_layer(c, L));
    const int wt = c->cfg.wtype, H = c->H, I = c->I, E = c->E;
    const float scale = std * hy::NORM_SCALE;
    HIP_TRY(hy::launch_synth_fill(L.router, (size_t)E * H, hy::stream_key(seed, layer, hy::TENSOR_ROUTER, 0), scale,
                                  nullptr));
    if (bias) HIP_TRY(hipMemcpy2D(L.router, (size_t)H * 4, bias, 4, 4, E, hipMemcpyHostToDevice));
    for (int e = 0; e < c->X; e++) {
        HIP_TRY(hy::launch_synth_matrix(wt, hy::stream_key(seed, layer, hy::TENSOR_GU, e), scale, 2 * I, H, I,
                                        L.gu_qs + (size_t)e * c->gu_qs_stride,
                                        L.gu_sc ? L.gu_sc + (size_t)e * c->gu_sc_stride : nullptr, nullptr));
        HIP_TRY(hy::launch_synth_matrix(wt, hy::stream_key(seed, layer, hy::TENSOR_DN, e), scale, H, I, 0,
                                        L.dn_qs + (size_t)e * c->dn_qs_stride,
                                        L.dn_sc ? L.dn_sc + (size_t)e * c->dn_sc_stride : nullptr, nullptr));
    }
    HIP_TRY(hipDeviceSynchronize());
    L.loaded = true;
    return HY_OK;
}

int hy_moe_set_ffn_norm(hy_moe_ctx* c, uint32_t layer, const float* w) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    if (layer >= c->layers.size()) return fail(HY_ERR_INVALID, "layer %u out of range", layer);
    LayerW& L = c->layers[layer];
    if (!w) {
        L.has_norm = false;
        return HY_OK;
    }
    HIP_TRY(hipSetDevice(c->cfg.device));
    HY_TRY(alloc_layer(c, L));
    HIP_TRY(hipMemcpy(L.ffn_norm, w, (size_t)c->H * 4, hipMemcpyHostToDevice));
    L.has_norm = true;
    return HY_OK;
}

int hy_moe_forward(hy_moe_ctx* c, uint32_t layer, const float* x, uint32_t T, float* out, void* stream) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    return forward_impl(c, layer, x, T, out, nullptr, static_cast<hipStream_t>(stream));
}

int hy_moe_forward_debug(hy_moe_ctx* c, uint32_t layer, const float* x, uint32_t T, float* out, float* lg, float* w,
                         int32_t* idx, void* stream) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    hipStream_t s = static_cast<hipStream_t>(stream);
    HY_TRY(forward_impl(c, layer, x, T, out, nullptr, s));
    if (lg) HIP_TRY(hipMemcpyAsync(lg, c->logits, (size_t)T * c->E * 4, hipMemcpyDeviceToDevice, s));
    if (w) HIP_TRY(hipMemcpyAsync(w, c->topw, (size_t)T * c->K * 4, hipMemcpyDeviceToDevice, s));
    if (idx) HIP_TRY(hipMemcpyAsync(idx, c->topi, (size_t)T * c->K * 4, hipMemcpyDeviceToDevice, s));
    return HY_OK;
}

int hy_moe_stack_forward(hy_moe_ctx* c, uint32_t first, uint32_t n, const float* x, uint32_t T, float eps,
                         float* out, void* stream) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    if (n == 0 || first + n > c->layers.size()) return fail(HY_ERR_INVALID, "layer range out of bounds");
    if (T == 0 || T > c->cfg.max_tokens) return fail(HY_ERR_INVALID, "T out of range");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t bytes = (size_t)T * c->H * 4;
    HIP_TRY(hipMemcpyAsync(c->cur, x, bytes, hipMemcpyDeviceToDevice, s));
    for (uint32_t l = 0; l < n; l++) {
        const LayerW& L = c->layers[first + l];
        const float* w = L.has_norm ? L.ffn_norm : nullptr;
        // quantized weights: the RMSNorm also writes the Q8_0 activations, so the
        // layer's routing pass does not quantize again
        const bool pq = c->cfg.wtype != HY_TYPE_F32;
        HY_TRY(timed(c, hy::KID_RMSNORM, s, [&] {
            if (pq) return hy::launch_rms_norm_quant(c->cur, w, (int)T, c->H, eps, c->xn, c->xq, c->xd, c->xs, s);
            return w ? hy::launch_rms_norm_w(c->cur, w, (int)T, c->H, eps, c->xn, s)
                     : hy::launch_rms_norm(c->cur, (int)T, c->H, eps, c->xn, s);
        }));
        // residual fused into the combine; in place on cur (each element read then written by one thread)
        HY_TRY(forward_impl(c, first + l, c->xn, T, c->cur, c->cur, s, pq));
    }
    HIP_TRY(hipMemcpyAsync(out, c->cur, bytes, hipMemcpyDeviceToDevice, s));
    return HY_OK;
}

// ---------------------------------------------------------------- stateless kernels
int hy_router_topk(const float* x, const float* wr, uint32_t T, uint32_t H, uint32_t E, uint32_t K, int32_t norm,
                   float scale, float* lg, float* w, int32_t* idx, void* stream) {
    if (!x || !wr || !lg || !w || !idx) return fail(HY_ERR_INVALID, "null pointer");
    if (T == 0 || H == 0 || H % 4 || E == 0 || E > (uint32_t)hy::MAX_E || K == 0 || K > E || K > (uint32_t)hy::MAX_K)
        return fail(HY_ERR_INVALID, "bad router shape T=%u H=%u E=%u K=%u", T, H, E, K);
    HIP_TRY(hy::launch_router(x, wr, (int)T, (int)H, (int)E, (int)K, renorm_rule(norm, K), scale, lg, w, idx,
                              static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_topkgating_easy(const float* lg, uint32_t T, uint32_t E, uint32_t K, float* w, int32_t* idx, void* stream) {
    if (!lg || !w || !idx) return fail(HY_ERR_INVALID, "null pointer");
    if (T == 0 || E == 0 || E > (uint32_t)hy::MAX_E || K == 0 || K > E || K > (uint32_t)hy::MAX_K)
        return fail(HY_ERR_INVALID, "bad gating shape");
    // topkgating_easy renormalises at every K (src/hunyuan_moe_full.cpp:104-108)
    HIP_TRY(hy::launch_topk_from_logits(lg, (int)T, (int)E, (int)K, 1, 1.0f, w, idx, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_route_logits(const float* lg, uint32_t T, uint32_t E, uint32_t K, int32_t norm, float scale, float* w,
                    int32_t* idx, void* stream) {
    if (!lg || !w || !idx) return fail(HY_ERR_INVALID, "null pointer");
    if (T == 0 || E == 0 || E > (uint32_t)hy::MAX_E || K == 0 || K > E || K > (uint32_t)hy::MAX_K)
        return fail(HY_ERR_INVALID, "bad routing shape");
    HIP_TRY(hy::launch_topk_from_logits(lg, (int)T, (int)E, (int)K, renorm_rule(norm, K), scale, w, idx,
                                        static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_route_logits_groups(const float* lg, uint32_t T, uint32_t E, uint32_t K, int32_t norm, float scale,
                           uint32_t n_group, uint32_t topk_group, float* w, int32_t* idx, float* probs, void* stream) {
    if (!lg || !w || !idx) return fail(HY_ERR_INVALID, "null pointer");
    if (T == 0 || E == 0 || E > (uint32_t)hy::MAX_E || K == 0 || K > E || K > (uint32_t)hy::MAX_K)
        return fail(HY_ERR_INVALID, "bad routing shape");
    if (n_group > 0 && topk_group > 64) return fail(HY_ERR_INVALID, "topk_group must be <= 64 (topk_f32's bound)");
    hy::RouteOpts opt;
    // n_group > E leaves every group empty (E / n_group == 0): E + 1 means the same
    opt.n_group = (int)std::min<uint32_t>(n_group, E + 1);
    opt.topk_group = (int)topk_group;
    opt.probs = probs;
    HIP_TRY(hy::launch_topk_from_logits(lg, (int)T, (int)E, (int)K, renorm_rule(norm, K), scale, w, idx,
                                        static_cast<hipStream_t>(stream), opt));
    return HY_OK;
}

int hy_aux_loss(const float* probs, const int32_t* counts, uint32_t T, uint32_t E, float* out, void* stream) {
    if (!probs || !counts || !out) return fail(HY_ERR_INVALID, "null pointer");
    if (T == 0 || E == 0 || E > (uint32_t)hy::MAX_E) return fail(HY_ERR_INVALID, "bad aux-loss shape");
    HIP_TRY(hy::launch_aux_loss(probs, counts, (int)T, (int)E, out, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_softmax_rows(float* x, uint32_t rows, uint32_t n, void* stream) {
    if (!x || rows == 0 || n == 0 || n > 1024) return fail(HY_ERR_INVALID, "bad softmax shape");
    HIP_TRY(hy::launch_softmax_rows(x, (int)rows, (int)n, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_quantize_q8_0(const float* x, uint32_t rows, uint32_t n, void* blocks, void* stream) {
    if (!x || !blocks || n % 32) return fail(HY_ERR_INVALID, "bad quantize arguments (n %% 32 == 0)");
    HIP_TRY(hy::launch_quant_q8_0(x, (size_t)rows * n, nullptr, nullptr, nullptr, static_cast<uint8_t*>(blocks),
                                  static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_dequantize(int32_t type, const void* blocks, size_t n, float* out, void* stream) {
    if (!blocks || !out || n % 32) return fail(HY_ERR_INVALID, "bad dequantize arguments");
    if (type != HY_TYPE_Q8_0 && type != HY_TYPE_Q4_0 && type != HY_TYPE_F32)
        return fail(HY_ERR_UNSUPPORTED, "type %d", type);
    HIP_TRY(hy::launch_dequant(type, static_cast<const uint8_t*>(blocks), n, out, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_block_dots(int32_t wtype, const void* w, const void* x, uint32_t rows, uint32_t n, int32_t path, int32_t* out,
                  void* stream) {
    if (!w || !x || !out || n % 32 || rows == 0 || rows > 4096) return fail(HY_ERR_INVALID, "bad block-dot args");
    if (wtype != HY_TYPE_Q8_0 && wtype != HY_TYPE_Q4_0) return fail(HY_ERR_UNSUPPORTED, "wtype %d", wtype);
    if (path != 0 && path != 1) return fail(HY_ERR_INVALID, "block-dot path %d (0 = VALU, 1 = MFMA)", path);
    auto* wb = static_cast<const uint8_t*>(w);
    auto* xb = static_cast<const uint8_t*>(x);
    if (path == 0)
        HIP_TRY(hy::launch_block_dots_valu(wtype, wb, xb, (int)rows, (int)(n / 32), out, static_cast<hipStream_t>(stream)));
    else
        HIP_TRY(hy::launch_block_dots_mfma(wtype, wb, xb, (int)rows, (int)(n / 32), out, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_rms_norm(const float* x, uint32_t T, uint32_t H, float eps, float* out, void* stream) {
    if (!x || !out || T == 0 || H == 0 || H % 4) return fail(HY_ERR_INVALID, "bad rms_norm args");
    HIP_TRY(hy::launch_rms_norm(x, (int)T, (int)H, eps, out, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_rms_norm_w(const float* x, const float* w, uint32_t T, uint32_t H, float eps, float* out, void* stream) {
    if (!w) return hy_rms_norm(x, T, H, eps, out, stream);
    if (!x || !out || T == 0 || H == 0 || H % 4) return fail(HY_ERR_INVALID, "bad rms_norm args");
    HIP_TRY(hy::launch_rms_norm_w(x, w, (int)T, (int)H, eps, out, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_topk_rows(const float* x, uint32_t rows, uint32_t n, uint32_t k, float* vals, int32_t* idx, void* stream) {
    if (!x || !vals || !idx || rows == 0 || n == 0 || n > 4096 || k == 0 || k > 64)
        return fail(HY_ERR_INVALID, "bad top-k arguments (n <= 4096, 1 <= k <= 64)");
    HIP_TRY(hy::launch_topk_rows(x, (int)rows, (int)n, (int)k, vals, idx, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_dispatch_pairs(const int32_t* topi, const float* topw, uint32_t T, uint32_t K, uint32_t E, int32_t* counts,
                      int32_t* offsets, int32_t* pos, void* stream) {
    HY_TRY(check_dispatch_args(topi, topw, T, K, E, counts, offsets, pos));
    hipStream_t s = static_cast<hipStream_t>(stream);
    // scratch for the lists the layer forward also builds
    void* ws = nullptr;
    if (hipMalloc(&ws, dispatch_ws_bytes(T, K, E)) != hipSuccess) return fail(HY_ERR_NOMEM, "dispatch scratch");
    hipError_t e = launch_dispatch_ws(topi, topw, T, K, E, counts, offsets, pos, ws, s);
    hipError_t e2 = hipStreamSynchronize(s);
    (void)hipFree(ws);
    if (e != hipSuccess || e2 != hipSuccess)
        return fail(HY_ERR_HIP, "dispatch failed: %s", hipGetErrorString(e != hipSuccess ? e : e2));
    return HY_OK;
}

int hy_dispatch_pairs_noalloc(const int32_t* topi, const float* topw, uint32_t T, uint32_t K, uint32_t E,
                              int32_t* counts, int32_t* offsets, int32_t* pos, void* stream) {
    HY_TRY(check_dispatch_args(topi, topw, T, K, E, counts, offsets, pos));
    const size_t bytes = dispatch_ws_bytes(T, K, E);
    if (bytes > kDispatchScratchMax)
        return fail(HY_ERR_INVALID, "dispatch of T=%u K=%u E=%u needs %zu bytes of scratch, more than the %zu this "
                    "entry point holds", T, K, E, bytes, kDispatchScratchMax);
    void* ws = nullptr;
    HY_TRY(scratch_of_device(&ws));
    HIP_TRY(launch_dispatch_ws(topi, topw, T, K, E, counts, offsets, pos, ws, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_einsum_dispatch(const float* x, uint32_t T, uint32_t H, const uint8_t* mask, uint32_t E, uint32_t C, float* out,
                       void* stream) {
    if (!x || !mask || !out || T == 0 || H == 0 || E == 0 || C == 0) return fail(HY_ERR_INVALID, "bad arguments");
    HIP_TRY(hy::launch_einsum_dispatch(x, (int)T, (int)H, mask, (int)E, (int)C, out, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

int hy_einsum_combine(const float* cw, const float* eo, uint32_t T, uint32_t H, uint32_t E, uint32_t C, float* out,
                      void* stream) {
    if (!cw || !eo || !out || T == 0 || H == 0 || E == 0 || C == 0) return fail(HY_ERR_INVALID, "bad arguments");
    HIP_TRY(hy::launch_einsum_combine(cw, eo, (int)T, (int)H, (int)E, (int)C, out, static_cast<hipStream_t>(stream)));
    return HY_OK;
}

// ---------------------------------------------------------------- memory / streams
int hy_device_count(int* n) {
    HIP_TRY(hipGetDeviceCount(n));
    return HY_OK;
}
int hy_set_device(int d) {
    HIP_TRY(hipSetDevice(d));
    return HY_OK;
}
int hy_malloc(void** p, size_t bytes) {
    if (hipMalloc(p, bytes) != hipSuccess) return fail(HY_ERR_NOMEM, "hipMalloc(%zu) failed", bytes);
    return HY_OK;
}
int hy_free(void* p) {
    HIP_TRY(hipFree(p));
    return HY_OK;
}
int hy_memcpy_h2d(void* d, const void* s, size_t b) {
    HIP_TRY(hipMemcpy(d, s, b, hipMemcpyHostToDevice));
    return HY_OK;
}
int hy_memcpy_d2h(void* d, const void* s, size_t b) {
    HIP_TRY(hipMemcpy(d, s, b, hipMemcpyDeviceToHost));
    return HY_OK;
}
int hy_memset(void* d, int v, size_t b) {
    HIP_TRY(hipMemset(d, v, b));
    return HY_OK;
}
int hy_copy_d2d(void* d, const void* src, size_t b, void* stream) {
    if (b && (!d || !src)) return fail(HY_ERR_INVALID, "null copy operand");
    HIP_TRY(hy::launch_copy(d, src, b, (hipStream_t)stream));
    return HY_OK;
}
int hy_device_synchronize(void) {
    HIP_TRY(hipDeviceSynchronize());
    return HY_OK;
}
int hy_stream_create(void** s) {
    hipStream_t st;
    HIP_TRY(hipStreamCreate(&st));
    *s = st;
    return HY_OK;
}
int hy_stream_destroy(void* s) {
    HIP_TRY(hipStreamDestroy(static_cast<hipStream_t>(s)));
    return HY_OK;
}
int hy_stream_synchronize(void* s) {
    HIP_TRY(hipStreamSynchronize(static_cast<hipStream_t>(s)));
    return HY_OK;
}
int hy_event_create(void** ev) {
    hipEvent_t e;
    HIP_TRY(hipEventCreate(&e));
    *ev = e;
    return HY_OK;
}
int hy_event_destroy(void* ev) {
    HIP_TRY(hipEventDestroy(static_cast<hipEvent_t>(ev)));
    return HY_OK;
}
int hy_event_record(void* ev, void* s) {
    HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(ev), static_cast<hipStream_t>(s)));
    return HY_OK;
}
int hy_graph_begin(void* s) {
    if (!s) return fail(HY_ERR_INVALID, "capture needs a created stream (not the null stream)");
    HIP_TRY(hipStreamBeginCapture(static_cast<hipStream_t>(s), hipStreamCaptureModeThreadLocal));
    return HY_OK;
}
int hy_graph_end(void* s, void** exec) {
    if (!s || !exec) return fail(HY_ERR_INVALID, "null stream/exec");
    hipGraph_t g = nullptr;
    HIP_TRY(hipStreamEndCapture(static_cast<hipStream_t>(s), &g));
    hipGraphExec_t x = nullptr;
    const hipError_t e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    HIP_TRY(e);
    *exec = x;
    return HY_OK;
}
int hy_graph_launch(void* exec, void* s) {
    if (!exec) return fail(HY_ERR_INVALID, "null graph");
    HIP_TRY(hipGraphLaunch(static_cast<hipGraphExec_t>(exec), static_cast<hipStream_t>(s)));
    return HY_OK;
}
int hy_graph_destroy(void* exec) {
    if (exec) HIP_TRY(hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec)));
    return HY_OK;
}
int hy_event_elapsed_ms(void* a, void* b, float* ms) {
    HIP_TRY(hipEventSynchronize(static_cast<hipEvent_t>(b)));
    HIP_TRY(hipEventElapsedTime(ms, static_cast<hipEvent_t>(a), static_cast<hipEvent_t>(b)));
    return HY_OK;
}
int hy_synth_fill(float* dev, size_t n, uint64_t seed, uint32_t layer, uint32_t tensor, uint32_t expert, float std,
                  void* stream) {
    if (!dev) return fail(HY_ERR_INVALID, "null pointer");
    HIP_TRY(hy::launch_synth_fill(dev, n, hy::stream_key(seed, layer, tensor, expert), std * hy::NORM_SCALE,
                                  static_cast<hipStream_t>(stream)));
    return HY_OK;
}

// ---------------------------------------------------------------- timing
int hy_moe_set_path(hy_moe_ctx* c, int32_t path) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    if (path < HY_PATH_AUTO || path > HY_PATH_MFMA) return fail(HY_ERR_INVALID, "path %d", path);
    if (path == HY_PATH_MFMA && !hy::mfma_path_ok(c->cfg.wtype, c->H, c->I))
        return fail(HY_ERR_UNSUPPORTED, "the MFMA path needs Q8_0/Q4_0 weights and H, I multiples of 128");
    c->path = path;
    return HY_OK;
}

int hy_moe_prof_enable(hy_moe_ctx* c, int32_t on) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    HY_TRY(drain_prof(c));
    c->prof = on != 0;
    for (int i = 0; i < hy::KID_COUNT; i++) {
        c->prof_n[i] = 0;
        c->prof_ms[i] = 0.0;
    }
    return HY_OK;
}
int hy_moe_prof_read(hy_moe_ctx* c, int32_t kid, uint64_t* n, double* ms) {
    if (!c || kid < 0 || kid >= hy::KID_COUNT) return fail(HY_ERR_INVALID, "bad kernel id");
    HY_TRY(drain_prof(c));
    if (n) *n = c->prof_n[kid];
    if (ms) *ms = c->prof_ms[kid];
    return HY_OK;
}
const char* hy_moe_prof_name(int32_t kid) { return (kid >= 0 && kid < hy::KID_COUNT) ? kKernelNames[kid] : ""; }
int32_t hy_moe_prof_count(void) { return hy::KID_COUNT; }

int hy_moe_last_routing(hy_moe_ctx* c, uint32_t* distinct, int32_t* counts) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    HIP_TRY(hipStreamSynchronize(c->last_stream));
    int meta[4];
    HIP_TRY(hipMemcpy(meta, c->meta, sizeof(meta), hipMemcpyDeviceToHost));
    if (distinct) *distinct = (uint32_t)meta[2];
    if (counts) HIP_TRY(hipMemcpy(counts, c->cnt, (size_t)c->E * 4, hipMemcpyDeviceToHost));
    return HY_OK;
}

int hy_moe_last_gate(hy_moe_ctx* c, float* aux_loss, uint32_t* expert_capacity, float* exp_capacity_rate) {
    if (!c) return fail(HY_ERR_INVALID, "null ctx");
    HIP_TRY(hipStreamSynchronize(c->last_stream));
    // the routing pass stores its token count beside the tile counts, so a graph replay
    // reports its own batch
    int meta[4];
    HIP_TRY(hipMemcpy(meta, c->meta, sizeof(meta), hipMemcpyDeviceToHost));
    const uint32_t T = (uint32_t)meta[3];
    if (T == 0) return fail(HY_ERR_STATE, "no forward has run");
    std::vector<int32_t> cnt(c->E);
    HIP_TRY(hipMemcpy(cnt.data(), c->cnt, (size_t)c->E * 4, hipMemcpyDeviceToHost));
    float aux = 0.0f;
    if (c->cfg.compute_aux_loss) HIP_TRY(hipMemcpy(&aux, c->aux, 4, hipMemcpyDeviceToHost));
    // src/hunyuan_moe_full.cpp:209-227: the capacity rule, or the largest count
    uint32_t cap = 0;
    if (c->cfg.drop_tokens) {
        cap = drop_capacity(c->cfg, T);
    } else {
        for (int32_t n : cnt) cap = std::max(cap, (uint32_t)n);
        cap = std::max(cap, c->cfg.min_capacity);
    }
    // :329-335: pairs given a slot, counted in floats, over T * K
    float placed = 0.0f;
    for (int32_t n : cnt) placed += (float)std::min<uint32_t>((uint32_t)n, cap);
    if (aux_loss) *aux_loss = aux;
    if (expert_capacity) *expert_capacity = cap;
    if (exp_capacity_rate) *exp_capacity_rate = placed / (float)(T * (uint32_t)c->K);
    return HY_OK;
}

}  // extern "C"
