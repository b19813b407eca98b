// hy_launch.hpp -- host-side launchers of the MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/hy_moe.h"
#include "hy_layout.hpp"

namespace hy {

// routing side (hy_route.hip)
// Routing options of topkgating_full beyond the default (zero: off): group-limited
// greedy when n_group > 0 and topk_group > 0; probs [T][E] (may be null) receives the
// gates (after the group mask) that the aux loss averages.
struct RouteOpts {
    int n_group = 0, topk_group = 0;
    float* probs = nullptr;
};
hipError_t launch_router(const float* x, const float* wr, int T, int H, int E, int K, int norm, float scale,
                         float* logits, float* topw, int* topi, hipStream_t s);
hipError_t launch_router_q(const float* x, const float* wr, int T, int H, int E, int K, int norm, float scale,
                           float* logits, float* topw, int* topi, int8_t* xq, float* xd, int* xs, hipStream_t s,
                           bool logits_only = false, RouteOpts opt = {});
hipError_t launch_topk_from_logits(const float* logits, int T, int E, int K, int norm, float scale, float* topw,
                                   int* topi, hipStream_t s, RouteOpts opt = {});
// aux loss from the gates [T][E] and the per-expert pair counts [E]: one float at out
hipError_t launch_aux_loss(const float* probs, const int* cnt, int T, int E, float* out, hipStream_t s);
hipError_t launch_softmax_rows(float* x, int rows, int n, hipStream_t s);
hipError_t launch_quant_q8_0(const float* x, size_t n, int8_t* q, float* d, int* qsum, uint8_t* blocks,
                             hipStream_t s);
hipError_t launch_route_decode(const float* x, const float* wr, int T, int H, int E, int K, int norm, float scale,
                               float* logits, float* topw, int* topi, int8_t* xq, float* xd, int* xs, int NT,
                               int has_shared, int* cnt, int* off, int* srt_tok, int* pair_pos, int* comb_pos,
                               float* comb_w, int* tile_e, int* tile_start, int* tile_n, int* meta, hipStream_t s);
// one-token batches whose routing runs inside the gate/up GEMV: the router logits
// [E] and, when xq is not null, the Q8_0 form of x, in one launch
hipError_t launch_decode_logits(const float* x, const float* wr, int H, int E, float* logits, int8_t* xq, float* xd,
                                int* xs, hipStream_t s);
// scratch: dispatch_scratch_bytes(T, K, E) of device memory (per-block counts)
size_t dispatch_scratch_bytes(int T, int K, int E);
hipError_t launch_dispatch(const int* topi, const float* topw, int T, int K, int E, int NT, int has_shared, int* cnt,
                           int* off, int* srt_tok, int* pair_pos, int* comb_pos, float* comb_w, int* tile_e,
                           int* tile_start, int* tile_n, int* meta, int* scratch, hipStream_t s,
                           int cap = 0x7fffffff);  // pairs at capacity slot >= cap: dropped
hipError_t launch_rms_norm(const float* x, int T, int H, float eps, float* out, hipStream_t s);
// RMSNorm (w may be null: unit weight) fused with the Q8_0 quantization of its output
hipError_t launch_rms_norm_quant(const float* x, const float* w, int T, int H, float eps, float* xn, int8_t* q,
                                 float* d, int* qsum, hipStream_t s);

// expert products, decode GEMV path (hy_gemv.hip)
constexpr int GEMV_NT = 4;  // tokens per GEMV tile
int gemv_tile_tokens();
hipError_t launch_gemv_up(int wtype, int max_tiles, const MatView& W, const Routing& R, const ActQ& X, const float* xf,
                          int T, int H, int I, int E, int K, int8_t* hq, float* hd, int* hs, float* hf,
                          hipStream_t s);
// Routing products a one-token gate/up GEMV writes (launch_gemv_up_route1): the
// top-k of logits[E] and every dispatch list launch_route_decode writes for T = 1.
struct Route1Out {
    const float* logits;
    int norm;
    float scale;
    int has_shared;
    float* topw;
    int* topi;
    int* cnt;
    int* off;
    int* srt_tok;
    int* pair_pos;
    int* comb_pos;
    float* comb_w;
    int* tile_e;
    int* tile_start;
    int* tile_n;
    int* meta;
};
// the gate/up GEMV of a one-token batch (T = 1, Q8_0 / Q4_0 ring kernel) with the
// routing done by its own waves from r.logits: K routed tiles (ascending expert) and
// the shared tile; false from gemv_route1_ok when the ring kernel does not take H
bool gemv_route1_ok(int wtype, int H);
hipError_t launch_gemv_up_route1(int wtype, const MatView& W, const Route1Out& r, const ActQ& X, int H, int I, int E,
                                 int K, int8_t* hq, float* hd, int* hs, hipStream_t s);
hipError_t launch_gemv_down(int wtype, int n_tiles_bound, const MatView& W, const Routing& R, const int8_t* hq,
                            const float* hd, const int* hs, const float* hf, int T, int H, int I, int E, int K,
                            float* y, hipStream_t s);
hipError_t launch_combine(const Routing& R, const float* y, int T, int H, int K, int has_shared, const float* resid,
                          float* out, hipStream_t s);
hipError_t launch_block_dots_valu(int wtype, const uint8_t* w, const uint8_t* x, int rows, int nb, int* out,
                                  hipStream_t s);
// the same dots through the grouped GEMM's LDS operand layout and block-dot MFMAs
hipError_t launch_block_dots_mfma(int wtype, const uint8_t* w, const uint8_t* x, int rows, int nb, int* out,
                                  hipStream_t s);

// expert products, MFMA path (hy_mfma.hip)
bool mfma_path_ok(int wtype, int H, int I);
// tile shape of the MFMA path for this batch, and its pairs per tile (the dispatch
// must tile with it)
enum MfmaShape { MM_SHAPE_WIDE = 0, MM_SHAPE_TALL = 1 };
int mfma_shape(int T, int K, int E, int H, int I);
int mfma_shape_tokens(int shape);
// the grouped GEMM's work counters (ints of device memory a caller keeps per context);
// launch_gather_act zeroes them for the gate/up and down launches that follow it
int mfma_counter_ints();
// the gate/up products' activations in expert-sorted slot order, block-major
// ([H/32][T*K+T][32 B] and [H/32][T*K+T] scales), from x's Q8_0 rows and the sorted pairs
hipError_t launch_gather_act(const ActQ& X, const Routing& R, int T, int K, int H, int8_t* gq, float* gd,
                             int* mm_ctr, hipStream_t s);
hipError_t launch_ffn_up_mfma(int wtype, int shape, int n_tiles_bound, const MatView& W, const Routing& R,
                              const ActQ& X, int T, int H, int I, int E, int K, int8_t* hq, float* hd, int* hs,
                              int* mm_ctr, hipStream_t s);
hipError_t launch_ffn_down_mfma(int wtype, int shape, int n_tiles_bound, const MatView& W, const Routing& R,
                                const int8_t* hq, const float* hd, int T, int H, int I, int E, int K, float* y,
                                int* mm_ctr, hipStream_t s);

// residency (hy_data.hip)
hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t s);
hipError_t launch_synth_matrix(int wtype, uint64_t key, float scale, int rows, int cols, int gu_I, uint8_t* qs,
                               uint16_t* sc, hipStream_t s);
hipError_t launch_synth_fill(float* out, size_t n, uint64_t key, float scale, hipStream_t s);
hipError_t launch_repack(int wtype, const uint8_t* src, int rows, int cols, int gu_I, uint8_t* qs, uint16_t* sc,
                         hipStream_t s);
hipError_t launch_dequant(int wtype, const uint8_t* src, size_t n, float* out, hipStream_t s);

// dense routing helpers of the reference API (hy_gate.hip)
hipError_t launch_topk_rows(const float* x, int rows, int n, int k, float* vals, int* idx, hipStream_t s);
hipError_t launch_einsum_dispatch(const float* x, int T, int H, const uint8_t* mask, int E, int C, float* out,
                                  hipStream_t s);
hipError_t launch_einsum_combine(const float* cw, const float* eo, int T, int H, int E, int C, float* out,
                                 hipStream_t s);
hipError_t launch_rms_norm_w(const float* x, const float* w, int T, int H, float eps, float* out, hipStream_t s);

// kernel ids for per-kernel timing
enum KernelId {
    KID_QUANT = 0,
    KID_ROUTER,
    KID_DISPATCH,
    KID_UP,
    KID_DOWN,
    KID_COMBINE,
    KID_RMSNORM,
    KID_AUX,
    KID_COUNT
};

// attention half of the decoder layer (hy_attn.hip)
enum { ROPE_NONE = 0, ROPE_1D = 1, ROPE_TABLE = 2 };
struct RopeNormArgs {
    const float* qkv;         // [T][nqkv] projection output
    int T, nh, nkv, hd, nqkv;
    int mode;                 // ROPE_NONE / ROPE_1D (positions or 0..T-1) / ROPE_TABLE (cos_t, sin_t rows)
    const int* positions;
    float theta;
    const float* cos_t;
    const float* sin_t;
    const float* q_norm;
    const float* k_norm;
    float eps;
    int norm_assoc;           // 0: (x * rms) * w, 1: x * (rms * w)
    float* q;                 // [T][nh][hd]
    float* k;                 // [nkv][L][hd], rows pos0 + t
    float* v;
    int L, pos0;
};
struct FlashArgs {
    const float* q;           // [T][nh][hd]
    const float* k;           // [nkv][L][hd]
    const float* v;
    float* out;               // [T][nh][hd]
    int T, nh, nkv, hd, L;
    int kv_len;               // keys 0..kv_len-1 exist
    int q_pos0;               // key index of query 0 (causal bound: key <= q_pos0 + t)
    int causal;
    float scale;
    // split over the keys (set by launch_flash_attn): chunks of cb key blocks, at most
    // nch per query tile, partial results in part (flash_attn_ws_floats)
    float* part = nullptr;
    int cb = 0, nch = 1;
};
// scratch of the split attention: partial tiles (at most FA_SPLIT_SLOTS) for head_dim
// hd; flash_attn_ws_slots: the slots a context of max_tokens queries and max_keys
// keys can use
constexpr int FA_SPLIT_SLOTS = 4096;
int flash_attn_ws_slots(int max_tokens, int max_keys, int nkv);
size_t flash_attn_ws_floats(int hd, int slots);
// C = A . W^T, plus R elementwise when R is not null (R may alias nothing written here).
// ws: gemm_nt_f32_ws_bytes() of device scratch for the stream-K split of mid-size grids
// (gemm_nt_f32_uses_ws); without it those grids run one tile per work group.
constexpr int GEMM_SK_GROUPS = 512;  // stream-K work groups: two per CU
size_t gemm_nt_f32_ws_bytes();
bool gemm_nt_f32_uses_ws(int M, int N, int K);
hipError_t launch_gemm_nt_f32(const float* A, const float* W, const float* R, float* C, int M, int N, int K,
                              hipStream_t s, float* ws = nullptr);
hipError_t launch_rope_qknorm(const RopeNormArgs& a, hipStream_t s);
// ws: flash_attn_ws_floats(hd, ws_slots) of device scratch, or nullptr (no split over
// the keys)
// T <= 8 (decode) with ws: the row-packed decode kernel on at most max_waves waves
// (0: as many as the chip holds)
hipError_t launch_flash_attn(const FlashArgs& a, hipStream_t s, float* ws = nullptr, int ws_slots = 0,
                             int max_waves = 0);
hipError_t launch_rope2d_table(int seq, int n_elem, int text_len, int img_h, int img_w, float base, float* cos_out,
                               float* sin_out, hipStream_t s);
hipError_t launch_gather_kv(const float* src, int nkv, int L, int pos0, int T, int hd, float* dst, hipStream_t s);
hipError_t launch_embed(const int* ids, const float* table, int T, int H, int vocab, float* out, hipStream_t s);
hipError_t launch_fill_f32(float* out, size_t n, float v, hipStream_t s);
hipError_t launch_rope_apply(float* x, int T, int heads, int hd, int mode, const int* positions, float theta,
                             const float* cos_t, const float* sin_t, hipStream_t s);

}  // namespace hy
