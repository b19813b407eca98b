// hy_launch.hpp -- host-side launchers of the MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/hy_moe.h"
#include "hy_layout.hpp"

namespace hy {

// routing side (hy_route.hip)
hipError_t launch_router(const float* x, const float* wr, int T, int H, int E, int K, int norm, float scale,
                         float* logits, float* topw, int* topi, hipStream_t s);
hipError_t launch_router_q(const float* x, const float* wr, int T, int H, int E, int K, int norm, float scale,
                           float* logits, float* topw, int* topi, int8_t* xq, float* xd, int* xs, hipStream_t s,
                           bool logits_only = false);
hipError_t launch_topk_from_logits(const float* logits, int T, int E, int K, int norm, float scale, float* topw,
                                   int* topi, hipStream_t s);
hipError_t launch_softmax_rows(float* x, int rows, int n, hipStream_t s);
hipError_t launch_quant_q8_0(const float* x, size_t n, int8_t* q, float* d, int* qsum, uint8_t* blocks,
                             hipStream_t s);
hipError_t launch_route_decode(const float* x, const float* wr, int T, int H, int E, int K, int norm, float scale,
                               float* logits, float* topw, int* topi, int8_t* xq, float* xd, int* xs, int NT,
                               int has_shared, int* cnt, int* off, int* srt_tok, int* pair_pos, int* comb_pos,
                               float* comb_w, int* tile_e, int* tile_start, int* tile_n, int* meta, hipStream_t s);
// scratch: dispatch_scratch_bytes(T, K, E) of device memory (per-block counts)
size_t dispatch_scratch_bytes(int T, int K, int E);
hipError_t launch_dispatch(const int* topi, const float* topw, int T, int K, int E, int NT, int has_shared, int* cnt,
                           int* off, int* srt_tok, int* pair_pos, int* comb_pos, float* comb_w, int* tile_e,
                           int* tile_start, int* tile_n, int* meta, int* scratch, hipStream_t s);
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
hipError_t launch_gemv_down(int wtype, int n_tiles_bound, int mode, const MatView& W, const Routing& R,
                            const int8_t* hq, const float* hd, const int* hs, const float* hf, int T, int H, int I,
                            int E, int K, float* y, const float* resid, float* out, hipStream_t s);
hipError_t launch_combine(const Routing& R, const float* y, int T, int H, int K, int has_shared, const float* resid,
                          float* out, hipStream_t s);
hipError_t launch_block_dots_valu(int wtype, const uint8_t* w, const uint8_t* x, int rows, int nb, int* out,
                                  hipStream_t s);

// expert products, MFMA path (hy_mfma.hip)
bool mfma_path_ok(int wtype, int H, int I);
// tile shape of the MFMA path for this batch, and its pairs per tile (the dispatch
// must tile with it)
enum MfmaShape { MM_SHAPE_WIDE = 0, MM_SHAPE_TALL = 1 };
int mfma_shape(int T, int K, int E, int H, int I);
int mfma_shape_tokens(int shape);
hipError_t launch_ffn_up_mfma(int wtype, int shape, int n_tiles_bound, const MatView& W, const Routing& R,
                              const ActQ& X, int T, int H, int I, int E, int K, int8_t* hq, float* hd, int* hs,
                              hipStream_t s);
hipError_t launch_ffn_down_mfma(int wtype, int shape, int n_tiles_bound, const MatView& W, const Routing& R,
                                const int8_t* hq, const float* hd, int T, int H, int I, int E, int K, float* y,
                                hipStream_t s);

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
    KID_COUNT
};

}  // namespace hy
