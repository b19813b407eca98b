/*
 * hy_attn.h -- C ABI of the MI355X (gfx950) attention half of a HunyuanImage-3
 * decoder layer: GQA self-attention with QK RMSNorm and rotary embeddings, in fp32.
 *
 * Conventions as hy_moe.h: plain pointers and sizes, "dev" = device (HBM) address,
 * "host" = host memory, `stream` = hipStream_t as void* (NULL: default stream), every
 * function returns HY_OK or a negative hy_status with hy_last_error() set, and
 * nothing is written to caller-owned outputs on failure.
 *
 * The reference's interface for this path is attention_forward_cpu and its
 * AttentionWeights / HunyuanConfig (src/hunyuan_model.h:13-40, 93-101), the KV-cache branch of
 * decoder_layer_extended_f32 (src/hunyuan_extended.cpp:52-176), rope_f32
 * (src/rms_norm.cpp:97-152) and build_2d_rope / apply_rope_2d_f32
 * (src/hunyuan_image_gen.cpp:11-117).  One context holds num_layers layers' weights and
 * key / value caches, resident on the device, and one work arena shared by them.
 */
#ifndef HY_ATTN_H
#define HY_ATTN_H

#include <stdint.h>

#include "hy_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The attention fields of HunyuanConfig (src/hunyuan_model.h:13-40): hidden_size,
 * num_attention_heads, num_key_value_heads, attention_head_dim, rms_norm_eps,
 * rope_theta.  The GPU kernels take head_dim 64 or 128 and 4 query heads per kv
 * head (HunyuanImage-3: 32 / 8); other shapes are HY_ERR_UNSUPPORTED.
 * max_tokens bounds T per call; max_cache the key / value cache length per layer. */
typedef struct {
    uint32_t hidden;      /* H */
    uint32_t n_heads;     /* query heads */
    uint32_t n_kv_heads;  /* key / value heads */
    uint32_t head_dim;    /* 64 or 128 */
    uint32_t num_layers;  /* resident layers */
    uint32_t max_tokens;  /* 1..16384 */
    uint32_t max_cache;   /* cache positions per layer (0: no cache) */
    float rms_norm_eps;
    float rope_theta;
    int32_t device;
} hy_attn_config;

typedef struct hy_attn_ctx hy_attn_ctx;

int hy_attn_create(const hy_attn_config* cfg, hy_attn_ctx** out);
int hy_attn_destroy(hy_attn_ctx* ctx);

/* AttentionWeights (src/hunyuan_model.h:93-101) of one layer, F32, host memory,
 * reference layout: qkv_weight [(n_heads + 2 n_kv_heads) head_dim][hidden] (query head
 * rows, then key heads, then value heads), o_weight [hidden][n_heads head_dim],
 * q_norm_weight and k_norm_weight [head_dim].  Uploaded once. */
int hy_attn_upload(hy_attn_ctx* ctx, uint32_t layer, const float* qkv_weight_host, const float* o_weight_host,
                   const float* q_norm_host, const float* k_norm_host);

/* The attention tensors of block `block` of a GGUF file into layer `layer`, as
 * load_layer_weights reads them (src/hunyuan_gguf_loader.cpp:249-257):
 * blk.N.attn_qkv.weight ne {H, (nh+2nkv) hd}, blk.N.attn_output.weight ne {nh hd, H},
 * blk.N.attn_q_norm.weight / attn_k_norm.weight ne {hd}, and blk.N.attn_norm.weight
 * ne {H} (input_layernorm; optional, absent: unit).  F32, F16, BF16, Q8_0 or Q4_0 (converted to
 * F32 on upload).  Types and shapes are checked before anything is uploaded. */
int hy_attn_upload_gguf(hy_attn_ctx* ctx, uint32_t layer, const hy_gguf* f, uint32_t block);

/* One layer's weights from the counter-based synthetic generator (projections
 * ~ N(0, std), norms 1), on the device. */
int hy_attn_synth_layer(hy_attn_ctx* ctx, uint32_t layer, uint64_t seed, float std);

/* attention_forward_cpu (src/attention.cpp:10-185): out = o_proj(causal GQA
 * attention of RMSNorm(RoPE(q)), RMSNorm(RoPE(k)), v) for T tokens of x [T][hidden].
 * positions_dev: int32 [T] rotary positions (NULL: 0..T-1).  debug_q_dev
 * [T][n_heads][head_dim], debug_k_dev / debug_v_dev [T][n_kv_heads][head_dim]
 * (each may be NULL) receive q, k, v after RoPE and norm, as the reference's debug
 * outputs.  Does not touch the cache. */
int hy_attn_forward(hy_attn_ctx* ctx, uint32_t layer, const float* x_dev, uint32_t T, const int32_t* positions_dev,
                    float* out_dev, float* debug_q_dev, float* debug_k_dev, float* debug_v_dev, void* stream);

/* The KV-cache branch of decoder_layer_extended_f32 (src/hunyuan_extended.cpp:52-176):
 * project the T new tokens, rotate them by rows 0..T-1 of the 2D tables cos_dev /
 * sin_dev [T][head_dim] (both NULL: no rotation, as use_2d_rope = false), QK RMSNorm,
 * append k / v at the cache's current length, and let every new token attend to
 * all cached positions (no mask among the new tokens, as the reference).
 * HY_ERR_INVALID when the cache would overflow (the cache is left unchanged). */
int hy_attn_forward_cached(hy_attn_ctx* ctx, uint32_t layer, const float* x_dev, uint32_t T, const float* cos_dev,
                           const float* sin_dev, float* out_dev, void* stream);
/* KVCache::reset (every layer) / current_len (one layer) (src/hunyuan_image_gen.h:179-193). */
int hy_attn_cache_reset(hy_attn_ctx* ctx);
int hy_attn_cache_len(const hy_attn_ctx* ctx, uint32_t layer, uint32_t* len);

/* build_2d_rope (src/hunyuan_image_gen.cpp:11-69) on the device: cos_dev / sin_dev
 * [seq][n_elem] for text_len text positions followed by an img_h x img_w grid. */
int hy_build_2d_rope(uint32_t seq, uint32_t n_elem, uint32_t text_len, uint32_t img_h, uint32_t img_w, float base,
                     float* cos_dev, float* sin_dev, void* stream);

/* decoder_layer_forward_cpu (src/decoder_layer.cpp:9-48) on the device, the attention
 * context supplying input_layernorm + self-attention and the MoE context the
 * post-attention half:
 *   h   = x + attention(RMSNorm(x) * w_in)            (residual 1, in the o_proj)
 *   out = h + MoE_layer(RMSNorm(h) * w_post)           (hy_moe_stack_forward, 1 layer)
 * w_in: hy_attn_set_input_norm (input_layernorm, GGUF blk.N.attn_norm.weight; NULL:
 * unit); w_post: the MoE layer's hy_moe_set_ffn_norm.  The contexts must share
 * hidden size and device; eps is this context's rms_norm_eps.  debug_h_dev
 * (nullable) receives h [T][hidden]. */
int hy_attn_set_input_norm(hy_attn_ctx* ctx, uint32_t layer, const float* w_host);
int hy_decoder_layer_forward(hy_attn_ctx* attn, uint32_t attn_layer, hy_moe_ctx* moe, uint32_t moe_layer,
                             const float* x_dev, uint32_t T, const int32_t* positions_dev, float* out_dev,
                             float* debug_h_dev, void* stream);

/* ---- the resident backbone ---------------------------------------------------
 * HunyuanFullModel (src/hunyuan_full_model.h, .cpp:173-318): embedding lookup ->
 * num_layers decoder layers -> final RMSNorm -> lm_head, every weight resident (the
 * reference loads and frees each layer per forward).  The model owns an attention
 * context and a MoE context of num_layers layers each; their layers are uploaded
 * through hy_attn_* / hy_moe_* on the handles hy_model_attn / hy_model_moe give. */
typedef struct {
    hy_moe_config moe;    /* num_layers, max_tokens and device must match attn's */
    hy_attn_config attn;
    uint32_t vocab;       /* vocab_size */
} hy_model_config;

typedef struct hy_model_ctx hy_model_ctx;

int hy_model_create(const hy_model_config* cfg, hy_model_ctx** out);
int hy_model_destroy(hy_model_ctx* ctx);
hy_attn_ctx* hy_model_attn(hy_model_ctx* ctx);
hy_moe_ctx* hy_model_moe(hy_model_ctx* ctx);
/* Global weights, F32 host arrays: token_embd.weight [vocab][hidden],
 * output_norm.weight [hidden], output.weight (lm_head) [vocab][hidden]; any may be
 * NULL to leave it as it is. */
int hy_model_upload_globals(hy_model_ctx* ctx, const float* embedding_host, const float* final_norm_host,
                            const float* lm_head_host);
/* The same three tensors from a GGUF file (F32, F16, BF16, Q8_0 or Q4_0; converted to F32). */
int hy_model_upload_globals_gguf(hy_model_ctx* ctx, const hy_gguf* f);
/* Synthetic global weights (embedding and lm_head ~ N(0, std), final norm 1). */
int hy_model_synth_globals(hy_model_ctx* ctx, uint64_t seed, float std);
/* HunyuanFullModel::forward (src/hunyuan_full_model.cpp:173-216): input_ids_dev int32
 * [T] (ids >= vocab give zero rows), positions_dev int32 [T] or NULL (0..T-1),
 * logits_dev f32 [T][vocab]. */
int hy_model_forward(hy_model_ctx* ctx, const int32_t* input_ids_dev, uint32_t T, const int32_t* positions_dev,
                     float* logits_dev, void* stream);
/* HunyuanFullModel::forward_hidden / forward_debug (src/hunyuan_full_model.cpp:218-269):
 * inputs_embeds_dev [T][hidden] through layers 0..n_layers-1 (n_layers 0: all) into
 * hidden_dev [T][hidden]. */
int hy_model_forward_hidden(hy_model_ctx* ctx, const float* inputs_embeds_dev, uint32_t T,
                            const int32_t* positions_dev, uint32_t n_layers, float* hidden_dev, void* stream);

/* lm_head_f32 (src/hunyuan_full_model.cpp:298-318) and the projections' GEMM:
 * out[t][v] = sum_h x[t][h] * w[v][h] (+ resid[t][v] when resid_dev is not NULL),
 * fp32 MFMA; x [T][hidden], w [vocab][hidden], all device memory; hidden a multiple
 * of 16.  Mid-size shapes split the reduction over a per-device scratch that the
 * library allocates on first use and orders between calls with an event: those shapes
 * return HY_ERR_UNSUPPORTED under stream capture (hy_model_forward, whose context
 * owns its scratch, can be captured). */
int hy_lm_head_f32(const float* x_dev, const float* w_dev, const float* resid_dev, uint32_t T, uint32_t hidden,
                   uint32_t vocab, float* out_dev, void* stream);

/* rope_f32 (src/rms_norm.cpp:97-152) in place on x_dev [T][heads][head_dim]
 * (positions_dev int32 [T] or NULL: 0..T-1), and apply_rope_2d_f32
 * (src/hunyuan_image_gen.cpp:71-117) with tables [T][head_dim]; the reference rotates
 * q and k in one call, here each is one call. */
int hy_rope_f32(float* x_dev, uint32_t T, uint32_t heads, uint32_t head_dim, float theta,
                const int32_t* positions_dev, void* stream);
int hy_rope_2d_f32(float* x_dev, uint32_t T, uint32_t heads, uint32_t head_dim, const float* cos_dev,
                   const float* sin_dev, void* stream);
/* embedding_lookup_f32 (src/hunyuan_full_model.cpp:276-290): out[t] = table[ids[t]];
 * ids outside 0..vocab-1 give zero rows. */
int hy_embedding_lookup_f32(const int32_t* ids_dev, const float* table_dev, uint32_t T, uint32_t hidden,
                            uint32_t vocab, float* out_dev, void* stream);

/* Decode (T <= 8 new tokens): the attention spreads the cached keys over up to
 * max_waves waves, each taking whole 32-key blocks of one kv head, and joins the waves'
 * partial results afterwards.  0 (the default) = half as many waves as the GPU
 * keeps resident (up to the resident count may be asked for); a smaller cap gives
 * each wave more blocks.  No counterpart in the
 * reference (its CPU attention loops over the cache); a tuning and testing knob. */
int hy_attn_set_decode_waves(hy_attn_ctx* ctx, uint32_t max_waves);

/* Per-kernel timing of this context's launches (as hy_moe_prof_*): kernel ids
 * 0 = qkv_proj, 1 = rope_qknorm, 2 = attention, 3 = o_proj. */
int hy_attn_prof_enable(hy_attn_ctx* ctx, int32_t on);
int hy_attn_prof_read(hy_attn_ctx* ctx, uint32_t kid, uint64_t* launches, double* total_ms);

#ifdef __cplusplus
}
#endif
#endif
