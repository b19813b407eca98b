/*
 * hy_oracle_attn.h -- CPU restatement of the HunyuanImage-3 attention half of a
 * decoder layer (GQA attention with QK-norm and 1D / 2D rotary embeddings).
 *
 * TEST INFRASTRUCTURE ONLY, like hy_oracle.h: the parity tests, the smoke check and
 * the benchmark's CPU-baseline leg call it to produce expected results; no product
 * code path links, loads or calls it.
 *
 * Every function follows the reference's scalar fp32 algorithm operation for
 * operation (sequential fp32 sums, no FMA contraction: built with
 * -ffp-contract=off), cited per function.  The GPU path computes the same
 * mathematics in fp32 with other summation orders (MFMA tiles, online softmax), so
 * parity with it is within a stated float tolerance, not bit for bit.
 *
 * Pins (tests/test_oracle_attn.py): torch's scaled_dot_product_attention and
 * matmul in float64 on the same inputs; closed forms (one token attends to itself
 * only; equal keys give the mean of the values; position 0 is the identity
 * rotation; rotations keep pair norms); the causal and GQA structure; the 2D table's
 * text / image position rules.
 */
#ifndef HY_ORACLE_ATTN_H
#define HY_ORACLE_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* rope_f32 (src/rms_norm.cpp:97-152): interleaved pairs (2d, 2d+1) of every head of
 * q [seq][n_heads][hd] and k [seq][n_kv][hd] rotated by pos * theta^(-2d/hd),
 * pos = positions[s] (or s when positions is NULL). */
void hyo_rope_f32(float* q, float* k, uint32_t seq, uint32_t n_heads, uint32_t n_kv, uint32_t hd, float theta,
                  const int32_t* positions);

/* build_2d_rope (src/hunyuan_image_gen.cpp:11-69): cos / sin tables [seq][n_elem]. */
void hyo_build_2d_rope(uint32_t seq, uint32_t n_elem, uint32_t text_len, uint32_t img_h, uint32_t img_w, float base,
                       float* cos_out, float* sin_out);

/* apply_rope_2d_f32 (src/hunyuan_image_gen.cpp:71-117): row t of the tables rotates
 * token t of q / k. */
void hyo_apply_rope_2d_f32(float* q, float* k, const float* cos_t, const float* sin_t, uint32_t n_tokens,
                           uint32_t n_heads, uint32_t n_kv, uint32_t hd);

/* attention_forward_cpu (src/attention.cpp:10-185): QKV projection, split, RoPE,
 * QK RMSNorm, causal GQA attention, merge, o_proj.  qkv_w [(nh+2nkv)*hd][H],
 * o_w [H][nh*hd], norms [hd].  dbg_q/k/v (nullable) receive q [T][nh][hd] and
 * k, v [T][nkv][hd] after RoPE and norm. */
void hyo_attention_forward(const float* x, const float* qkv_w, const float* o_w, const float* q_norm,
                           const float* k_norm, uint32_t T, uint32_t H, uint32_t nh, uint32_t nkv, uint32_t hd,
                           float eps, float theta, const int32_t* positions, float* out, float* dbg_q, float* dbg_k,
                           float* dbg_v);

/* The KV-cache branch of decoder_layer_extended_f32 (src/hunyuan_extended.cpp:52-176):
 * project the T new tokens, apply the 2D rotary tables when given (row t of
 * cos/sin for new token t; NULL: no rotation), QK RMSNorm, append k / v to the
 * cache at cur_len.., and let every new token attend to all cur_len + T cached
 * positions (no causal mask among the new tokens, as the reference).  Cache layout
 * [nkv][max_len][hd].  Returns -1 when the cache would overflow, else 0 (cur_len
 * advanced by T). */
typedef struct hyo_kv_cache {
    float* k;
    float* v;
    uint32_t max_len, cur_len;
} hyo_kv_cache;
int hyo_attention_cached(const float* x, const float* qkv_w, const float* o_w, const float* q_norm,
                         const float* k_norm, uint32_t T, uint32_t H, uint32_t nh, uint32_t nkv, uint32_t hd,
                         float eps, const float* cos_t, const float* sin_t, hyo_kv_cache* cache, float* out);

#ifdef __cplusplus
}
#endif
#endif
