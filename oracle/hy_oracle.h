/*
 * hy_oracle.h -- CPU restatement of the HunyuanImage-3 MoE feed-forward block.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: the parity tests,
 * the smoke check and the CPU-baseline leg of the benchmark call it to produce
 * expected results.  No product code path links, loads or calls it; the GPU
 * library fails loudly instead of falling back to anything in here.
 *
 * Two families of functions live here:
 *
 *  (a) "ref" semantics -- the reference's scalar fp32 algorithm, operation for
 *      operation (single sequential fp32 accumulator, expf, insertion top-k,
 *      silu(first half) * second half, shared + routed).  Compiled with
 *      -ffp-contract=off so no FMA contraction sneaks in.  Cited per function.
 *
 *  (b) "q" semantics -- what the GPU path computes: the router logits use a
 *      fixed 64-lane blocked fmaf order shared bit-for-bit with the GPU kernel,
 *      experts are selected on logits (lower index wins ties), activations are
 *      quantized to GGUF Q8_0 (ggml's scalar quantize_row_q8_0 definition),
 *      expert products are exact int32 per-32-block dots rescaled in fp32
 *      (ggml's vec_dot_q8_0_q8_0 / vec_dot_q4_0_q8_0 definition).
 *
 * The q semantics fix every float operation and its order (router: 64-lane blocked
 * fmaf; softmax denominator: 64-lane tree; expert rows: block-sequential
 * fmaf((float)s_b, d_w*d_x, acc); exp: hyo_expf; combine: fmaf in ascending expert
 * order), so the GPU path reproduces them bit for bit.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   - ref-semantics routing/dispatch/combine/moe_forward_full: bit-exact
 *     against the reference's own hunyuan_moe_full.cpp compiled into
 *     oracle/_ref, and against committed fixtures made from it;
 *   - swiglu / rms_norm / moe_forward_cpu twin: closed forms, the reference's
 *     inline expert FFN (hunyuan_moe_full.cpp:470-496 via moe_forward_full),
 *     brute-force float64;
 *   - fp16 conversion: exhaustive against numpy float16;
 *   - block codecs and int dots: byte tables, round trips, brute force int64,
 *     known answers (all-127 x all-127 block = 516128);
 *   - q-semantics MoE: float64 brute force on dequantized values.
 */
#ifndef HY_ORACLE_H
#define HY_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml_type values for the weight formats this path handles. */
enum { HYO_F32 = 0, HYO_F16 = 1, HYO_Q4_0 = 2, HYO_Q8_0 = 8 };

#define HYO_QK 32
typedef struct { uint16_t d; int8_t  qs[HYO_QK]; }     hyo_block_q8_0; /* 34 B */
typedef struct { uint16_t d; uint8_t qs[HYO_QK / 2]; } hyo_block_q4_0; /* 18 B */

/* MoERoutingConfig, field for field (reference src/hunyuan_moe_full.h:25-47). */
typedef struct {
    uint32_t num_experts;
    uint32_t moe_topk;
    int32_t  group_limited_greedy;
    uint32_t n_group;
    uint32_t topk_group;
    int32_t  drop_tokens;
    int32_t  random_routing_dropped_token;
    float    capacity_factor;
    uint32_t min_capacity;
    int32_t  norm_topk_prob;
    float    routed_scaling_factor;
    int32_t  compute_aux_loss;
} hyo_routing_cfg;

void hyo_routing_cfg_default(hyo_routing_cfg* c);

/* ---------------- fp16 ---------------- */
float    hyo_fp16_to_fp32(uint16_t h);      /* IEEE binary16 -> binary32, exact */
uint16_t hyo_fp32_to_fp16(float f);         /* round to nearest even */
float    hyo_fp16_to_fp32_ref(uint16_t h);  /* reference decoder: subnormals -> +-0,
                                               no inf/nan (hunyuan_gguf_loader.cpp:19-32) */

/* ---------------- block codecs ---------------- */
size_t hyo_type_row_bytes(int type, size_t n);            /* bytes of one n-element row */
void hyo_quantize_row_q8_0(const float* x, void* y, size_t n);
void hyo_quantize_row_q4_0(const float* x, void* y, size_t n);
void hyo_dequantize_row_q8_0(const void* x, float* y, size_t n);
void hyo_dequantize_row_q4_0(const void* x, float* y, size_t n);     /* GGUF layout */
void hyo_dequantize_row_q8_0_ref(const void* x, float* y, size_t n); /* reference loader */
void hyo_dequantize_row_q4_0_ref(const void* x, float* y, size_t n); /* reference loader */
void hyo_dequantize_row(int type, const void* x, float* y, size_t n);

/* per-32-block exact int32 dots: out[b] = sum_j w_b[j] * x_b[j] */
void  hyo_block_dots_q8_0_q8_0(const void* w, const void* x, size_t n, int32_t* out);
void  hyo_block_dots_q4_0_q8_0(const void* w, const void* x, size_t n, int32_t* out);
float hyo_vec_dot_q8_0_q8_0(const void* w, const void* x, size_t n);
float hyo_vec_dot_q4_0_q8_0(const void* w, const void* x, size_t n);

/* ---------------- synthetic data (shared bit-for-bit with the GPU generator) ------- */
uint64_t hyo_stream_key(uint64_t seed, uint32_t layer, uint32_t tensor, uint32_t expert);
float    hyo_synth_normal(uint64_t key, uint64_t idx, float stddev);
void     hyo_synth_fill(uint64_t key, uint64_t idx0, size_t n, float stddev, float* out);

/* ---------------- (a) reference semantics ---------------- */
void hyo_rms_norm_f32(const float* x, const float* w, float* out, uint32_t T, uint32_t H, float eps);
void hyo_swiglu_ffn_f32(const float* x, const float* gu, const float* dn, float* out,
                        uint32_t n, uint32_t H, uint32_t I);
void hyo_softmax_f32(float* x, uint32_t n);
void hyo_topk_f32(const float* x, uint32_t n, uint32_t k, float* vals, int32_t* idx);
void hyo_topkgating_easy(const float* logits, uint32_t T, uint32_t E, uint32_t K,
                         float* w, int32_t* idx);
/* topkgating_full: capacity C is chosen by the function (as the reference does) and
 * the [T,E,C] arrays are allocated inside; free with hyo_free. */
typedef struct {
    uint32_t capacity;
    float    aux_loss;
    float    exp_capacity_rate;
    uint8_t* dispatch_mask;   /* [T,E,C] */
    float*   combine_weights; /* [T,E,C] */
    int32_t* exp_counts;      /* [E] */
    float*   router_probs;    /* [T,E] */
} hyo_gate_full;
int  hyo_topkgating_full(const float* logits, uint32_t T, const hyo_routing_cfg* cfg, hyo_gate_full* out);
void hyo_gate_full_free(hyo_gate_full* g);
void hyo_einsum_dispatch(const float* x, uint32_t T, uint32_t H, const uint8_t* mask,
                         uint32_t E, uint32_t C, float* disp);
void hyo_einsum_combine(const float* cw, const float* eo, uint32_t T, uint32_t H,
                        uint32_t E, uint32_t C, float* out);
void hyo_router_logits_seq(const float* x, const float* wr, uint32_t T, uint32_t H, uint32_t E,
                           float* logits);
int  hyo_moe_forward_full(const float* x, uint32_t T, uint32_t H, const float* wr,
                          const float* shared_gu, const float* shared_dn,
                          const float* gu_stacked, const float* dn_stacked,
                          uint32_t E, uint32_t I, const hyo_routing_cfg* cfg, float* out);
int  hyo_moe_forward_cpu(const float* x, const float* wr,
                         const float* shared_gu, const float* shared_dn,
                         const float* gu_stacked, const float* dn_stacked,
                         uint32_t T, uint32_t H, uint32_t E, uint32_t I, uint32_t K,
                         float* out, float* dbg_probs, float* dbg_w, int32_t* dbg_idx);

/* ---------------- (b) q semantics (the GPU path's definition) ---------------- */
/* exp used by the q semantics: Cody-Waite reduction + degree-7 Taylor (fmaf Horner)
 * + ldexpf, evaluated identically by the GPU kernels. */
float hyo_expf(float x);
/* Router logit order: lane l in [0,64) owns elements h with (h/4) % 64 == l and
 * accumulates them in increasing h with fmaf from 0; the 64 lane partials are
 * then folded p[l] += p[l+s] for s = 32,16,8,4,2,1; logit = p[0]. */
void hyo_router_logits_blocked(const float* x, const float* wr, uint32_t T, uint32_t H,
                               uint32_t E, float* logits);
/* top-K on logits, descending, equal logits keep the lower expert index; weights are
 * softmax(logits) at the selected experts renormalised by max(sum, 1e-8), else
 * multiplied by scale.  norm 1 renormalises only when K > 1 (topkgating_full,
 * src/hunyuan_moe_full.cpp:230), norm 2 at every K (moe_forward_cpu,
 * src/attention.cpp:268-275), norm 0 never. */
/* q-semantics top-k selection (NaN ranks below every number, NaNs in index order;
 * topk_f32 for rows without NaN), n <= 64 */
void hyo_select_q(const float* x, uint32_t n, uint32_t k, float* vals, int32_t* idx);
void hyo_route_topk(const float* logits, uint32_t T, uint32_t E, uint32_t K, int norm,
                    float scale, float* w, int32_t* idx);
/* The same with group-limited greedy (src/hunyuan_moe_full.cpp:135-166) when n_group > 0
 * and topk_group > 0 (topk_group <= 64; n_group > E puts no expert in a group): on the q probabilities p_e = hyo_expf(l_e - m) / s
 * (s the 64-lane tree sum), group scores max(0, max p over the group's E/n_group
 * experts), the topk_group best groups by hyo_topk_f32, experts of the other groups
 * set to 0, then top-K by hyo_topk_f32 on the probabilities (equal values: lower
 * index) and the weights from the (masked) probabilities.  probs (may be NULL)
 * receives the masked probabilities [T][E], the gates the aux loss averages. */
void hyo_route_topk_groups(const float* logits, uint32_t T, uint32_t E, uint32_t K, int norm, float scale,
                           uint32_t n_group, uint32_t topk_group, float* w, int32_t* idx, float* probs);
/* Load-balancing aux loss of src/hunyuan_moe_full.cpp:182-206 over the routing's
 * probabilities [T][E] and indices [T][K]: tokens per expert / T times the expert's
 * probability summed over tokens in order / T, summed over experts, times E*E. */
float hyo_aux_loss_q(const float* probs, const int32_t* idx, uint32_t T, uint32_t E, uint32_t K);
/* Expert capacity under token dropping (src/hunyuan_moe_full.cpp:210-214):
 * max(K, (uint32)(capacity_factor * K * T / E)), then at least min_capacity. */
uint32_t hyo_drop_capacity(uint32_t T, uint32_t E, uint32_t K, float capacity_factor, uint32_t min_capacity);
/* keep[t][k] = 1 when pair (t, k) takes a capacity slot < capacity: slots are given in
 * the order k = 0..K-1, t = 0..T-1 (src/hunyuan_moe_full.cpp:245-304). */
void hyo_capacity_keep(const int32_t* idx, uint32_t T, uint32_t E, uint32_t K, uint32_t capacity, uint8_t* keep);

/* One MoE layer over GGUF-layout weights of type wtype (F32, Q8_0 or Q4_0).
 * gu: [(E) experts][2I rows] rows of H elements; dn: [E][H rows] rows of I elements;
 * shared_gu/shared_dn: one expert (may be NULL).  Row = ggml row (ne0 = in). */
typedef struct {
    uint32_t H, I, E, K;
    int      wtype;
    int      norm_topk_prob;  /* 0, 1 or 2 as hyo_route_topk's norm */
    float    routed_scaling_factor;
    const float* router;      /* [E,H] f32 */
    const void*  shared_gu;
    const void*  shared_dn;
    const void*  gu;
    const void*  dn;
    /* routing options beyond the default, 0 = off */
    uint32_t n_group, topk_group; /* group-limited greedy when both > 0 (hyo_route_topk_groups) */
    uint32_t capacity;            /* token dropping: pairs past this capacity slot contribute nothing */
} hyo_qlayer;

int hyo_moe_forward_q(const hyo_qlayer* L, const float* x, uint32_t T, float* out,
                      float* dbg_logits, float* dbg_w, int32_t* dbg_idx, int nthreads);
/* Routing of the whole batch: logits [T][E] (may be NULL), weights and indices [T][K],
 * masked probabilities [T][E] (may be NULL) and keep [T][K] (may be NULL; all 1 without
 * a capacity). */
int hyo_moe_route_q(const hyo_qlayer* L, const float* x, uint32_t T, float* logits, float* w, int32_t* idx,
                    float* probs, uint8_t* keep, int nthreads);
/* Sampled tokens of the layer (rows are independent without a capacity; with one, the
 * whole batch is routed first). */
int hyo_moe_forward_q_rows(const hyo_qlayer* L, const float* x, uint32_t T,
                           const uint32_t* rows, uint32_t n_rows, float* out, int nthreads);
/* RMSNorm(eps, unit weight) -> MoE -> residual, over n_layers layers. */
int hyo_moe_stack_q(const hyo_qlayer* layers, uint32_t n_layers, const float* x, uint32_t T,
                    float eps, float* out, int nthreads);
/* The same with a post-attention RMSNorm weight per layer (norm_w or an entry NULL:
 * unit weight): h <- h + MoE(RMSNorm(h) * w_l), src/decoder_layer.cpp:33-42. */
int hyo_moe_stack_qw(const hyo_qlayer* layers, const float* const* norm_w, uint32_t n_layers, const float* x,
                     uint32_t T, float eps, float* out, int nthreads);
/* RMSNorm of T rows in the GPU kernels' blocked order (w NULL: unit weight). */
void hyo_rms_norm_blocked_rows(const float* x, const float* w, float* out, uint32_t T, uint32_t H, float eps);

void hyo_free(void* p);

#ifdef __cplusplus
}
#endif
#endif
