/*
 * hy_moe.h -- C ABI of the MI355X (gfx950) HunyuanImage-3 MoE feed-forward block.
 *
 * Plain pointers and sizes only.  "dev" pointers are device (HBM) addresses, "host"
 * pointers are ordinary host memory; `stream` is a hipStream_t passed as void*
 * (NULL = the default stream).  Every function returns HY_OK (0) or a negative
 * hy_status; hy_last_error() gives a message for the calling thread's last failure.
 * On failure nothing is written to caller-owned outputs.
 *
 * The reference's interface for this path is the C++ API of
 * src/hunyuan_moe_full.h:76-155 plus moe_forward_cpu / swiglu_ffn_f32 /
 * MoEWeights (src/hunyuan_model.h:118-156).  Each entry point below names the
 * reference function it replaces.  include/hunyuan_moe_full.h re-exposes the
 * reference's own names and signatures on top of this ABI.
 */
#ifndef HY_MOE_H
#define HY_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    HY_OK = 0,
    HY_ERR_INVALID = -1,     /* bad argument or shape */
    HY_ERR_UNSUPPORTED = -2, /* routing feature or weight type the GPU path does not run */
    HY_ERR_HIP = -3,         /* HIP runtime error */
    HY_ERR_NOMEM = -4,       /* device allocation failed */
    HY_ERR_STATE = -5        /* e.g. layer not loaded */
} hy_status;

/* ggml_type values accepted as weight formats (ggml.h numbering). */
enum { HY_TYPE_F32 = 0, HY_TYPE_Q4_0 = 2, HY_TYPE_Q8_0 = 8 };

/* Values of norm_topk_prob (config field and routing calls).
 *   HY_NORM_OFF    w_k = p_k * routed_scaling_factor
 *   HY_NORM_TOPK   w_k = p_k / max(sum_k p_k, 1e-8) when K > 1, else p * routed_scaling_factor:
 *                  topkgating_full, src/hunyuan_moe_full.cpp:230 (`norm_topk_prob && K > 1`),
 *                  the rule moe_forward_full routes with.  Any other nonzero value means this.
 *   HY_NORM_ALWAYS renormalise at every K: topkgating_easy (src/hunyuan_moe_full.cpp:104-108)
 *                  and moe_forward_cpu (src/attention.cpp:268-275); one expert gets weight 1. */
enum { HY_NORM_OFF = 0, HY_NORM_TOPK = 1, HY_NORM_ALWAYS = 2 };

/* Shapes and routing of one resident MoE stack.  The routing fields mirror
 * MoERoutingConfig (src/hunyuan_moe_full.h:25-47) and topkgating_full's use of them
 * (src/hunyuan_moe_full.cpp:117-335): softmax -> [group-limited greedy] -> top-k ->
 * renormalise or scale -> [capacity slots, token dropping]; [aux loss].
 * random_routing_dropped_token has no field: the reference declares it and never
 * reads it.  Batches that use group-limited greedy, dropping or the aux loss are routed
 * by the general path at every T (the one-launch decode routing covers the default). */
typedef struct {
    uint32_t hidden;        /* H, multiple of 32 */
    uint32_t intermediate;  /* I, multiple of 32 */
    uint32_t num_experts;   /* E, 1..64 */
    uint32_t topk;          /* K, 1..min(E, 64) (topk_f32's bound) */
    uint32_t num_layers;    /* resident layers */
    uint32_t max_tokens;    /* largest T per call, 1..16384; sizes the work arena */
    int32_t  wtype;         /* HY_TYPE_F32 / HY_TYPE_Q8_0 / HY_TYPE_Q4_0 */
    int32_t  has_shared;    /* 1: one shared expert (num_shared_expert = 1) */
    int32_t  norm_topk_prob;       /* HY_NORM_*: moe_forward_full routes with HY_NORM_TOPK */
    float    routed_scaling_factor;
    int32_t  group_limited_greedy; /* 1: group-limited greedy with n_group / topk_group below */
    int32_t  drop_tokens;          /* 1: capacity from capacity_factor / min_capacity, excess pairs dropped */
    int32_t  compute_aux_loss;     /* 1: the load-balancing aux loss (hy_moe_last_gate) */
    int32_t  device;               /* HIP device ordinal */
    /* appended after the fields above, which keep their offsets */
    uint32_t n_group;              /* groups of num_experts / n_group experts; 0: off */
    uint32_t topk_group;           /* groups kept per token (<= 64); 0: off */
    float    capacity_factor;      /* drop_tokens: capacity max(K, (uint32)(capacity_factor*K*T/E)) */
    uint32_t min_capacity;         /* lower bound of the capacity, with or without dropping */
} hy_moe_config;

typedef struct hy_moe_ctx hy_moe_ctx;

const char* hy_last_error(void);

/* ---- context and resident weights ---------------------------------------- */

/* Replaces the per-call weight handling of moe_forward_full
 * (src/hunyuan_moe_full.h:121-142) and the layer streaming of
 * HunyuanFullModel::forward (src/hunyuan_full_model.cpp:193-207): every layer's
 * router, shared expert and routed experts stay resident in HBM. */
int hy_moe_create(const hy_moe_config* cfg, hy_moe_ctx** out);
int hy_moe_destroy(hy_moe_ctx* ctx);
/* bytes of HBM the resident weights of one layer take */
size_t hy_moe_layer_bytes(const hy_moe_ctx* ctx);

/* Upload one layer from host memory in ggml layout (ne0 = in-features, GGUF
 * blocks of 32 along it).  Replaces StackedExpertWeights::build_from_experts
 * (src/hunyuan_extended.cpp:8-26) and the tensors load_layer_weights reads
 * (src/hunyuan_gguf_loader.cpp:229-280):
 *   router    f32 [E][H]                         (blk.N.ffn_gate.weight)
 *   shared_gu wtype rows [2I][H]                 (blk.N.ffn_shared_gate_up.weight)
 *   shared_dn wtype rows [H][I]                  (blk.N.ffn_shared_down.weight)
 *   gu        wtype rows [E][2I][H], expert-major (blk.N.ffn_expert_E_gate_up.weight)
 *   dn        wtype rows [E][H][I]               (blk.N.ffn_expert_E_down.weight)
 * Rows [0,I) of a gate_up matrix are the gate (SiLU) half, [I,2I) the up half, as
 * src/hunyuan_moe_full.cpp:482-485 reads them. */
int hy_moe_upload_layer(hy_moe_ctx* ctx, uint32_t layer, const float* router_host,
                        const void* shared_gu_host, const void* shared_dn_host,
                        const void* gu_host, const void* dn_host);

/* Generate one layer on the device from the counter-based synthetic generator
 * (weights ~ N(0,std) quantized to wtype; router ~ N(0,std), column 0 replaced
 * by router_bias_host[E] when given).  Same values as the oracle's synth_layer. */
int hy_moe_synth_layer(hy_moe_ctx* ctx, uint32_t layer, uint64_t seed, float std,
                       const float* router_bias_host);

/* The layer's post-attention RMSNorm weight [H] (post_attention_layernorm, GGUF
 * blk.N.ffn_norm.weight), applied by hy_moe_stack_forward before the layer's MoE:
 * DecoderLayerWeights::post_attn_ln_weight as decoder_layer_forward_cpu uses it
 * (src/decoder_layer.cpp:33-34, src/hunyuan_gguf_loader.cpp:251).  w_host NULL
 * returns the layer to unit weight (the default). */
int hy_moe_set_ffn_norm(hy_moe_ctx* ctx, uint32_t layer, const float* w_host);

/* ---- GGUF files ------------------------------------------------------------ */

/* A GGUF file (format versions 2 and 3), memory mapped read-only.  Replaces the
 * gguf_* use of HunyuanGGUFLoader::open_layer / load_tensor
 * (src/hunyuan_gguf_loader.cpp:84-190) for the MoE tensors; tensor data is handed
 * out as the file's bytes (no dequantization). */
typedef struct hy_gguf hy_gguf;
int hy_gguf_open(const char* path, hy_gguf** out);
int hy_gguf_close(hy_gguf* f);
int hy_gguf_n_tensors(const hy_gguf* f, uint64_t* n);
/* Tensor by name: ggml type, dims (ne[0] innermost, unused dims 1), byte size and a
 * host pointer into the mapping (nbytes 0 and data NULL for a type the reader does
 * not size).  Any output may be NULL. */
int hy_gguf_tensor(const hy_gguf* f, const char* name, int32_t* ggml_type, uint32_t* n_dims, uint64_t* ne4,
                   uint64_t* nbytes, const void** data);
/* A tensor's values as f32 (n = its element count), for F32, F16, BF16, Q8_0 and
 * Q4_0 (GGUF block layouts): read_tensor_data / load_tensor
 * (src/hunyuan_gguf_loader.cpp:160-222), which dequantizes whatever it reads.  Two
 * deliberate differences: fp16 subnormal scales are kept (the reference flushes them
 * to 0) and Q4_0 uses the GGUF nibble order (low nibble = element j, high = j+16). */
int hy_gguf_tensor_f32(const hy_gguf* f, const char* name, float* out_host, uint64_t n);
/* Metadata (HunyuanGGUFLoader::get_metadata_u32 / _f32, src/hunyuan_gguf_loader.cpp:286-297),
 * but a missing key or a value of another type is an error instead of a default. */
int hy_gguf_get_u32(const hy_gguf* f, const char* key, uint32_t* out);
int hy_gguf_get_f32(const hy_gguf* f, const char* key, float* out);

/* Upload layer `layer` of the context from block `block` of a GGUF file with the
 * tensor names the reference's converter writes and its loader reads
 * (scripts/convert_to_gguf.py:70-137, src/hunyuan_gguf_loader.cpp:229-280):
 *   blk.N.ffn_gate.weight                  any    ne {H, E}   (router)
 *   blk.N.ffn_shared_gate_up.weight        expert ne {H, 2I}
 *   blk.N.ffn_shared_down.weight           expert ne {I, H}
 *   blk.N.ffn_expert_<e>_gate_up.weight    expert ne {H, 2I}, e = 0..E-1
 *   blk.N.ffn_expert_<e>_down.weight       expert ne {I, H}
 *   blk.N.ffn_norm.weight                  any    ne {H}   (optional; absent: unit)
 * "any": F32, F16, BF16, Q8_0 or Q4_0, turned into f32 as hy_gguf_tensor_f32 does
 * (the reference loader reads every tensor through read_tensor_data,
 * src/hunyuan_gguf_loader.cpp:167-222, and its converter gives all tensors of a file
 * one type, scripts/convert_to_gguf.py:196-200).  "expert": the context's wtype, used
 * as stored; into an F32 context any type is turned into f32; Q4_0 into a Q8_0
 * context is re-encoded exactly (same scales, q = nibble - 8).  Other combinations
 * would change the weights and are HY_ERR_UNSUPPORTED.  Shapes must match the context
 * (else HY_ERR_INVALID naming the tensor); hunyuan.hidden_size /
 * moe_intermediate_size / num_experts / moe_topk, when present, must agree with it too.
 * Replaces load_layer_weights + StackedExpertWeights (src/hunyuan_extended.cpp:8-26):
 * the blocks are repacked on the device once. */
int hy_moe_upload_layer_gguf(hy_moe_ctx* ctx, uint32_t layer, const hy_gguf* f, uint32_t block);

/* ---- forward ------------------------------------------------------------- */

/* One MoE layer: out = shared(x) + sum_k w_k expert_k(x).
 * Replaces moe_forward_full (src/hunyuan_moe_full.h:121-142, .cpp:405-516) and its
 * twin moe_forward_cpu (src/hunyuan_model.h:147-156, src/attention.cpp:191-313).
 * x_dev, out_dev: f32 [T][H] device; 1 <= T <= max_tokens.  Stream-ordered. */
int hy_moe_forward(hy_moe_ctx* ctx, uint32_t layer, const float* x_dev, uint32_t T,
                   float* out_dev, void* stream);

/* Same, also copying the routing into caller device buffers (any may be NULL):
 * logits [T][E] f32, weights [T][K] f32, indices [T][K] i32 in rank order.
 * Mirrors moe_forward_cpu's debug_router_* outputs (src/attention.cpp:278-280). */
int hy_moe_forward_debug(hy_moe_ctx* ctx, uint32_t layer, const float* x_dev, uint32_t T,
                         float* out_dev, float* logits_dev, float* weights_dev,
                         int32_t* indices_dev, void* stream);

/* n_layers x [ h -> h + MoE(RMSNorm(h) * w) ] over resident layers
 * first..first+n_layers-1, w the layer's ffn_norm weight (hy_moe_set_ffn_norm; unit
 * by default).  The decoder-layer MoE half of decoder_layer_forward_cpu
 * (src/decoder_layer.cpp:33-42) with rms_norm_f32 (src/rms_norm.cpp:9-33), stacked.
 * For quantized weights the RMSNorm and the Q8_0 quantization of its output run as
 * one pass, and the residual add is part of the combine. */
int hy_moe_stack_forward(hy_moe_ctx* ctx, uint32_t first_layer, uint32_t n_layers,
                         const float* x_dev, uint32_t T, float eps, float* out_dev, void* stream);

/* Expert-product kernels the forward uses: AUTO (default) takes the int8-MFMA grouped
 * GEMM for T > 16 and the dequant-GEMV (VALU dot4) for decode batches; VALU / MFMA
 * force one (MFMA needs Q8_0/Q4_0 weights and H, I multiples of 128).  Both compute
 * the same float operations in the same order, so they agree bit for bit.  No
 * counterpart in the reference (which has one scalar path); kept so both paths stay
 * testable at any T. */
enum { HY_PATH_AUTO = 0, HY_PATH_VALU = 1, HY_PATH_MFMA = 2 };
int hy_moe_set_path(hy_moe_ctx* ctx, int32_t path);

/* ---- stateless kernels (component parity) ----------------------------------- */

/* Router: logits = x Wr^T (64-lane blocked fmaf order), top-k on logits with lower
 * index winning ties, weights = softmax at the selection renormalised (or scaled).
 * logits_dev [T][E] is required (it is the intermediate of the two passes).
 * Replaces the router GEMV of src/hunyuan_moe_full.cpp:414-423 plus
 * topkgating_easy (src/hunyuan_moe_full.h:83-89).  norm_topk_prob is a HY_NORM_* value
 * (topkgating_easy itself is HY_NORM_ALWAYS). */
int hy_router_topk(const float* x_dev, const float* wr_dev, uint32_t T, uint32_t H, uint32_t E,
                   uint32_t K, int32_t norm_topk_prob, float routed_scaling_factor,
                   float* logits_dev, float* weights_dev, int32_t* indices_dev, void* stream);

/* topkgating_easy (src/hunyuan_moe_full.h:83-89) from precomputed logits. */
int hy_topkgating_easy(const float* logits_dev, uint32_t T, uint32_t E, uint32_t K,
                       float* weights_dev, int32_t* indices_dev, void* stream);

/* Top-k selection and weights from precomputed logits with the routing options of
 * topkgating_full (src/hunyuan_moe_full.cpp:229-243): norm_topk_prob is a HY_NORM_*
 * value (HY_NORM_TOPK: renormalise when K > 1, else scale by routed_scaling_factor). */
int hy_route_logits(const float* logits_dev, uint32_t T, uint32_t E, uint32_t K, int32_t norm_topk_prob,
                    float routed_scaling_factor, float* weights_dev, int32_t* indices_dev, void* stream);

/* hy_route_logits with group-limited greedy (src/hunyuan_moe_full.cpp:135-166) when
 * n_group > 0 and topk_group > 0 (topk_group <= 64): per token, groups of E / n_group experts
 * score the largest probability in them, the topk_group best groups stay and the other
 * groups' experts get probability 0, then the top K of those probabilities (equal
 * values: lower index) with their probabilities as weights.  probs_dev [T][E] (may be
 * NULL) receives the probabilities after that mask, the gates the aux loss averages. */
int hy_route_logits_groups(const float* logits_dev, uint32_t T, uint32_t E, uint32_t K, int32_t norm_topk_prob,
                           float routed_scaling_factor, uint32_t n_group, uint32_t topk_group, float* weights_dev,
                           int32_t* indices_dev, float* probs_dev, void* stream);

/* Load-balancing aux loss of topkgating_full (src/hunyuan_moe_full.cpp:182-206) from the
 * gates probs_dev [T][E] and the pairs per expert counts_dev [E] (hy_dispatch_pairs):
 * sum over experts of (count / T) * (gate summed over tokens in order / T), times E^2.
 * One float at out_dev. */
int hy_aux_loss(const float* probs_dev, const int32_t* counts_dev, uint32_t T, uint32_t E, float* out_dev,
                void* stream);

/* softmax_f32 (src/hunyuan_moe_full.h:148) over each of `rows` rows of n (n <= 1024). */
int hy_softmax_rows(float* x_dev, uint32_t rows, uint32_t n, void* stream);

/* Activation quantizer: rows of n f32 -> GGUF Q8_0 blocks (34 B), ggml's scalar
 * quantize_row_q8_0 definition.  The same device code feeds the expert GEMMs. */
int hy_quantize_q8_0(const float* x_dev, uint32_t rows, uint32_t n, void* blocks_dev, void* stream);

/* GGUF dequantization (src/hunyuan_gguf_loader.cpp:10-72 block formats; Q4_0 in the
 * GGUF nibble order) of n elements of type `type` into f32. */
int hy_dequantize(int32_t type, const void* blocks_dev, size_t n, float* out_dev, void* stream);

/* Exact per-32-block int32 dots of weight blocks (Q8_0 or Q4_0 rows) with Q8_0
 * activation blocks, computed by the device dot routines the expert kernels use:
 * out[r][b] = sum_j w[r][b][j] * x[b][j].  `path` 0 = the decode GEMV's VALU dot4
 * routine; 1 = the grouped GEMM's operand path: the weight rows staged in its LDS layout
 * (Q4_0 through its stage unpack), the activation block in a swizzled B tile, and its
 * v_mfma_i32_32x32x32_i8 block-dot tiles.  rows <= 4096.  No counterpart in the
 * reference (ggml's vec_dot block sums, the per-block part of src/hunyuan_gguf_loader.cpp:
 * 10-72's formats). */
int hy_block_dots(int32_t wtype, const void* w_blocks_dev, const void* x_blocks_dev, uint32_t rows,
                  uint32_t n, int32_t path, int32_t* out_dev, void* stream);

/* RMSNorm over T rows of H: out = x * (1/sqrtf(ss/H + eps)) * w, ss in the router's
 * blocked order; w_dev may be NULL for unit weight.  rms_norm_f32
 * (src/rms_norm.cpp:9-33). */
int hy_rms_norm(const float* x_dev, uint32_t T, uint32_t H, float eps, float* out_dev, void* stream);
int hy_rms_norm_w(const float* x_dev, const float* w_dev, uint32_t T, uint32_t H, float eps,
                  float* out_dev, void* stream);

/* topk_f32 (src/hunyuan_moe_full.h:154-155, .cpp:56-82) over each of `rows` rows of n
 * values (n <= 4096, k <= 64): descending, equal values keep the lower index. */
int hy_topk_rows(const float* x_dev, uint32_t rows, uint32_t n, uint32_t k, float* vals_dev,
                 int32_t* idx_dev, void* stream);

/* Token -> expert dispatch of T*K routed pairs (indices_dev [T][K]): per-expert counts
 * [E], list offsets [E+1], and each pair's position in the expert-sorted order
 * (pos_dev [T][K]).  Inside an expert the order is the reference's capacity-slot
 * priority (flat slot k*T + t ascending, src/hunyuan_moe_full.cpp:245-304), so
 * pos - offsets[e] is the dispatch_mask slot c.  Indices must lie in [0, E) (as the
 * router produces them); a pair with an out-of-range index is left out. */
int hy_dispatch_pairs(const int32_t* indices_dev, const float* weights_dev, uint32_t T, uint32_t K,
                      uint32_t E, int32_t* counts_dev, int32_t* offsets_dev, int32_t* pos_dev,
                      void* stream);

/* hy_dispatch_pairs without any allocation: no counterpart in the reference; for
 * callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments and results; the
 * workspace is a fixed 4 MiB array in device memory that each GPU holds until the
 * process ends, enough for every call with T*K <= 262,144 pairs (larger needs are
 * rejected with HY_ERR_INVALID).  Stream-ordered: it returns without waiting, the
 * outputs are ready when the stream gets there.  All calls on one GPU share that
 * array, so calls that overlap on one GPU (different streams, or different threads
 * without ordering) race and must be ordered by the caller. */
int hy_dispatch_pairs_noalloc(const int32_t* indices_dev, const float* weights_dev, uint32_t T,
                              uint32_t K, uint32_t E, int32_t* counts_dev, int32_t* offsets_dev,
                              int32_t* pos_dev, void* stream);

/* einsum_dispatch (src/hunyuan_moe_full.h:95-102): out[e][c][:] = sum of x[t][:] over
 * t with mask[t][e][c] (mask: one byte per entry). */
int hy_einsum_dispatch(const float* x_dev, uint32_t T, uint32_t H, const uint8_t* mask_dev,
                       uint32_t E, uint32_t C, float* out_dev, void* stream);

/* einsum_combine (src/hunyuan_moe_full.h:108-115): out[t][:] = sum over (e, c) of
 * combine_weights[t][e][c] * expert_output[e][c][:], e and c ascending. */
int hy_einsum_combine(const float* cw_dev, const float* eo_dev, uint32_t T, uint32_t H, uint32_t E,
                      uint32_t C, float* out_dev, void* stream);

/* ---- device memory / streams / timing helpers ------------------------------ */
int hy_device_count(int* n);
int hy_set_device(int device);
int hy_malloc(void** p, size_t bytes);
int hy_free(void* p);
int hy_memcpy_h2d(void* dst_dev, const void* src_host, size_t bytes);
int hy_memcpy_d2h(void* dst_host, const void* src_dev, size_t bytes);
int hy_memset(void* dst_dev, int value, size_t bytes);
/* Device-to-device copy by a plain streaming kernel (16-byte loads and stores, no
 * copy engine).  Besides moving data it is the yardstick for the hardware byte
 * counters: a copy of n bytes reads n and writes n. */
int hy_copy_d2d(void* dst_dev, const void* src_dev, size_t bytes, void* stream);
int hy_device_synchronize(void);
int hy_stream_create(void** stream);
int hy_stream_destroy(void* stream);
int hy_stream_synchronize(void* stream);
int hy_event_create(void** ev);
int hy_event_destroy(void* ev);
int hy_event_record(void* ev, void* stream);
int hy_event_elapsed_ms(void* start, void* stop, float* ms);
/* Capture of stream work into a replayable graph: begin / end (instantiate) / launch /
 * destroy.  No counterpart in the reference (its layer runs on the CPU); for callers
 * that replay a fixed-shape step (decode) without per-kernel launch costs.
 * hy_moe_forward and hy_moe_stack_forward allocate nothing, read nothing back to the
 * host and record no memset, so they can be captured, with profiling off; a replay
 * equals the eager call bit for bit.  A replay reads the pointers and sizes of the
 * captured calls.  The stream must be a created stream (hy_stream_create), not the
 * null stream. */
int hy_graph_begin(void* stream);
int hy_graph_end(void* stream, void** graph_exec);
int hy_graph_launch(void* graph_exec, void* stream);
int hy_graph_destroy(void* graph_exec);
/* Fill f32 [n] with the synthetic N(0,std) stream (seed, layer, tensor, expert). */
int hy_synth_fill(float* dev, size_t n, uint64_t seed, uint32_t layer, uint32_t tensor,
                  uint32_t expert, float std, void* stream);

/* Per-kernel timing of the forward path, recorded with HIP events on the launch
 * stream.  While enabled, every kernel launch of hy_moe_forward* is bracketed by
 * events; hy_moe_prof_read returns, per kernel id, the launch count and total
 * milliseconds since the last reset.  Names via hy_moe_prof_name. */
int hy_moe_prof_enable(hy_moe_ctx* ctx, int32_t on);
int hy_moe_prof_read(hy_moe_ctx* ctx, int32_t kernel_id, uint64_t* launches, double* total_ms);
const char* hy_moe_prof_name(int32_t kernel_id);
int32_t hy_moe_prof_count(void);

/* Counters of the last forward (host copy after completion): distinct routed
 * experts D, and tokens routed to each expert (counts [E]). */
int hy_moe_last_routing(hy_moe_ctx* ctx, uint32_t* distinct, int32_t* counts_host);

/* Gate statistics of the last forward (of hy_moe_stack_forward: its last layer), as
 * topkgating_full reports them in MoEGateOutput (src/hunyuan_moe_full.cpp:180-335):
 * the aux loss (0 unless compute_aux_loss), the expert capacity (with drop_tokens the
 * capacity rule, else the largest expert count; at least min_capacity) and the share
 * of the T*K pairs that took a capacity slot.  Waits for the forward to finish; any
 * output may be NULL. */
int hy_moe_last_gate(hy_moe_ctx* ctx, float* aux_loss, uint32_t* expert_capacity, float* exp_capacity_rate);

#ifdef __cplusplus
}
#endif
#endif
