// hy_route.hip -- routing-side kernels: router GEMV + top-k, activation Q8_0
// quantizer, token->expert dispatch, RMSNorm, softmax.
#include "hy_device.hpp"
#include "hy_launch.hpp"
#include "hy_layout.hpp"

namespace hy {

// ----------------------------------------------------------------------------
// Router.  Reference: src/hunyuan_moe_full.cpp:414-423 (GEMV), :41-50 (softmax),
// :56-82 (top-k), :104-108 / :230-243 (renormalisation).
//
// logits[t][e]: lane l of a wave owns x/Wr elements h = 4l + 256i (+0..3) and
// accumulates them with fmaf in increasing h; the 64 partials fold in the tree
// p[l] += p[l+s], s = 32..1.  Top-k on the logits: K rounds of a wave max, lowest
// lane among equal maxima (lower expert index wins ties), then weights
// p_k = exp(l_k - m) / sum_e exp(l_e - m) renormalised by max(sum_k p_k, 1e-8),
// exp = hy_expf and the denominator summed in the 64-lane tree.
// ----------------------------------------------------------------------------
constexpr int ROUTER_WAVES = 4;

// Group-limited greedy (src/hunyuan_moe_full.cpp:135-178) for one token, one expert
// per lane, step by step on the probabilities p_e = exp(l_e - m) / s (the exp and the
// 64-lane tree sum of topk_wave): group g of the E / n_group experts from g * (E /
// n_group) scores max(0, its p_e); the topk_group best groups (wave max, lower index
// on ties) stay, the other groups' experts get p = 0; the top K of the masked p (equal
// values: lower index) are selected and weighted by their masked p.  Experts past
// n_group * (E / n_group) belong to no group and keep their p.
__device__ __forceinline__ void topk_groups_wave(float v_in, int E, int K, int norm, float scale, int n_group,
                                                 int topk_group, int lane, float* w_out, int* i_out, float* p_out) {
    const float orig = lane < E ? v_in : -INFINITY;
    const float m0 = wave_max(orig);
    const float s = wave_sum(lane < E ? hy_expf(orig - m0) : 0.0f);
    float p = lane < E ? hy_expf(orig - m0) / s : 0.0f;
    const int gs = E / n_group;
    // lane g < n_group: the score of group g
    float gsc = -INFINITY;
    for (int g = 0; g < n_group; g++) {
        const float m = wave_max(gs > 0 && lane >= g * gs && lane < (g + 1) * gs ? p : 0.0f);
        if (lane == g) gsc = m;
    }
    // the best min(topk_group, n_group) groups (more rounds would re-pick group 0)
    int keep_g = 0;
    const int rounds = topk_group < n_group ? topk_group : n_group;
    for (int r = 0; r < rounds; r++) {
        const float m = wave_max(gsc);
        const int sel = (int)__builtin_ctzll(__ballot(gsc == m));
        if (lane == sel) {
            keep_g = 1;
            gsc = -INFINITY;
        }
    }
    const int my_g = gs > 0 ? lane / gs : n_group;
    const bool grouped = my_g < n_group;
    const int kept = __shfl(keep_g, grouped ? my_g : 0, WAVE);
    if (grouped && !kept) p = 0.0f;
    if (p_out && lane < E) p_out[lane] = p;
    // top K of the masked probabilities (K <= E open lanes; NaN ranks lowest)
    float v = lane < E ? p : -INFINITY;
    bool open = lane < E;
    float selv = 0.0f;
    int seli = 0;
    for (int k = 0; k < K; k++) {
        float m;
        const int sel = wave_argmax_round(v, open, m);
        if (lane == k) {
            selv = m;
            seli = sel;
        }
        if (lane == sel) {
            v = -INFINITY;
            open = false;
        }
    }
    float ps = 0.0f;
    for (int k = 0; k < K; k++) ps += __shfl(selv, k, WAVE);
    if (ps < 1e-8f) ps = 1e-8f;
    if (lane < K) {
        w_out[lane] = norm ? selv / ps : selv * scale;
        i_out[lane] = seli;
    }
}

// Router logits.  Work item of one wave = (TPW tokens) x (EPW experts); a block's
// four waves take consecutive items, experts varying fastest so they share the
// token rows in L1.  Decode batches (T <= 16) use <1,1> (one dot per wave), T <= 32
// <8,1>, up to 2047 tokens <4,8> (each Wr float4 feeds 4 tokens, 32 accumulators per
// lane), larger batches <8,8>: each loaded float4 feeds 8 dots, 64 accumulators per lane
// (1.05 GB of L2 reads at T=4096 against 1.57 GB for <4,8>: 61 vs 78 us; at T=512 its
// 512 waves are too few, 27 vs 23 us).  The
// h loop is software-pipelined: the loads of the next D - 1 chunks of 256 elements
// are in flight while a chunk is accumulated (a large batch has about one wave per
// SIMD, so the wave itself must cover the memory latency).  The per-lane
// accumulation order is unchanged.
// chunks of 256 elements in flight per lane: about 144 VGPRs of staged operands
constexpr int router_depth(int tpw, int epw) {
    return 144 / (4 * (tpw + epw)) >= 8 ? 8 : (144 / (4 * (tpw + epw)) < 2 ? 2 : 144 / (4 * (tpw + epw)));
}

// FULL: every lane's every chunk is in range (H a multiple of 256, and of D chunks),
// so the accumulation needs no per-chunk select
template <int TPW, int EPW, bool FULL = false>
__device__ __forceinline__ void router_logits_block(const float* __restrict__ x, const float* __restrict__ wr, int T,
                                                    int H, int E, float* __restrict__ logits, int block) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int n_eg = (E + EPW - 1) / EPW;
    const int item = block * ROUTER_WAVES + wave;
    const int t0 = (item / n_eg) * TPW, e0 = (item % n_eg) * EPW;
    if (t0 >= T) return;
    float acc[TPW][EPW];
#pragma unroll
    for (int t = 0; t < TPW; t++)
#pragma unroll
        for (int e = 0; e < EPW; e++) acc[t][e] = 0.0f;
    constexpr int D = router_depth(TPW, EPW);
    const int nch = (H + 4 * WAVE - 1) / (4 * WAVE);
    float4 xb[D][TPW], wb[D][EPW];
    // chunk i of this lane: elements h0 = 4 lane + 256 i .. + 3 (H % 4 == 0: a lane's
    // 4 elements are all in range or all out).  The loads are unconditional, from
    // clamped rows / offsets (always in bounds): tokens past T and experts past E
    // accumulate a copy that is never stored, chunks past the lane's end are skipped
    // in the accumulation.  (Zero-filling loads under a condition would make the
    // compiler wait for every load at the branch join, serialising the pipeline.)
    const float* xrow[TPW];
    const float* wrow[EPW];
#pragma unroll
    for (int t = 0; t < TPW; t++) xrow[t] = x + (size_t)min(t0 + t, T - 1) * H;
#pragma unroll
    for (int e = 0; e < EPW; e++) wrow[e] = wr + (size_t)min(e0 + e, E - 1) * H;
    auto load = [&](int i, float4* xd, float4* wd) {
        const int h0 = min(4 * lane + 4 * WAVE * i, H - 4);
#pragma unroll
        for (int t = 0; t < TPW; t++) xd[t] = *reinterpret_cast<const float4*>(xrow[t] + h0);
#pragma unroll
        for (int e = 0; e < EPW; e++) wd[e] = *reinterpret_cast<const float4*>(wrow[e] + h0);
    };
#pragma unroll
    for (int d = 0; d < D - 1; d++) load(d, xb[d], wb[d]);
    for (int i0 = 0; i0 < nch; i0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int i = i0 + d;
            // refill the slot of chunk i - 1 with chunk i + D - 1
            load(i + D - 1, xb[(d + D - 1) % D], wb[(d + D - 1) % D]);
            __builtin_amdgcn_sched_barrier(0);  // keep the refill ahead of the math
            // chunk past the lane's end: the accumulators keep their values (a select,
            // not a branch, so no wait is forced on the loads in flight)
            const bool ok = FULL || (i < nch && 4 * lane + 4 * WAVE * i < H);
#pragma unroll
            for (int t = 0; t < TPW; t++)
#pragma unroll
                for (int e = 0; e < EPW; e++) {
                    const float4 xv = xb[d][t], wv = wb[d][e];
                    float a = acc[t][e];
                    a = fmaf(xv.x, wv.x, a);
                    a = fmaf(xv.y, wv.y, a);
                    a = fmaf(xv.z, wv.z, a);
                    a = fmaf(xv.w, wv.w, a);
                    acc[t][e] = ok ? a : acc[t][e];
                }
        }
    }
    // the 64-lane tree p[l] += p[l + s], s = 32..1, one level at a time over all the
    // accumulators, so each level's shuffles are in flight together
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1)
#pragma unroll
        for (int t = 0; t < TPW; t++)
#pragma unroll
            for (int e = 0; e < EPW; e++) acc[t][e] += shfl_down(acc[t][e], sh);
    if (lane == 0) {
#pragma unroll
        for (int t = 0; t < TPW; t++)
#pragma unroll
            for (int e = 0; e < EPW; e++)
                if (t0 + t < T && e0 + e < E) logits[(size_t)(t0 + t) * E + e0 + e] = acc[t][e];
    }
}

template <int TPW, int EPW, bool FULL = false>
__global__ __launch_bounds__(ROUTER_WAVES * WAVE) void router_logits_kernel(
    const float* __restrict__ x, const float* __restrict__ wr, int T, int H, int E, float* __restrict__ logits) {
    router_logits_block<TPW, EPW, FULL>(x, wr, T, H, E, logits, (int)blockIdx.x);
}

// Top-k + weights per token (one wave each), optionally quantizing the token's
// activation row to Q8_0 in the same pass (saves a launch in the decode regime).
// Activation quantizer body (ggml quantize_row_q8_0 definition): one element per lane,
// a half-wave per 32-block.  Writes the int8 plane, the scale as f32 (the exact value
// of the fp16 scale), the block's int sum, and optionally GGUF blocks.
__device__ __forceinline__ void quant_q8_0_elem(const float* __restrict__ x, size_t n, size_t idx,
                                                int8_t* __restrict__ q, float* __restrict__ d,
                                                int* __restrict__ qsum, uint8_t* __restrict__ blocks) {
    const bool live = idx < n;  // n is a multiple of 32: a half-wave is all live or all dead
    const float v = live ? x[idx] : 0.0f;
    const Q8Result r = quant_q8_0_lane32(v);
    int s = r.q;
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) s += shfl_xor(s, m, 32);
    if (!live) return;
    const size_t b = idx / QK;
    const int j = (int)(idx % QK);
    if (q) q[idx] = r.q;
    if (j == 0) {
        if (d) d[b] = h2f(r.dh);
        if (qsum) qsum[b] = s;
    }
    if (blocks) {
        uint8_t* blk = blocks + b * 34;
        blk[2 + j] = (uint8_t)r.q;
        if (j == 0) {
            blk[0] = (uint8_t)(r.dh & 0xff);
            blk[1] = (uint8_t)(r.dh >> 8);
        }
    }
}

// Selection (one wave per token, work groups [0, ceil(T/4))) and, when xq is given,
// the Q8_0 quantization of x by the work groups after those (256 elements each), so
// decode batches need no separate quantization launch.
__global__ __launch_bounds__(256) void route_select_kernel(const float* __restrict__ logits, int T, int E, int K,
                                                           int norm, float scale, float* __restrict__ topw,
                                                           int* __restrict__ topi, const float* __restrict__ x,
                                                           int H, int8_t* __restrict__ xq, float* __restrict__ xd,
                                                           int* __restrict__ xs, RouteOpts opt) {
    const int sel_groups = (T + 3) / 4;
    if ((int)blockIdx.x >= sel_groups) {
        const size_t idx = (size_t)(blockIdx.x - sel_groups) * 256 + threadIdx.x;
        quant_q8_0_elem(x, (size_t)T * H, idx, xq, xd, xs, nullptr);
        return;
    }
    const int tok = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (tok >= T) return;
    const float v = lane < E ? logits[(size_t)tok * E + lane] : 0.0f;
    float* p_out = opt.probs ? opt.probs + (size_t)tok * E : nullptr;
    if (opt.n_group > 0 && opt.topk_group > 0)
        topk_groups_wave(v, E, K, norm, scale, opt.n_group, opt.topk_group, lane, topw + (size_t)tok * K,
                         topi + (size_t)tok * K, p_out);
    else
        topk_wave(v, E, K, norm, scale, lane, topw + (size_t)tok * K, topi + (size_t)tok * K, p_out);
}

hipError_t launch_router(const float* x, const float* wr, int T, int H, int E, int K, int norm, float scale,
                         float* logits, float* topw, int* topi, hipStream_t s) {
    return launch_router_q(x, wr, T, H, E, K, norm, scale, logits, topw, topi, nullptr, nullptr, nullptr, s);
}

hipError_t launch_router_q(const float* x, const float* wr, int T, int H, int E, int K, int norm, float scale,
                           float* logits, float* topw, int* topi, int8_t* xq, float* xd, int* xs, hipStream_t s,
                           bool logits_only, RouteOpts opt) {
    const dim3 blk(ROUTER_WAVES * WAVE);
    auto grid_for = [&](int tpw, int epw) {
        const int items = ((T + tpw - 1) / tpw) * ((E + epw - 1) / epw);
        return dim3((items + ROUTER_WAVES - 1) / ROUTER_WAVES);
    };
    if (T <= 16) {
        // decode batches: one (token, expert) item per wave, T x E waves; a wave that
        // covers several tokens serialises their dot products (9.3 vs 4.5 us at T=8)
        hipLaunchKernelGGL((router_logits_kernel<1, 1>), grid_for(1, 1), blk, 0, s, x, wr, T, H, E, logits);
    } else if (T <= 32) {
        hipLaunchKernelGGL((router_logits_kernel<8, 1>), grid_for(8, 1), blk, 0, s, x, wr, T, H, E, logits);
    } else {
        // full chunks: H a multiple of D x 256 elements
        auto full = [&](int d) { return H % (4 * WAVE * d) == 0; };
        if (T >= 2048) {
            if (full(router_depth(8, 8)))
                hipLaunchKernelGGL((router_logits_kernel<8, 8, true>), grid_for(8, 8), blk, 0, s, x, wr, T, H, E, logits);
            else
                hipLaunchKernelGGL((router_logits_kernel<8, 8>), grid_for(8, 8), blk, 0, s, x, wr, T, H, E, logits);
        } else {
            if (full(router_depth(4, 8)))
                hipLaunchKernelGGL((router_logits_kernel<4, 8, true>), grid_for(4, 8), blk, 0, s, x, wr, T, H, E, logits);
            else
                hipLaunchKernelGGL((router_logits_kernel<4, 8>), grid_for(4, 8), blk, 0, s, x, wr, T, H, E, logits);
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || logits_only) return e;
    const unsigned quant_groups = xq ? (unsigned)(((size_t)T * H + 255) / 256) : 0u;
    hipLaunchKernelGGL(route_select_kernel, dim3((T + 3) / 4 + quant_groups), dim3(256), 0, s, logits, T, E, K, norm,
                       scale, topw, topi, x, H, xq, xd, xs, opt);
    return hipGetLastError();
}

// top-k gating from given logits (topkgating_easy, src/hunyuan_moe_full.cpp:88-113;
// with options, the selection of topkgating_full :129-243): one wave per token.
hipError_t launch_topk_from_logits(const float* logits, int T, int E, int K, int norm, float scale, float* topw,
                                   int* topi, hipStream_t s, RouteOpts opt) {
    hipLaunchKernelGGL(route_select_kernel, dim3((T + 3) / 4), dim3(256), 0, s, logits, T, E, K, norm, scale, topw,
                       topi, nullptr, 0, nullptr, nullptr, nullptr, opt);
    return hipGetLastError();
}

// Load-balancing aux loss (src/hunyuan_moe_full.cpp:182-206), one work group:
// tokens_per_expert = count / T (the per-token mask summed as floats is the exact count;
// counts from the dispatch), router_prob_per_expert = the expert's gate summed over
// tokens in order / T (thread e sums column e); then thread 0 adds the E products in
// expert order and multiplies by E * E.
constexpr int AUX_THREADS = 1024, AUX_ROWS = 128, AUX_D = 4;  // rows per chunk, chunks in flight

__global__ __launch_bounds__(AUX_THREADS) void aux_loss_kernel(const float* __restrict__ probs,
                                                               const int* __restrict__ cnt, int T, int E,
                                                               float* __restrict__ out) {
    // gate rows arrive in chunks of AUX_ROWS x E floats, read by all threads with
    // coalesced loads AUX_D chunks ahead (one work group streams the whole matrix, so
    // its bytes in flight set the rate) into registers, then through a double-buffered
    // LDS stage; thread e < E adds its expert's column in token order, one rounding per
    // add, as the sequential sum does
    __shared__ float stage[2][AUX_ROWS * MAX_E];
    __shared__ float prod[MAX_E];
    constexpr int PER = AUX_ROWS * MAX_E / AUX_THREADS;
    const int tid = threadIdx.x;
    const int chunk = AUX_ROWS * E;                 // floats per chunk
    const size_t total = (size_t)T * E;
    const int nchunks = (T + AUX_ROWS - 1) / AUX_ROWS;
    float v[AUX_D][PER];
    // unconditional loads from clamped addresses (a value past the chunk or the matrix
    // is never stored): branch-free, so each store waits only for its own chunk's loads
    auto load = [&](int c, float (&dst)[PER]) {
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const size_t g = (size_t)c * chunk + (size_t)(j * AUX_THREADS + tid);
            dst[j] = probs[g < total ? g : total - 1];
        }
    };
    auto store = [&](int buf, const float (&src)[PER]) {
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int i = j * AUX_THREADS + tid;
            if (i < chunk) stage[buf][i] = src[j];
        }
    };
#pragma unroll
    for (int d = 0; d < AUX_D; d++)
        if (d < nchunks) load(d, v[d]);
    store(0, v[0]);
    __syncthreads();
    float r = 0.0f;
    for (int c0 = 0; c0 < nchunks; c0 += AUX_D) {
#pragma unroll
        for (int d = 0; d < AUX_D; d++) {
            const int c = c0 + d;   // chunk c's rows are in stage[c & 1]; v[d] held them
            if (c >= nchunks) break;
            if (tid < E) {
                const int rows = min(AUX_ROWS, T - c * AUX_ROWS);
                const float* col = stage[c & 1] + tid;
                int k = 0;
                for (; k + 16 <= rows; k += 16) {   // 16 reads in flight, then their adds in order
                    float q[16];
#pragma unroll
                    for (int j = 0; j < 16; j++) q[j] = col[(k + j) * E];
#pragma unroll
                    for (int j = 0; j < 16; j++) r += q[j];
                }
                for (; k < rows; k++) r += col[k * E];
            }
            // chunk c + 1 into the other buffer (summed, as chunk c - 1, before the last
            // barrier), and chunk c + AUX_D into the registers chunk c came from
            if (c + 1 < nchunks) store((c + 1) & 1, v[(d + 1) % AUX_D]);
            if (c + AUX_D < nchunks) load(c + AUX_D, v[d]);
            __syncthreads();
        }
    }
    if (tid < E) {
        const float tpe = (float)cnt[tid] / (float)T, rpe = r / (float)T;
        prod[tid] = tpe * rpe;
    }
    __syncthreads();
    if (tid == 0) {
        float l = 0.0f;
        for (int i = 0; i < E; i++) l += prod[i];
        out[0] = l * (float)(E * E);
    }
}

hipError_t launch_aux_loss(const float* probs, const int* cnt, int T, int E, float* out, hipStream_t s) {
    hipLaunchKernelGGL(aux_loss_kernel, dim3(1), dim3(AUX_THREADS), 0, s, probs, cnt, T, E, out);
    return hipGetLastError();
}

// softmax_f32 (src/hunyuan_moe_full.cpp:41-50) per row: max, exp, sum, divide.
__global__ __launch_bounds__(256) void softmax_rows_kernel(float* x, int rows, int n) {
    const int row = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (row >= rows) return;
    float* r = x + (size_t)row * n;
    float m = -INFINITY;
    for (int i = lane; i < n; i += WAVE) m = fmaxf(m, r[i]);
    m = wave_max(m);
    float s = 0.0f;
    for (int i = lane; i < n; i += WAVE) {
        const float e = expf(r[i] - m);
        r[i] = e;
        s += e;
    }
    s = wave_sum(s);
    for (int i = lane; i < n; i += WAVE) r[i] = r[i] / s;
}

hipError_t launch_softmax_rows(float* x, int rows, int n, hipStream_t s) {
    hipLaunchKernelGGL(softmax_rows_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, rows, n);
    return hipGetLastError();
}

// ----------------------------------------------------------------------------
// Activation quantizer (ggml quantize_row_q8_0 definition).  One element per lane,
// a half-wave per 32-block.  Writes the int8 plane, the scale as f32 (the exact
// value of the fp16 scale), the block's int sum, and optionally GGUF blocks.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quant_q8_0_kernel(const float* __restrict__ x, size_t n,
                                                         int8_t* __restrict__ q, float* __restrict__ d,
                                                         int* __restrict__ qsum, uint8_t* __restrict__ blocks) {
    quant_q8_0_elem(x, n, (size_t)blockIdx.x * blockDim.x + threadIdx.x, q, d, qsum, blocks);
}

// The same quantizer for the activation planes only (no GGUF blocks), 8 elements per
// lane: a 32-block is 4 lanes (max and sum over 2 xor steps).  max and the int sum
// are order-free, and each element takes the same operations, so the bytes equal
// quant_q8_0_elem's.
__global__ __launch_bounds__(256) void quant_q8_0_vec_kernel(const float* __restrict__ x, size_t n8,
                                                             int8_t* __restrict__ q, float* __restrict__ d,
                                                             int* __restrict__ qsum) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // group of 8 elements
    const bool live = i < n8;  // n8 is a multiple of 4: a block's 4 lanes are all live or all dead
    float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
    if (live) {
        v0 = reinterpret_cast<const float4*>(x)[2 * i];
        v1 = reinterpret_cast<const float4*>(x)[2 * i + 1];
    }
    const float xs[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(xs[j]));
    amax = fmaxf(amax, shfl_xor(amax, 1, 4));
    amax = fmaxf(amax, shfl_xor(amax, 2, 4));
    const float dd = amax / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    int sum = 0;
    uint32_t p0 = 0, p1 = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int qv = (int)__builtin_roundf(xs[j] * id);
        sum += qv;
        if (j < 4)
            p0 |= ((uint32_t)(qv & 0xff)) << (8 * j);
        else
            p1 |= ((uint32_t)(qv & 0xff)) << (8 * (j - 4));
    }
    sum += shfl_xor(sum, 1, 4);
    sum += shfl_xor(sum, 2, 4);
    if (!live) return;
    reinterpret_cast<uint2*>(q)[i] = make_uint2(p0, p1);
    if ((i & 3) == 0) {
        d[i / 4] = h2f(f2h(dd));
        qsum[i / 4] = sum;
    }
}

hipError_t launch_quant_q8_0(const float* x, size_t n, int8_t* q, float* d, int* qsum, uint8_t* blocks,
                             hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (!blocks && q && d && qsum) {
        const size_t n8 = n / 8;
        hipLaunchKernelGGL(quant_q8_0_vec_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s, x, n8, q, d,
                           qsum);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(quant_q8_0_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n, q, d, qsum,
                       blocks);
    return hipGetLastError();
}

// ----------------------------------------------------------------------------
// Dispatch: counting sort of the T*K (token, expert) pairs by expert.  Within an
// expert the order is the reference's capacity-slot priority
// (src/hunyuan_moe_full.cpp:245-304): flat slot i = k*T + t ascending, i.e. all
// rank-0 choices by token, then rank-1, ...  A pair's position inside its expert's
// list is therefore the reference's dispatch_mask slot c.  Also builds the per-token
// combine lists (pairs in ascending expert order, the einsum_combine summation
// order of :387-397) and a list of tiles of at most NT pairs.
// Three launches, no atomics outside LDS:
//  1. dispatch_rank_kernel, one work group per (block of 1024 tokens, rank k): an LDS
//     bitmap of the block's tokens per expert gives each pair its rank among the
//     block's pairs of that expert and rank, and the block's count per expert;
//  2. dispatch_scan_kernel, one work group: block counts -> exclusive bases in k-major
//     order, expert offsets and tiles;
//  3. dispatch_scatter_kernel, one thread per pair: position = offset + base + rank,
//     the sorted token list and the combine lists.
// ----------------------------------------------------------------------------
constexpr int DSP_BLOCK = 1024;  // tokens per rank work group

__device__ __forceinline__ int wave_excl_scan(int v, int lane) {
    int incl = v;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const int u = __shfl_up(incl, d, WAVE);
        if (lane >= d) incl += u;
    }
    return incl - v;
}


struct DispatchOut {
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

__global__ __launch_bounds__(DSP_BLOCK) void dispatch_rank_kernel(const int* __restrict__ topi, int T, int K, int E,
                                                                 int* __restrict__ blk_cnt, int* __restrict__ rank) {
    __shared__ uint32_t mask[MAX_E][DSP_BLOCK / 32];
    __shared__ int wpre[MAX_E][DSP_BLOCK / 32];
    const int blk = blockIdx.x, k = blockIdx.y, tid = threadIdx.x;
    const int nblk = gridDim.x;
    for (int i = tid; i < MAX_E * (DSP_BLOCK / 32); i += DSP_BLOCK) (&mask[0][0])[i] = 0u;
    __syncthreads();
    const int t = blk * DSP_BLOCK + tid;
    int e = t < T ? topi[(size_t)t * K + k] : -1;
    if (e >= E) e = -1;  // an out-of-range id is dropped (never produced by the router)
    if (e >= 0) atomicOr(&mask[e][tid / 32], 1u << (tid % 32));
    __syncthreads();
    // per expert: exclusive prefix of the 32 words' popcounts (a half-wave per expert)
    for (int i = tid; i < MAX_E * (DSP_BLOCK / 32); i += DSP_BLOCK) {
        const int ee = i / 32, w = i % 32;
        const int c = __popc(mask[ee][w]);
        int incl = c;
#pragma unroll
        for (int d = 1; d < 32; d <<= 1) {
            const int u = __shfl_up(incl, d, 32);
            if (w >= d) incl += u;
        }
        wpre[ee][w] = incl - c;
        if (w == 31 && ee < E) blk_cnt[((size_t)k * nblk + blk) * E + ee] = incl;
    }
    __syncthreads();
    if (e >= 0)
        rank[(size_t)t * K + k] = wpre[e][tid / 32] + __popc(mask[e][tid / 32] & ((1u << (tid % 32)) - 1u));
}

// blk_cnt [K][nblk][E] (k-major: the priority order) -> exclusive bases in place
__global__ __launch_bounds__(256) void dispatch_scan_kernel(int T, int K, int E, int NT, int has_shared, int nblk,
                                                            int cap, int* __restrict__ blk_cnt, DispatchOut o) {
    __shared__ int cnt_s[MAX_E];
    const int tid = threadIdx.x, lane = tid % WAVE;
    const int nkb = K * nblk;
    if (tid < E) {
        // 16 counts loaded before any base is stored, so the loads overlap
        int run = 0;
        for (int kb0 = 0; kb0 < nkb; kb0 += 16) {
            int c[16];
#pragma unroll
            for (int j = 0; j < 16; j++) c[j] = kb0 + j < nkb ? blk_cnt[(size_t)(kb0 + j) * E + tid] : 0;
#pragma unroll
            for (int j = 0; j < 16; j++)
                if (kb0 + j < nkb) {
                    blk_cnt[(size_t)(kb0 + j) * E + tid] = run;
                    run += c[j];
                }
        }
        cnt_s[tid] = run;
    }
    __syncthreads();
    if (tid < WAVE) {
        // c pairs of the expert, the first min(c, cap) of them computed (capacity slots,
        // src/hunyuan_moe_full.cpp:296-304: a pair at slot >= capacity is dropped)
        const int c = lane < E ? cnt_s[lane] : 0;
        const int kc = c < cap ? c : cap;
        const int nt = (kc + NT - 1) / NT;
        const int off = wave_excl_scan(c, lane), toff = wave_excl_scan(nt, lane);
        const int total = __shfl(off + c, WAVE - 1, WAVE), routed = __shfl(toff + nt, WAVE - 1, WAVE);
        const int distinct = __popcll(__ballot(c > 0));
        const int ns = has_shared ? (T + NT - 1) / NT : 0;
        if (lane < E) {
            o.cnt[lane] = c;
            o.off[lane] = off;
            o.meta[META_TILE_OFF + lane] = toff;
            for (int j = 0; j < nt; j++) {
                o.tile_e[toff + j] = lane;
                o.tile_start[toff + j] = j * NT;
                o.tile_n[toff + j] = min(NT, kc - j * NT);
            }
        }
        if (lane == 0) {
            o.off[E] = total;
            o.meta[0] = routed;
            o.meta[1] = routed + ns;
            o.meta[2] = distinct;
            o.meta[3] = T;
            o.meta[META_TILE_OFF + E] = routed;
            o.meta[META_TILE_OFF + E + 1] = routed + ns;
        }
        for (int j = lane; j < ns; j += WAVE) {
            o.tile_e[routed + j] = E;
            o.tile_start[routed + j] = j * NT;
            o.tile_n[routed + j] = min(NT, T - j * NT);
        }
    }
}

__global__ __launch_bounds__(256) void dispatch_scatter_kernel(const int* __restrict__ topi,
                                                               const float* __restrict__ topw, int T, int K, int E,
                                                               int nblk, int cap, const int* __restrict__ blk_base,
                                                               DispatchOut o) {
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= T * K) return;
    const int t = p / K, k = p - t * K;
    const int e = topi[p];
    if (e < 0 || e >= E) return;
    const int slot = blk_base[((size_t)k * nblk + t / DSP_BLOCK) * E + e] + o.pair_pos[p];
    const int pos = o.off[e] + slot;
    o.pair_pos[p] = pos;
    o.srt_tok[pos] = t;
    // combine list slot: the token's experts are distinct, so the pair's place in
    // ascending expert order is the count of the token's smaller experts
    int r = 0;
    for (int j = 0; j < K; j++) r += topi[(size_t)t * K + j] < e;
    o.comb_pos[(size_t)t * K + r] = pos;
    o.comb_w[(size_t)t * K + r] = slot < cap ? topw[p] : 0.0f;  // a dropped pair adds nothing
}

// ----------------------------------------------------------------------------
// Decode routing after the router logits (T <= 16, T*K <= 256), one launch:
//  * work group 0 selects the top-k of every token (one wave per token, topk_wave)
//    and builds the dispatch lists exactly as launch_dispatch does: pairs ranked in
//    k-major capacity-slot priority, per-expert offsets and tiles (then the shared
//    expert's), per-token combine lists in ascending expert order;
//  * work groups 1.. quantize x to Q8_0, 256 elements each.
// (Folding the logits into this launch needs a hand-off between work groups: with an
// agent-scope release, which writes back the XCD's L2, and with write-through stores
// and agent-scope loads alike, it measured slower than the kernel boundary.)
// ----------------------------------------------------------------------------
struct DecodeRouteArgs {
    const float* x;
    const float* logits;
    int T, H, E, K, norm;
    float scale;
    float* topw;
    int* topi;
    int8_t* xq;
    float* xd;
    int* xs;
    int NT, has_shared;
    DispatchOut o;
};


// route_decode_kernel's work group: RD_WAVES waves, one per token of a decode batch
// (4, 8 or 16 for T <= 4, 8, 16; at T = 8 one token per wave instead of two: router
// 12.6-13.0 -> 10.7-11.0 us)
template <int RD_WAVES>
__global__ __launch_bounds__(RD_WAVES * WAVE) void route_decode_kernel(DecodeRouteArgs a) {
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    if (blockIdx.x > 0) {
        const size_t idx = (size_t)(blockIdx.x - 1) * (RD_WAVES * WAVE) + tid;
        quant_q8_0_elem(a.x, (size_t)a.T * a.H, idx, a.xq, a.xd, a.xs, nullptr);
        return;
    }
    const int T = a.T, E = a.E, K = a.K;

    // ---- selection: one wave per token
    __shared__ int sel_e[MAX_DECODE_PAIRS];
    __shared__ float sel_w[MAX_DECODE_PAIRS];
    __shared__ int rank_s[MAX_DECODE_PAIRS], pos_s[MAX_DECODE_PAIRS];
    __shared__ int cnt_s[MAX_E], off_s[MAX_E + 1], toff_s[MAX_E + 2];
    // a wave's tokens t = wave + 4i: all their logits rows are loaded before the first
    // selection, so the loads' latency is paid once
    constexpr int TPWV = (16 + RD_WAVES - 1) / RD_WAVES;  // decode batches: T <= 16
    float lv[TPWV];
#pragma unroll
    for (int i = 0; i < TPWV; i++) {
        const int t = wave + i * RD_WAVES;
        lv[i] = (t < T && lane < E) ? a.logits[(size_t)t * E + lane] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < TPWV; i++) {
        const int t = wave + i * RD_WAVES;
        if (t >= T) break;
        topk_wave(lv[i], E, K, a.norm, a.scale, lane, sel_w + t * K, sel_e + t * K);
        if (lane < K) {
            a.topw[t * K + lane] = sel_w[t * K + lane];
            a.topi[t * K + lane] = sel_e[t * K + lane];
        }
    }
    if (tid < MAX_E) cnt_s[tid] = 0;
    __syncthreads();
    // ---- dispatch: rank of each pair inside its expert in k-major order (all pairs of
    // earlier ranks, then the same rank's earlier tokens).  Thread q takes the q-th pair
    // of that order (token q % T, rank q / T); the pairs before it with the same expert
    // are counted from each wave's ballots of the expert ids' six bits.
    static_assert(MAX_E <= 64 && MAX_DECODE_PAIRS <= RD_WAVES * WAVE, "six id bits, one pair per thread");
    __shared__ unsigned long long bal_s[RD_WAVES][7];
    const int P = T * K;
    const bool qv = tid < P;
    const int qt = tid % T, qk = tid / T;
    const int qe = qv ? sel_e[qt * K + qk] : 0;
    {
        unsigned long long b[7];
#pragma unroll
        for (int i = 0; i < 6; i++) b[i] = __ballot(qv && ((qe >> i) & 1));
        b[6] = __ballot(qv);
        if (lane == 0)
#pragma unroll
            for (int i = 0; i < 7; i++) bal_s[wave][i] = b[i];
    }
    __syncthreads();
    if (qv) {
        int rank = 0;
        for (int w = 0; w <= wave; w++) {
            unsigned long long m = bal_s[w][6];
#pragma unroll
            for (int i = 0; i < 6; i++) m &= ((qe >> i) & 1) ? bal_s[w][i] : ~bal_s[w][i];
            if (w == wave) m &= (1ull << lane) - 1ull;
            rank += __popcll(m);
        }
        rank_s[qt * K + qk] = rank;
        atomicAdd(&cnt_s[qe], 1);
    }
    __syncthreads();
    const int pt = tid / K;  // this thread's pair in token order (token pt, rank tid % K)
    const int NT = a.NT;
    if (wave == 0) {
        const int c = lane < E ? cnt_s[lane] : 0;
        const int nt = (c + NT - 1) / NT;
        const int off = wave_excl_scan(c, lane), toff = wave_excl_scan(nt, lane);
        const int total = __shfl(off + c, WAVE - 1, WAVE), routed = __shfl(toff + nt, WAVE - 1, WAVE);
        const int distinct = __popcll(__ballot(c > 0));
        const int all = routed + (a.has_shared ? (T + NT - 1) / NT : 0);
        if (lane < E) {
            off_s[lane] = off;
            toff_s[lane] = toff;
            a.o.cnt[lane] = c;
            a.o.off[lane] = off;
            a.o.meta[META_TILE_OFF + lane] = toff;
            for (int j = 0; j < nt; j++) {
                a.o.tile_e[toff + j] = lane;
                a.o.tile_start[toff + j] = j * NT;
                a.o.tile_n[toff + j] = min(NT, c - j * NT);
            }
        }
        if (lane == 0) {
            off_s[E] = total;
            toff_s[E] = routed;
            a.o.off[E] = total;
            a.o.meta[0] = routed;
            a.o.meta[1] = all;
            a.o.meta[2] = distinct;
            a.o.meta[3] = T;
            a.o.meta[META_TILE_OFF + E] = routed;
            a.o.meta[META_TILE_OFF + E + 1] = all;
        }
    }
    __syncthreads();
    if (a.has_shared) {
        const int ns = (T + NT - 1) / NT;
        for (int j = tid; j < ns; j += RD_WAVES * WAVE) {
            a.o.tile_e[toff_s[E] + j] = E;
            a.o.tile_start[toff_s[E] + j] = j * NT;
            a.o.tile_n[toff_s[E] + j] = min(NT, T - j * NT);
        }
    }
    if (tid < P) {
        const int pos = off_s[sel_e[tid]] + rank_s[tid];
        pos_s[tid] = pos;
        a.o.pair_pos[tid] = pos;
        a.o.srt_tok[pos] = pt;
    }
    __syncthreads();
    // combine lists: each token's pairs in ascending expert order (a token's experts
    // are distinct, so a pair's place is the count of its token's smaller experts)
    if (tid < P) {
        const int e = sel_e[tid];
        int r = 0;
        for (int j = 0; j < K; j++) r += sel_e[pt * K + j] < e;
        a.o.comb_pos[pt * K + r] = pos_s[tid];
        a.o.comb_w[pt * K + r] = sel_w[tid];
    }
}

hipError_t launch_route_decode(const float* x, const float* wr, int T, int H, int E, int K, int norm, float scale,
                               float* logits, float* topw, int* topi, int8_t* xq, float* xd, int* xs, int NT,
                               int has_shared, int* cnt, int* off, int* srt_tok, int* pair_pos, int* comb_pos,
                               float* comb_w, int* tile_e, int* tile_start, int* tile_n, int* meta, hipStream_t s) {
    // one work group selects and lists every pair: T <= 16 tokens (one per wave), T*K <= 256 pairs
    if (T < 1 || T > 16 || T * K > MAX_DECODE_PAIRS || E > MAX_E) return hipErrorInvalidValue;
    hipError_t e = launch_router_q(x, wr, T, H, E, K, norm, scale, logits, topw, topi, nullptr, nullptr, nullptr, s,
                                   /*logits_only=*/true);
    if (e != hipSuccess) return e;
    DecodeRouteArgs a{x, logits, T, H, E, K, norm, scale, topw, topi, xq, xd, xs, NT, has_shared,
                      DispatchOut{cnt, off, srt_tok, pair_pos, comb_pos, comb_w, tile_e, tile_start, tile_n, meta}};
    // no quantization work groups when the caller quantized x already (xq == null)
    const int waves = T <= 4 ? 4 : (T <= 8 ? 8 : 16);
    const unsigned quant_groups = xq ? (unsigned)(((size_t)T * H + waves * WAVE - 1) / (waves * WAVE)) : 0u;
    if (waves == 4)
        hipLaunchKernelGGL(route_decode_kernel<4>, dim3(1 + quant_groups), dim3(4 * WAVE), 0, s, a);
    else if (waves == 8)
        hipLaunchKernelGGL(route_decode_kernel<8>, dim3(1 + quant_groups), dim3(8 * WAVE), 0, s, a);
    else
        hipLaunchKernelGGL(route_decode_kernel<16>, dim3(1 + quant_groups), dim3(16 * WAVE), 0, s, a);
    return hipGetLastError();
}

// One-token batches whose routing runs inside the gate/up GEMV (hy_gemv.hip): the
// router logits (one dot per wave, the <1,1> item) and, in the work groups after
// those, the Q8_0 quantization of x (256 elements each) in one launch.
__global__ __launch_bounds__(ROUTER_WAVES * WAVE) void decode_logits_kernel(const float* __restrict__ x,
                                                                          const float* __restrict__ wr, int H, int E,
                                                                          int logit_blocks, float* __restrict__ logits,
                                                                          int8_t* xq, float* xd, int* xs) {
    if ((int)blockIdx.x < logit_blocks) {
        router_logits_block<1, 1>(x, wr, 1, H, E, logits, (int)blockIdx.x);
        return;
    }
    const size_t idx = (size_t)((int)blockIdx.x - logit_blocks) * 256 + threadIdx.x;
    quant_q8_0_elem(x, (size_t)H, idx, xq, xd, xs, nullptr);
}

hipError_t launch_decode_logits(const float* x, const float* wr, int H, int E, float* logits, int8_t* xq, float* xd,
                                int* xs, hipStream_t s) {
    if (H % 32 != 0 || E < 1 || E > MAX_E) return hipErrorInvalidValue;
    const int logit_blocks = (E + ROUTER_WAVES - 1) / ROUTER_WAVES;
    // no quantization work groups when the caller quantized x already (xq == null)
    const int quant_groups = xq ? (H + 255) / 256 : 0;
    hipLaunchKernelGGL(decode_logits_kernel, dim3((unsigned)(logit_blocks + quant_groups)), dim3(ROUTER_WAVES * WAVE),
                       0, s, x, wr, H, E, logit_blocks, logits, xq, xd, xs);
    return hipGetLastError();
}

size_t dispatch_scratch_bytes(int T, int K, int E) {
    return (size_t)((T + DSP_BLOCK - 1) / DSP_BLOCK) * K * E * sizeof(int);
}

hipError_t launch_dispatch(const int* topi, const float* topw, int T, int K, int E, int NT, int has_shared,
                           int* cnt, int* off, int* srt_tok, int* pair_pos, int* comb_pos, float* comb_w,
                           int* tile_e, int* tile_start, int* tile_n, int* meta, int* scratch, hipStream_t s, int cap) {
    DispatchOut o{cnt, off, srt_tok, pair_pos, comb_pos, comb_w, tile_e, tile_start, tile_n, meta};
    const int nblk = (T + DSP_BLOCK - 1) / DSP_BLOCK;
    hipLaunchKernelGGL(dispatch_rank_kernel, dim3(nblk, K), dim3(DSP_BLOCK), 0, s, topi, T, K, E, scratch, pair_pos);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(256), 0, s, T, K, E, NT, has_shared, nblk, cap, scratch, o);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(dispatch_scatter_kernel, dim3((T * K + 255) / 256), dim3(256), 0, s, topi, topw, T, K, E, nblk,
                       cap, scratch, o);
    return hipGetLastError();
}

// ----------------------------------------------------------------------------
// RMSNorm with unit weight (src/rms_norm.cpp:9-33): sum of squares in the router's
// blocked fmaf order, then x * (1 / sqrtf(ss / H + eps)).  One wave per row.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x, int T, int H, float eps,
                                                       float* __restrict__ out) {
    const int row = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (row >= T) return;
    const float* xr = x + (size_t)row * H;
    float a = 0.0f;
    for (int h0 = 4 * lane; h0 < H; h0 += 4 * WAVE) {
        const float4 v = *reinterpret_cast<const float4*>(xr + h0);
        a = fmaf(v.x, v.x, a);
        a = fmaf(v.y, v.y, a);
        a = fmaf(v.z, v.z, a);
        a = fmaf(v.w, v.w, a);
    }
    const float ss = __shfl(tree_sum64(a), 0, WAVE);
    const float rms = 1.0f / sqrtf(ss / (float)H + eps);
    float* o = out + (size_t)row * H;
    for (int h0 = 4 * lane; h0 < H; h0 += 4 * WAVE) {
        const float4 v = *reinterpret_cast<const float4*>(xr + h0);
        *reinterpret_cast<float4*>(o + h0) = make_float4(v.x * rms, v.y * rms, v.z * rms, v.w * rms);
    }
}

hipError_t launch_rms_norm(const float* x, int T, int H, float eps, float* out, hipStream_t s) {
    hipLaunchKernelGGL(rms_norm_kernel, dim3((T + 3) / 4), dim3(256), 0, s, x, T, H, eps, out);
    return hipGetLastError();
}

// RMSNorm (optionally weighted) fused with the Q8_0 quantization of its output, one
// wave per row: the sum of squares in the same blocked order as rms_norm_kernel, then
// xn = x * rms (* w) written as f32 (the router's input) and quantized 8 elements per
// lane exactly as quant_q8_0_vec_kernel does (4 lanes per 32-block).  The values
// equal rms_norm_kernel / rms_norm_w_kernel followed by quant_q8_0_vec_kernel bit for
// bit; x is read twice from cache instead of xn being written and read back.
__global__ __launch_bounds__(256) void rms_norm_quant_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                             int T, int H, float eps, float* __restrict__ xn,
                                                             int8_t* __restrict__ q, float* __restrict__ d,
                                                             int* __restrict__ qsum) {
    const int row = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (row >= T) return;  // whole waves: the shuffles below stay within live waves
    const float* xr = x + (size_t)row * H;
    float a = 0.0f;
    for (int h0 = 4 * lane; h0 < H; h0 += 4 * WAVE) {
        const float4 v = *reinterpret_cast<const float4*>(xr + h0);
        a = fmaf(v.x, v.x, a);
        a = fmaf(v.y, v.y, a);
        a = fmaf(v.z, v.z, a);
        a = fmaf(v.w, v.w, a);
    }
    const float ss = __shfl(tree_sum64(a), 0, WAVE);
    const float rms = 1.0f / sqrtf(ss / (float)H + eps);
    const int nb = H / QK;
    for (int base = 0; base < H; base += 8 * WAVE) {  // the same trip count on every lane
        const int h8 = base + 8 * lane;
        const bool live = h8 < H;  // H is a multiple of 32: a block's 4 lanes agree
        float xs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (live) {
            const float4 v0 = *reinterpret_cast<const float4*>(xr + h8);
            const float4 v1 = *reinterpret_cast<const float4*>(xr + h8 + 4);
            const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            if (w) {
                const float4 w0 = *reinterpret_cast<const float4*>(w + h8);
                const float4 w1 = *reinterpret_cast<const float4*>(w + h8 + 4);
                const float ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                for (int j = 0; j < 8; j++) xs[j] = vv[j] * rms * ww[j];
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) xs[j] = vv[j] * rms;
            }
            float* o = xn + (size_t)row * H + h8;
            *reinterpret_cast<float4*>(o) = make_float4(xs[0], xs[1], xs[2], xs[3]);
            *reinterpret_cast<float4*>(o + 4) = make_float4(xs[4], xs[5], xs[6], xs[7]);
        }
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(xs[j]));
        amax = fmaxf(amax, shfl_xor(amax, 1, 4));
        amax = fmaxf(amax, shfl_xor(amax, 2, 4));
        const float dd = amax / 127.0f;
        const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
        int sum = 0;
        uint32_t p0 = 0, p1 = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int qv = (int)__builtin_roundf(xs[j] * id);
            sum += qv;
            if (j < 4)
                p0 |= ((uint32_t)(qv & 0xff)) << (8 * j);
            else
                p1 |= ((uint32_t)(qv & 0xff)) << (8 * (j - 4));
        }
        sum += shfl_xor(sum, 1, 4);
        sum += shfl_xor(sum, 2, 4);
        if (!live) continue;
        const size_t i8 = ((size_t)row * H + h8) / 8;
        reinterpret_cast<uint2*>(q)[i8] = make_uint2(p0, p1);
        if ((lane & 3) == 0) {
            const size_t b = (size_t)row * nb + h8 / QK;
            d[b] = h2f(f2h(dd));
            qsum[b] = sum;
        }
    }
}

// The same RMSNorm + Q8_0 with the row read once: for H a multiple of 256 up to 4096 a
// lane keeps its 4 H/256 elements (4 lane + 256 i .. +3, the sum-of-squares order)
// in registers, and the 8 lanes holding one 32-wide block reduce its amax and sum.
// Same values bit for bit.
constexpr int RMSQ_MAX_CHUNKS = 16;
__global__ __launch_bounds__(256) void rms_norm_quant_reg_kernel(const float* __restrict__ x,
                                                                 const float* __restrict__ w, int T, int H, float eps,
                                                                 float* __restrict__ xn, int8_t* __restrict__ q,
                                                                 float* __restrict__ d, int* __restrict__ qsum) {
    const int row = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (row >= T) return;  // whole waves: the shuffles below stay within live waves
    const int nc = H / (4 * WAVE);
    const float* xr = x + (size_t)row * H;
    float4 v[RMSQ_MAX_CHUNKS];
#pragma unroll
    for (int i = 0; i < RMSQ_MAX_CHUNKS; i++)
        if (i < nc) v[i] = *reinterpret_cast<const float4*>(xr + 4 * lane + 4 * WAVE * i);
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < RMSQ_MAX_CHUNKS; i++)
        if (i < nc) {
            a = fmaf(v[i].x, v[i].x, a);
            a = fmaf(v[i].y, v[i].y, a);
            a = fmaf(v[i].z, v[i].z, a);
            a = fmaf(v[i].w, v[i].w, a);
        }
    const float ss = __shfl(tree_sum64(a), 0, WAVE);
    const float rms = 1.0f / sqrtf(ss / (float)H + eps);
    const int nb = H / QK;
#pragma unroll
    for (int i = 0; i < RMSQ_MAX_CHUNKS; i++) {
        if (i >= nc) continue;  // (uniform; keeps the loop unrolled and v[] in registers)
        const int h = 4 * lane + 4 * WAVE * i;
        float xs[4] = {v[i].x * rms, v[i].y * rms, v[i].z * rms, v[i].w * rms};
        if (w) {
            const float4 ww = *reinterpret_cast<const float4*>(w + h);
            xs[0] *= ww.x;
            xs[1] *= ww.y;
            xs[2] *= ww.z;
            xs[3] *= ww.w;
        }
        *reinterpret_cast<float4*>(xn + (size_t)row * H + h) = make_float4(xs[0], xs[1], xs[2], xs[3]);
        float amax = fmaxf(fmaxf(fabsf(xs[0]), fabsf(xs[1])), fmaxf(fabsf(xs[2]), fabsf(xs[3])));
        amax = fmaxf(amax, shfl_xor(amax, 1, 8));
        amax = fmaxf(amax, shfl_xor(amax, 2, 8));
        amax = fmaxf(amax, shfl_xor(amax, 4, 8));
        const float dd = amax / 127.0f;
        const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
        int sum = 0;
        uint32_t p = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int qv = (int)__builtin_roundf(xs[j] * id);
            sum += qv;
            p |= ((uint32_t)(qv & 0xff)) << (8 * j);
        }
        sum += shfl_xor(sum, 1, 8);
        sum += shfl_xor(sum, 2, 8);
        sum += shfl_xor(sum, 4, 8);
        *reinterpret_cast<uint32_t*>(q + (size_t)row * H + h) = p;
        if ((lane & 7) == 0) {
            const size_t b = (size_t)row * nb + h / QK;
            d[b] = h2f(f2h(dd));
            qsum[b] = sum;
        }
    }
}

hipError_t launch_rms_norm_quant(const float* x, const float* w, int T, int H, float eps, float* xn, int8_t* q,
                                 float* d, int* qsum, hipStream_t s) {
    if (H % (4 * WAVE) == 0 && H <= 4 * WAVE * RMSQ_MAX_CHUNKS)
        hipLaunchKernelGGL(rms_norm_quant_reg_kernel, dim3((T + 3) / 4), dim3(256), 0, s, x, w, T, H, eps, xn, q, d,
                           qsum);
    else
        hipLaunchKernelGGL(rms_norm_quant_kernel, dim3((T + 3) / 4), dim3(256), 0, s, x, w, T, H, eps, xn, q, d,
                           qsum);
    return hipGetLastError();
}

}  // namespace hy
