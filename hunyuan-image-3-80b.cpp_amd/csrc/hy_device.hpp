// hy_device.hpp -- device helpers shared by the gfx950 kernels of the MoE block.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hy {

constexpr int QK = 32;       // GGUF block length (Q8_0 and Q4_0)
constexpr int WAVE = 64;     // CDNA wavefront
constexpr int MAX_E = 64;    // experts per layer handled by the routing kernels
constexpr int MAX_K = 64;    // top-k bound: topk_f32's best[64] (src/hunyuan_moe_full.cpp:61)
// dispatch meta block: [0] routed tiles, [1] all tiles, [2] distinct experts, [3] unused,
// [4 + e] first tile of expert e (e = 0..E, E = shared), [4 + E + 1] end of the tiles
constexpr int META_TILE_OFF = 4;
constexpr int MAX_DECODE_PAIRS = 256;  // T*K handled by the one-launch decode routing
constexpr int META_INTS = META_TILE_OFF + MAX_E + 2;

// ---------------------------------------------------------------- fp16

__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}
// round to nearest even (v_cvt_f16_f32 in the default rounding mode)
__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// ---------------------------------------------------------------- synthetic data
// Counter-based generator: splitmix64 finaliser, normal approximated by the centred
// sum of four 16-bit uniforms.  Integer ops plus one int->float conversion and one
// float multiply, identical to the CPU definition.

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__host__ __device__ __forceinline__ uint64_t stream_key(uint64_t seed, uint32_t layer, uint32_t tensor,
                                                        uint32_t expert) {
    return mix64(mix64(seed) ^ (((uint64_t)layer << 40) | ((uint64_t)tensor << 24) | (uint64_t)expert));
}

constexpr float NORM_SCALE = 2.6428990e-05f;  // 1 / sqrt((65536^2 - 1) / 3)

__device__ __forceinline__ float synth_normal(uint64_t key, uint64_t idx, float scale) {
    uint64_t r = mix64(key ^ (idx * 0xD1B54A32D192ED03ull));
    int32_t s = (int32_t)(r & 0xffffu) + (int32_t)((r >> 16) & 0xffffu) + (int32_t)((r >> 32) & 0xffffu) +
                (int32_t)(r >> 48) - 131070;
    return (float)s * scale;  // scale = stddev * NORM_SCALE, rounded once on the host
}

// tensor ids of the generator streams
enum {
    TENSOR_X = 0, TENSOR_ROUTER = 1, TENSOR_GU = 2, TENSOR_DN = 3,
    TENSOR_QKV = 4, TENSOR_O = 5, TENSOR_EMBED = 6, TENSOR_LM_HEAD = 7
};

// ---------------------------------------------------------------- wave helpers

template <typename T>
__device__ __forceinline__ T shfl_down(T v, int d) { return __shfl_down(v, d, WAVE); }
template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int m, int width = WAVE) { return __shfl_xor(v, m, width); }

// Fold 64 lane partials in the fixed tree p[l] += p[l+s], s = 32..1; lane 0 holds
// the result.  This is the reduction order the oracle restates.
__device__ __forceinline__ float tree_sum64(float v) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) v += shfl_down(v, s);
    return v;
}

// max(v, the value of the lane the DPP control CTRL names); every source lane of the
// controls used here is in range, and the callers run whole waves
template <int CTRL>
__device__ __forceinline__ float dpp_fmax(float v) {
    const int o = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false);
    return fmaxf(v, __builtin_bit_cast(float, o));
}
__device__ __forceinline__ float lane_f32(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// 64-lane maximum, in every lane (call with the whole wave active).  Inside each 16-lane
// row: quad permutes [1,0,3,2] and [2,3,0,1] (xor 1, xor 2), then the half-row mirror
// and the row mirror, which pair lanes whose quads / half-rows already agree; then the
// four rows' maxima are read as scalars.  No LDS-crossbar shuffles (ds_bpermute), which
// made the top-k's serial argmax rounds latency-bound.  max is exact and order-free:
// any pairing gives the same value.
__device__ __forceinline__ float wave_max(float v) {
    v = dpp_fmax<0xB1>(v);   // quad_perm [1,0,3,2]
    v = dpp_fmax<0x4E>(v);   // quad_perm [2,3,0,1]
    v = dpp_fmax<0x141>(v);  // row_half_mirror
    v = dpp_fmax<0x140>(v);  // row_mirror
    return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) v += shfl_xor(v, s);
    return v;
}

// ---------------------------------------------------------------- Q8_0 quantizer
// ggml's scalar quantize_row_q8_0: d = amax/127, q = roundf(x * (1/d)), d stored as
// fp16.  Called by the 32 lanes of a half-wave, one element each (xor width 32).
struct Q8Result {
    int8_t q;
    uint16_t dh;
};

__device__ __forceinline__ Q8Result quant_q8_0_lane32(float x) {
    float amax = fabsf(x);
#pragma unroll
    for (int s = 16; s >= 1; s >>= 1) amax = fmaxf(amax, shfl_xor(amax, s, 32));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    Q8Result r;
    r.q = (int8_t)__builtin_roundf(x * id);
    r.dh = f2h(d);
    return r;
}

// ---------------------------------------------------------------- int8 dots
__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// exp(x) spelled out so the CPU oracle evaluates the same operations: Cody-Waite
// reduction x = n*ln2 + r (ln2 split in a 16-bit head, exact n*head, and a tail),
// e^r by its Taylor series to degree 7 in Horner form with fmaf, scaling by 2^n.
__device__ __forceinline__ float hy_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_inff();
    if (x < -103.97208404541015625f) return 0.0f;
    const float n = __builtin_rintf(x * 1.44269504f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.42860682e-6f, r);
    float p = 1.98412698e-4f;
    p = fmaf(p, r, 1.38888889e-3f);
    p = fmaf(p, r, 8.33333377e-3f);
    p = fmaf(p, r, 4.16666679e-2f);
    p = fmaf(p, r, 1.66666672e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)n);
}

// silu(g) * u as the reference spells it (src/hunyuan_moe_full.cpp:484), with hy_expf
__device__ __forceinline__ float swiglu(float g, float u) {
    return g * (1.0f / (1.0f + hy_expf(-g))) * u;
}

// One round of a wave top-k: the lowest untaken lane (open) holding the largest value
// m of the untaken lanes (v of taken lanes and lanes past the candidates is -inf), so
// equal values go to the lower index (src/hunyuan_moe_full.cpp:67).  A NaN ranks below
// every number: wave_max skips NaN operands, and once only NaNs are left (no open lane
// equals m) the lowest open lane is taken -- an all-NaN row selects 0, 1, 2, ... as the
// reference's insertion top-k does.  `open` must hold at least one lane.
__device__ __forceinline__ int wave_argmax_round(float v, bool open, float& m) {
    m = wave_max(v);
    unsigned long long bal = __ballot(open && v == m);
    if (bal == 0) {
        bal = __ballot(open);
        m = __builtin_nanf("");
    }
    return (int)__builtin_ctzll(bal);
}

// Top-k of one token's logits, one expert per lane (lanes >= E hold none): K rounds
// of wave_argmax_round (K <= E), then p_k = exp(l_k - m) / sum_e exp(l_e - m), m the
// largest logit (NaN skipped; NaN when every logit is), with the denominator summed in
// the 64-lane tree,
// renormalised by max(sum_k p_k, 1e-8) or scaled (src/hunyuan_moe_full.cpp:230-243;
// norm = 0 when K = 1).  Lanes k < K write w_out[k], i_out[k]; p_out (optional) gets
// every expert's probability.
__device__ __forceinline__ void topk_wave(float v_in, int E, int K, int norm, float scale, int lane,
                                          float* w_out, int* i_out, float* p_out = nullptr) {
    float v = lane < E ? v_in : -INFINITY;
    const float orig = v;
    bool open = lane < E;
    float m0 = 0.0f;
    float selv = 0.0f;
    int seli = 0;
    for (int k = 0; k < K; k++) {
        float m;
        const int sel = wave_argmax_round(v, open, m);
        if (k == 0) m0 = m;
        if (lane == k) { selv = m; seli = sel; }
        if (lane == sel) {
            v = -INFINITY;
            open = false;
        }
    }
    // denominator: 64-lane tree of exp(l_e - m) (lanes >= E add 0)
    const float s = wave_sum(lane < E ? hy_expf(orig - m0) : 0.0f);
    // p_k for the lane's own rank k = lane (lanes >= K carry 0)
    const float p = lane < K ? hy_expf(selv - m0) / s : 0.0f;
    // sum_k p_k in rank order (every lane computes the same value)
    float ps = 0.0f;
    for (int k = 0; k < K; k++) ps += __shfl(p, k, WAVE);
    if (ps < 1e-8f) ps = 1e-8f;
    if (lane < K) {
        w_out[lane] = norm ? p / ps : p * scale;
        i_out[lane] = seli;
    }
    if (p_out && lane < E) p_out[lane] = hy_expf(orig - m0) / s;  // the gates the aux loss averages
}

}  // namespace hy
