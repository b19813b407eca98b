/*
 * hy_oracle.c -- CPU restatement of the HunyuanImage-3 MoE block.
 *
 * TEST INFRASTRUCTURE ONLY (the checker): used by tests/, the smoke check and
 * the benchmark's CPU-baseline leg, never by the product path.
 *
 * Build: gcc -std=c11 -O2 -ffp-contract=off -fno-fast-math -fopenmp (oracle/Makefile).
 * -ffp-contract=off keeps every "a*b + c" of the reference as two roundings,
 * the way the reference's x86-64 build (no -march, no FMA) evaluates it.
 *
 * Citations are to the reference tree (MaurerAnton/hunyuan-image-3-80b.cpp).
 */
#include "hy_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

void hyo_free(void* p) { free(p); }

void hyo_routing_cfg_default(hyo_routing_cfg* c) {
    /* defaults of MoERoutingConfig, src/hunyuan_moe_full.h:25-47 */
    memset(c, 0, sizeof(*c));
    c->num_experts = 64;
    c->moe_topk = 8;
    c->capacity_factor = 1.0f;
    c->min_capacity = 8;
    c->norm_topk_prob = 1;
    c->routed_scaling_factor = 1.0f;
}

/* ======================================================================
 * fp16 <-> fp32
 * ====================================================================== */

float hyo_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { /* subnormal: m * 2^-24, renormalise */
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            m &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 + 1 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t hyo_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf or nan (quiet) */
        return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) { /* below 2^-14: fp16 subnormal or zero */
        if (ax < 0x33000000u) return sign; /* < 2^-25 (the 2^-25 tie goes to even 0) */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* value / 2^-24 = m * 2^(e-126) */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t mant = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* src/hunyuan_gguf_loader.cpp:19-32: exponent 0 becomes signed zero, exponent 31 is
 * treated as a normal exponent (no inf/nan). */
float hyo_fp16_to_fp32_ref(uint16_t d_half) {
    uint32_t sign = (uint32_t)(d_half & 0x8000u) << 16;
    uint32_t e = (d_half >> 10) & 0x1fu;
    uint32_t mant = d_half & 0x3ffu;
    uint32_t bits = (e == 0) ? sign : (sign | ((e - 15u + 127u) << 23) | (mant << 13));
    float d;
    memcpy(&d, &bits, 4);
    return d;
}

/* ======================================================================
 * GGUF block codecs
 * ====================================================================== */

size_t hyo_type_row_bytes(int type, size_t n) {
    switch (type) {
    case HYO_F32: return n * 4;
    case HYO_F16: return n * 2;
    case HYO_Q8_0: return n / HYO_QK * sizeof(hyo_block_q8_0);
    case HYO_Q4_0: return n / HYO_QK * sizeof(hyo_block_q4_0);
    default: return 0;
    }
}

/* ggml's scalar Q8_0 quantizer (public GGUF format): d = amax/127, q = roundf(x/d)
 * computed as roundf(x * (1/d)); d stored as fp16 (round to nearest even). */
void hyo_quantize_row_q8_0(const float* x, void* vy, size_t n) {
    hyo_block_q8_0* y = (hyo_block_q8_0*)vy;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n > (1u << 20))
#endif
    for (int64_t b = 0; b < (int64_t)(n / HYO_QK); b++) {
        const float* xb = x + b * HYO_QK;
        float amax = 0.0f;
        for (int j = 0; j < HYO_QK; j++) {
            float v = fabsf(xb[j]);
            if (v > amax) amax = v;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[b].d = hyo_fp32_to_fp16(d);
        for (int j = 0; j < HYO_QK; j++) y[b].qs[j] = (int8_t)roundf(xb[j] * id);
    }
}

/* ggml's scalar Q4_0 quantizer: the signed value of largest magnitude maps to -8,
 * d = max/-8, q = min(15, trunc(x/d + 8.5)); element j goes to the low nibble of
 * byte j, element j+16 to the high nibble. */
void hyo_quantize_row_q4_0(const float* x, void* vy, size_t n) {
    hyo_block_q4_0* y = (hyo_block_q4_0*)vy;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n > (1u << 20))
#endif
    for (int64_t b = 0; b < (int64_t)(n / HYO_QK); b++) {
        const float* xb = x + b * HYO_QK;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < HYO_QK; j++) {
            const float v = xb[j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        const float d = max / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[b].d = hyo_fp32_to_fp16(d);
        for (int j = 0; j < HYO_QK / 2; j++) {
            const float x0 = xb[j] * id;
            const float x1 = xb[HYO_QK / 2 + j] * id;
            int q0 = (int)(int8_t)(x0 + 8.5f);
            int q1 = (int)(int8_t)(x1 + 8.5f);
            if (q0 > 15) q0 = 15;
            if (q1 > 15) q1 = 15;
            y[b].qs[j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

void hyo_dequantize_row_q8_0(const void* vx, float* y, size_t n) {
    const hyo_block_q8_0* x = (const hyo_block_q8_0*)vx;
    for (size_t b = 0; b < n / HYO_QK; b++) {
        const float d = hyo_fp16_to_fp32(x[b].d);
        for (int j = 0; j < HYO_QK; j++) y[b * HYO_QK + j] = (float)x[b].qs[j] * d;
    }
}

void hyo_dequantize_row_q4_0(const void* vx, float* y, size_t n) {
    const hyo_block_q4_0* x = (const hyo_block_q4_0*)vx;
    for (size_t b = 0; b < n / HYO_QK; b++) {
        const float d = hyo_fp16_to_fp32(x[b].d);
        for (int j = 0; j < HYO_QK / 2; j++) {
            y[b * HYO_QK + j] = (float)((int)(x[b].qs[j] & 0x0f) - 8) * d;
            y[b * HYO_QK + j + HYO_QK / 2] = (float)((int)(x[b].qs[j] >> 4) - 8) * d;
        }
    }
}

/* src/hunyuan_gguf_loader.cpp:10-39 */
void hyo_dequantize_row_q8_0_ref(const void* src, float* dst, size_t n) {
    const uint8_t* data = (const uint8_t*)src;
    for (size_t b = 0; b < n / 32; b++) {
        uint16_t dh;
        memcpy(&dh, data + b * 34, 2);
        const float d = hyo_fp16_to_fp32_ref(dh);
        const int8_t* q = (const int8_t*)(data + b * 34 + 2);
        for (size_t i = 0; i < 32; i++) dst[b * 32 + i] = (float)q[i] * d;
    }
}

/* src/hunyuan_gguf_loader.cpp:41-72: element i from byte i/2 (low nibble for even i),
 * sign-extended as a 4-bit two's complement value.  Differs from GGUF Q4_0. */
void hyo_dequantize_row_q4_0_ref(const void* src, float* dst, size_t n) {
    const uint8_t* data = (const uint8_t*)src;
    for (size_t b = 0; b < n / 32; b++) {
        uint16_t dh;
        memcpy(&dh, data + b * 18, 2);
        const float d = hyo_fp16_to_fp32_ref(dh);
        const uint8_t* q = data + b * 18 + 2;
        for (size_t i = 0; i < 32; i++) {
            uint8_t val = q[i / 2];
            int8_t qi = (int8_t)((i & 1) ? (val >> 4) : (val & 0xF));
            qi = (qi & 0x8) ? (int8_t)(qi - 16) : qi;
            dst[b * 32 + i] = (float)qi * d;
        }
    }
}

void hyo_dequantize_row(int type, const void* x, float* y, size_t n) {
    switch (type) {
    case HYO_F32: memcpy(y, x, n * 4); break;
    case HYO_F16:
        for (size_t i = 0; i < n; i++) y[i] = hyo_fp16_to_fp32(((const uint16_t*)x)[i]);
        break;
    case HYO_Q8_0: hyo_dequantize_row_q8_0(x, y, n); break;
    case HYO_Q4_0: hyo_dequantize_row_q4_0(x, y, n); break;
    default: break;
    }
}

void hyo_block_dots_q8_0_q8_0(const void* vw, const void* vx, size_t n, int32_t* out) {
    const hyo_block_q8_0* w = (const hyo_block_q8_0*)vw;
    const hyo_block_q8_0* x = (const hyo_block_q8_0*)vx;
    for (size_t b = 0; b < n / HYO_QK; b++) {
        int32_t s = 0;
        for (int j = 0; j < HYO_QK; j++) s += (int32_t)w[b].qs[j] * (int32_t)x[b].qs[j];
        out[b] = s;
    }
}

void hyo_block_dots_q4_0_q8_0(const void* vw, const void* vx, size_t n, int32_t* out) {
    const hyo_block_q4_0* w = (const hyo_block_q4_0*)vw;
    const hyo_block_q8_0* x = (const hyo_block_q8_0*)vx;
    for (size_t b = 0; b < n / HYO_QK; b++) {
        int32_t s0 = 0, s1 = 0;
        for (int j = 0; j < HYO_QK / 2; j++) {
            s0 += ((int32_t)(w[b].qs[j] & 0x0f) - 8) * (int32_t)x[b].qs[j];
            s1 += ((int32_t)(w[b].qs[j] >> 4) - 8) * (int32_t)x[b].qs[j + HYO_QK / 2];
        }
        out[b] = s0 + s1;
    }
}

/* ggml vec_dot_q8_0_q8_0 (generic): sumf += sumi * (dw * dx) */
float hyo_vec_dot_q8_0_q8_0(const void* vw, const void* vx, size_t n) {
    const hyo_block_q8_0* w = (const hyo_block_q8_0*)vw;
    const hyo_block_q8_0* x = (const hyo_block_q8_0*)vx;
    float sumf = 0.0f;
    for (size_t b = 0; b < n / HYO_QK; b++) {
        int32_t s = 0;
        for (int j = 0; j < HYO_QK; j++) s += (int32_t)w[b].qs[j] * (int32_t)x[b].qs[j];
        sumf += (float)s * (hyo_fp16_to_fp32(w[b].d) * hyo_fp16_to_fp32(x[b].d));
    }
    return sumf;
}

/* ggml vec_dot_q4_0_q8_0 (generic): sumf += sumi * dw * dx */
float hyo_vec_dot_q4_0_q8_0(const void* vw, const void* vx, size_t n) {
    const hyo_block_q4_0* w = (const hyo_block_q4_0*)vw;
    const hyo_block_q8_0* x = (const hyo_block_q8_0*)vx;
    float sumf = 0.0f;
    for (size_t b = 0; b < n / HYO_QK; b++) {
        int32_t s0 = 0, s1 = 0;
        for (int j = 0; j < HYO_QK / 2; j++) {
            s0 += ((int32_t)(w[b].qs[j] & 0x0f) - 8) * (int32_t)x[b].qs[j];
            s1 += ((int32_t)(w[b].qs[j] >> 4) - 8) * (int32_t)x[b].qs[j + HYO_QK / 2];
        }
        sumf += (float)(s0 + s1) * hyo_fp16_to_fp32(w[b].d) * hyo_fp16_to_fp32(x[b].d);
    }
    return sumf;
}

/* ======================================================================
 * Synthetic data: counter-based, order independent, identical on the GPU.
 * splitmix64 finaliser as the hash; a normal variate is approximated by the
 * centred sum of four 16-bit uniforms (Irwin-Hall n=4), scaled to unit variance.
 * All steps are integer ops plus one int->float conversion and one float
 * multiply, so the GPU generator reproduces the values bit for bit.
 * ====================================================================== */

static uint64_t hyo_mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t hyo_stream_key(uint64_t seed, uint32_t layer, uint32_t tensor, uint32_t expert) {
    return hyo_mix64(hyo_mix64(seed) ^ (((uint64_t)layer << 40) | ((uint64_t)tensor << 24) |
                                        (uint64_t)expert));
}

#define HYO_NORM_SCALE 2.6428990e-05f /* 1 / sqrt((65536^2 - 1) / 3) */

float hyo_synth_normal(uint64_t key, uint64_t idx, float stddev) {
    uint64_t r = hyo_mix64(key ^ (idx * 0xD1B54A32D192ED03ull));
    int32_t s = (int32_t)(r & 0xffffu) + (int32_t)((r >> 16) & 0xffffu) +
                (int32_t)((r >> 32) & 0xffffu) + (int32_t)(r >> 48) - 131070;
    return (float)s * (stddev * HYO_NORM_SCALE);
}

void hyo_synth_fill(uint64_t key, uint64_t idx0, size_t n, float stddev, float* out) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n > (1u << 20))
#endif
    for (int64_t i = 0; i < (int64_t)n; i++) out[i] = hyo_synth_normal(key, idx0 + (uint64_t)i, stddev);
}

/* ======================================================================
 * (a) Reference semantics
 * ====================================================================== */

/* src/rms_norm.cpp:9-33 */
void hyo_rms_norm_f32(const float* x, const float* w, float* out, uint32_t T, uint32_t H, float eps) {
    for (uint32_t i = 0; i < T; i++) {
        const float* xi = x + (size_t)i * H;
        float* oi = out + (size_t)i * H;
        float sum_sq = 0.0f;
        for (uint32_t j = 0; j < H; j++) sum_sq += xi[j] * xi[j];
        float rms = 1.0f / sqrtf(sum_sq / (float)H + eps);
        for (uint32_t j = 0; j < H; j++) oi[j] = xi[j] * rms * w[j];
    }
}

/* src/rms_norm.cpp:39-91: tmp = x W_gu^T; h = silu(tmp[:, :I]) * tmp[:, I:]; out = h W_d^T */
void hyo_swiglu_ffn_f32(const float* x, const float* gu, const float* dn, float* out,
                        uint32_t n, uint32_t H, uint32_t I) {
    const uint32_t mid2 = 2 * I;
    float* tmp = (float*)malloc((size_t)n * mid2 * sizeof(float));
    float* act = (float*)malloc((size_t)n * I * sizeof(float));
    for (uint32_t i = 0; i < n; i++)
        for (uint32_t j = 0; j < mid2; j++) {
            float s = 0.0f;
            for (uint32_t k = 0; k < H; k++) s += x[(size_t)i * H + k] * gu[(size_t)j * H + k];
            tmp[(size_t)i * mid2 + j] = s;
        }
    for (uint32_t i = 0; i < n; i++)
        for (uint32_t j = 0; j < I; j++) {
            float g = tmp[(size_t)i * mid2 + j];
            float u = tmp[(size_t)i * mid2 + I + j];
            float silu_g = g * (1.0f / (1.0f + expf(-g)));
            act[(size_t)i * I + j] = silu_g * u;
        }
    for (uint32_t i = 0; i < n; i++)
        for (uint32_t j = 0; j < H; j++) {
            float s = 0.0f;
            for (uint32_t k = 0; k < I; k++) s += act[(size_t)i * I + k] * dn[(size_t)j * I + k];
            out[(size_t)i * H + j] = s;
        }
    free(tmp);
    free(act);
}

/* src/hunyuan_moe_full.cpp:41-50 */
void hyo_softmax_f32(float* x, uint32_t n) {
    float max_val = x[0];
    for (uint32_t i = 1; i < n; i++)
        if (x[i] > max_val) max_val = x[i];
    float sum = 0.0f;
    for (uint32_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - max_val);
        sum += x[i];
    }
    for (uint32_t i = 0; i < n; i++) x[i] /= sum;
}

/* src/hunyuan_moe_full.cpp:56-82: insertion top-k, descending; the strict '<' keeps
 * the earlier (lower) index ahead of an equal later value. */
void hyo_topk_f32(const float* x, uint32_t n, uint32_t k, float* vals, int32_t* idx) {
    struct { float v; int32_t i; } best[64];
    uint32_t n_best = 0;
    memset(best, 0, sizeof(best));
    for (uint32_t i = 0; i < n; i++) {
        float val = x[i];
        uint32_t pos = n_best;
        while (pos > 0 && best[pos - 1].v < val) pos--;
        if (pos < k) {
            uint32_t top = n_best < k - 1 ? n_best : k - 1;
            for (uint32_t j = top; j > pos; j--) best[j] = best[j - 1];
            best[pos].v = val;
            best[pos].i = (int32_t)i;
            if (n_best < k) n_best++;
        }
    }
    for (uint32_t i = 0; i < k; i++) {
        vals[i] = best[i].v;
        idx[i] = best[i].i;
    }
}

/* src/hunyuan_moe_full.cpp:88-113 */
void hyo_topkgating_easy(const float* logits, uint32_t T, uint32_t E, uint32_t K,
                         float* w, int32_t* idx) {
    float* probs = (float*)malloc(E * sizeof(float));
    float* vals = (float*)malloc(K * sizeof(float));
    for (uint32_t t = 0; t < T; t++) {
        memcpy(probs, logits + (size_t)t * E, E * sizeof(float));
        hyo_softmax_f32(probs, E);
        hyo_topk_f32(probs, E, K, vals, idx + (size_t)t * K);
        float sum = 0;
        for (uint32_t k = 0; k < K; k++) sum += vals[k];
        if (sum < 1e-8f) sum = 1e-8f;
        for (uint32_t k = 0; k < K; k++) w[(size_t)t * K + k] = vals[k] / sum;
    }
    free(probs);
    free(vals);
}

static uint32_t hyo_max_u32(uint32_t a, uint32_t b) { return a > b ? a : b; }

/* src/hunyuan_moe_full.cpp:119-346, all features.  The capacity is the one this
 * function computes (the reference writes its [T,E,C] arrays with that stride too). */
int hyo_topkgating_full(const float* logits, uint32_t T, const hyo_routing_cfg* cfg, hyo_gate_full* out) {
    const uint32_t E = cfg->num_experts, K = cfg->moe_topk;
    if (K == 0 || K > 64 || K > E) return -1;
    memset(out, 0, sizeof(*out));

    /* Step 1: softmax */
    float* gates = (float*)malloc((size_t)T * E * sizeof(float));
    for (uint32_t t = 0; t < T; t++) {
        memcpy(gates + (size_t)t * E, logits + (size_t)t * E, E * sizeof(float));
        hyo_softmax_f32(gates + (size_t)t * E, E);
    }
    out->router_probs = (float*)malloc((size_t)T * E * sizeof(float));
    memcpy(out->router_probs, gates, (size_t)T * E * sizeof(float));

    /* Step 2: group-limited greedy (:135-166) */
    if (cfg->group_limited_greedy && cfg->n_group > 0 && cfg->topk_group > 0) {
        uint32_t gs = E / cfg->n_group;
        float* gscore = (float*)malloc((size_t)T * cfg->n_group * sizeof(float));
        for (uint32_t t = 0; t < T; t++)
            for (uint32_t g = 0; g < cfg->n_group; g++) {
                float m = 0;
                for (uint32_t e = 0; e < gs; e++)
                    if (gates[(size_t)t * E + g * gs + e] > m) m = gates[(size_t)t * E + g * gs + e];
                gscore[(size_t)t * cfg->n_group + g] = m;
            }
        float* gv = (float*)malloc(cfg->topk_group * sizeof(float));
        int32_t* gi = (int32_t*)malloc(cfg->topk_group * sizeof(int32_t));
        for (uint32_t t = 0; t < T; t++) {
            hyo_topk_f32(gscore + (size_t)t * cfg->n_group, cfg->n_group, cfg->topk_group, gv, gi);
            for (uint32_t g = 0; g < cfg->n_group; g++) {
                int sel = 0;
                for (uint32_t kg = 0; kg < cfg->topk_group; kg++)
                    if (gi[kg] == (int32_t)g) { sel = 1; break; }
                if (!sel) memset(gates + (size_t)t * E + g * gs, 0, gs * sizeof(float));
            }
        }
        free(gscore); free(gv); free(gi);
    }

    /* Step 3: top-k (:168-178) */
    float* tkv = (float*)malloc(K * sizeof(float));
    int32_t* tki = (int32_t*)malloc(K * sizeof(int32_t));
    float* egate = (float*)malloc((size_t)T * K * sizeof(float));
    int32_t* eidx = (int32_t*)malloc((size_t)T * K * sizeof(int32_t));
    for (uint32_t t = 0; t < T; t++) {
        hyo_topk_f32(gates + (size_t)t * E, E, K, tkv, tki);
        memcpy(egate + (size_t)t * K, tkv, K * sizeof(float));
        memcpy(eidx + (size_t)t * K, tki, K * sizeof(int32_t));
    }

    /* Step 4: aux loss (:180-207) */
    float l_aux = 0.0f;
    if (cfg->compute_aux_loss) {
        float* m = (float*)calloc((size_t)T * E, sizeof(float));
        for (uint32_t t = 0; t < T; t++)
            for (uint32_t k = 0; k < K; k++) m[(size_t)t * E + eidx[(size_t)t * K + k]] = 1.0f;
        float* tpe = (float*)calloc(E, sizeof(float));
        float* ppe = (float*)calloc(E, sizeof(float));
        for (uint32_t e = 0; e < E; e++) {
            for (uint32_t t = 0; t < T; t++) {
                tpe[e] += m[(size_t)t * E + e];
                ppe[e] += gates[(size_t)t * E + e];
            }
            tpe[e] /= (float)T;
            ppe[e] /= (float)T;
        }
        for (uint32_t e = 0; e < E; e++) l_aux += tpe[e] * ppe[e];
        l_aux *= (float)(E * E);
        free(m); free(tpe); free(ppe);
    }
    out->aux_loss = l_aux;

    /* Step 5: capacity (:209-227) */
    uint32_t C;
    if (cfg->drop_tokens) {
        C = hyo_max_u32(K, (uint32_t)(cfg->capacity_factor * (float)K * (float)T / (float)E));
        if (C < cfg->min_capacity) C = cfg->min_capacity;
    } else {
        uint32_t* cnt = (uint32_t*)calloc(E, sizeof(uint32_t));
        for (uint32_t t = 0; t < T; t++)
            for (uint32_t k = 0; k < K; k++) cnt[eidx[(size_t)t * K + k]]++;
        C = 0;
        for (uint32_t e = 0; e < E; e++)
            if (cnt[e] > C) C = cnt[e];
        if (C < cfg->min_capacity) C = cfg->min_capacity;
        free(cnt);
    }
    out->capacity = C;

    /* Step 6: probabilities (:229-243) */
    if (cfg->norm_topk_prob && K > 1) {
        for (uint32_t t = 0; t < T; t++) {
            float s = 0;
            for (uint32_t k = 0; k < K; k++) s += gates[(size_t)t * E + eidx[(size_t)t * K + k]];
            if (s < 1e-8f) s = 1e-8f;
            for (uint32_t k = 0; k < K; k++)
                egate[(size_t)t * K + k] = gates[(size_t)t * E + eidx[(size_t)t * K + k]] / s;
        }
    } else {
        for (uint32_t t = 0; t < T; t++)
            for (uint32_t k = 0; k < K; k++)
                egate[(size_t)t * K + k] =
                    gates[(size_t)t * E + eidx[(size_t)t * K + k]] * cfg->routed_scaling_factor;
    }

    /* Step 7: k-major priority -> dispatch mask, combine weights (:245-326) */
    const size_t TKE = (size_t)T * K * E;
    out->exp_counts = (int32_t*)calloc(E, sizeof(int32_t));
    for (uint32_t k = 0; k < K; k++)
        for (uint32_t t = 0; t < T; t++) out->exp_counts[eidx[(size_t)t * K + k]]++;
    /* priority of flat slot i = k*T + t within its expert = number of earlier flat
     * slots routed to the same expert; max over k per (t,e) */
    int32_t* tpmax = (int32_t*)malloc((size_t)T * E * sizeof(int32_t));
    for (size_t i = 0; i < (size_t)T * E; i++) tpmax[i] = -1;
    int32_t* run = (int32_t*)calloc(E, sizeof(int32_t));
    for (uint32_t k = 0; k < K; k++)
        for (uint32_t t = 0; t < T; t++) {
            int32_t e = eidx[(size_t)t * K + k];
            int32_t p = run[e]++;
            if (p > tpmax[(size_t)t * E + e]) tpmax[(size_t)t * E + e] = p;
        }
    (void)TKE;
    out->dispatch_mask = (uint8_t*)calloc((size_t)T * E * C, 1);
    out->combine_weights = (float*)calloc((size_t)T * E * C, sizeof(float));
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t e = 0; e < E; e++) {
            int32_t p = tpmax[(size_t)t * E + e];
            if (p >= 0 && (uint32_t)p < C) out->dispatch_mask[((size_t)t * E + e) * C + p] = 1;
        }
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t e = 0; e < E; e++) {
            float prob = 0;
            for (uint32_t k = 0; k < K; k++)
                if (eidx[(size_t)t * K + k] == (int32_t)e) { prob = egate[(size_t)t * K + k]; break; }
            for (uint32_t c = 0; c < C; c++)
                if (out->dispatch_mask[((size_t)t * E + e) * C + c])
                    out->combine_weights[((size_t)t * E + e) * C + c] = prob;
        }
    float cntc = 0;
    for (size_t i = 0; i < (size_t)T * E * C; i++)
        if (out->dispatch_mask[i]) cntc += 1;
    out->exp_capacity_rate = cntc / (float)(T * K);

    free(gates); free(tkv); free(tki); free(egate); free(eidx); free(tpmax); free(run);
    return 0;
}

void hyo_gate_full_free(hyo_gate_full* g) {
    free(g->dispatch_mask); free(g->combine_weights); free(g->exp_counts); free(g->router_probs);
    memset(g, 0, sizeof(*g));
}

/* src/hunyuan_moe_full.cpp:352-373 */
void hyo_einsum_dispatch(const float* x, uint32_t T, uint32_t H, const uint8_t* mask,
                         uint32_t E, uint32_t C, float* disp) {
    memset(disp, 0, (size_t)E * C * H * sizeof(float));
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t e = 0; e < E; e++)
            for (uint32_t c = 0; c < C; c++)
                if (mask[((size_t)t * E + e) * C + c])
                    for (uint32_t h = 0; h < H; h++)
                        disp[((size_t)e * C + c) * H + h] += x[(size_t)t * H + h];
}

/* src/hunyuan_moe_full.cpp:379-399 (sum in e-ascending, c-ascending order) */
void hyo_einsum_combine(const float* cw, const float* eo, uint32_t T, uint32_t H,
                        uint32_t E, uint32_t C, float* out) {
    memset(out, 0, (size_t)T * H * sizeof(float));
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t e = 0; e < E; e++)
            for (uint32_t c = 0; c < C; c++) {
                float w = cw[((size_t)t * E + e) * C + c];
                if (w == 0) continue;
                for (uint32_t h = 0; h < H; h++)
                    out[(size_t)t * H + h] += w * eo[((size_t)e * C + c) * H + h];
            }
}

/* src/hunyuan_moe_full.cpp:414-423 (twin src/attention.cpp:213-222): one sequential
 * fp32 accumulator per logit, h ascending. */
void hyo_router_logits_seq(const float* x, const float* wr, uint32_t T, uint32_t H, uint32_t E,
                           float* logits) {
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t e = 0; e < E; e++) {
            float s = 0;
            for (uint32_t h = 0; h < H; h++) s += x[(size_t)t * H + h] * wr[(size_t)e * H + h];
            logits[(size_t)t * E + e] = s;
        }
}

/* src/hunyuan_moe_full.cpp:405-516.  Buffers use the gating's own capacity for both
 * the mask and the [E,C,H] arrays (the reference sizes them with K*T/E+1, min 8, and
 * agrees with this whenever the two capacities coincide). */
int hyo_moe_forward_full(const float* x, uint32_t T, uint32_t H, const float* wr,
                         const float* shared_gu, const float* shared_dn,
                         const float* gu_stacked, const float* dn_stacked,
                         uint32_t E, uint32_t I, const hyo_routing_cfg* cfg, float* out) {
    float* logits = (float*)malloc((size_t)T * E * sizeof(float));
    hyo_router_logits_seq(x, wr, T, H, E, logits);
    hyo_routing_cfg c2 = *cfg;
    c2.num_experts = E;
    hyo_gate_full g;
    if (hyo_topkgating_full(logits, T, &c2, &g) != 0) { free(logits); return -1; }
    free(logits);
    const uint32_t C = g.capacity;

    float* shared_out = NULL;
    if (shared_gu && shared_dn) {
        shared_out = (float*)malloc((size_t)T * H * sizeof(float));
        hyo_swiglu_ffn_f32(x, shared_gu, shared_dn, shared_out, T, H, I);
    }
    float* disp = (float*)malloc((size_t)E * C * H * sizeof(float));
    hyo_einsum_dispatch(x, T, H, g.dispatch_mask, E, C, disp);
    float* eo = (float*)calloc((size_t)E * C * H, sizeof(float));
    const uint32_t mid = 2 * I;
    float* guo = (float*)malloc(mid * sizeof(float));
    float* act = (float*)malloc(I * sizeof(float));
    for (uint32_t e = 0; e < E; e++) {
        const float* gu = gu_stacked + (size_t)e * mid * H;
        const float* dn = dn_stacked + (size_t)e * H * I;
        for (uint32_t c = 0; c < C; c++) {
            const float* tok = disp + ((size_t)e * C + c) * H;
            float* ot = eo + ((size_t)e * C + c) * H;
            int has = 0;
            for (uint32_t h = 0; h < H; h++)
                if (tok[h] != 0) { has = 1; break; }
            if (!has) continue;
            for (uint32_t j = 0; j < mid; j++) {
                float s = 0;
                for (uint32_t h = 0; h < H; h++) s += tok[h] * gu[(size_t)j * H + h];
                guo[j] = s;
            }
            for (uint32_t j = 0; j < I; j++) {
                float gg = guo[j], u = guo[I + j];
                float sg = gg * (1.0f / (1.0f + expf(-gg)));
                act[j] = sg * u;
            }
            for (uint32_t j = 0; j < H; j++) {
                float s = 0;
                for (uint32_t k = 0; k < I; k++) s += act[k] * dn[(size_t)j * I + k];
                ot[j] = s;
            }
        }
    }
    free(guo); free(act); free(disp);
    float* comb = (float*)malloc((size_t)T * H * sizeof(float));
    hyo_einsum_combine(g.combine_weights, eo, T, H, E, C, comb);
    free(eo);
    if (shared_out) {
        for (size_t i = 0; i < (size_t)T * H; i++) out[i] = shared_out[i] + comb[i];
        free(shared_out);
    } else {
        memcpy(out, comb, (size_t)T * H * sizeof(float));
    }
    free(comb);
    hyo_gate_full_free(&g);
    return 0;
}

/* src/attention.cpp:191-313 (the twin the built binary runs): same math, top-k in
 * rank order without the 1e-8 clamp, routed outputs summed in rank order.
 * dbg_probs receives the softmax probabilities (the reference copies its
 * router_logits buffer after the in-place softmax, attention.cpp:278). */
int hyo_moe_forward_cpu(const float* x, const float* wr,
                        const float* shared_gu, const float* shared_dn,
                        const float* gu_stacked, const float* dn_stacked,
                        uint32_t T, uint32_t H, uint32_t E, uint32_t I, uint32_t K,
                        float* out, float* dbg_probs, float* dbg_w, int32_t* dbg_idx) {
    if (K == 0 || K > 64 || K > E) return -1;
    float* shared_out = (float*)malloc((size_t)T * H * sizeof(float));
    hyo_swiglu_ffn_f32(x, shared_gu, shared_dn, shared_out, T, H, I);
    float* rl = (float*)malloc((size_t)T * E * sizeof(float));
    hyo_router_logits_seq(x, wr, T, H, E, rl);
    for (uint32_t i = 0; i < T; i++) {
        float* r = rl + (size_t)i * E;
        float m = r[0];
        for (uint32_t e = 1; e < E; e++)
            if (r[e] > m) m = r[e];
        float s = 0.0f;
        for (uint32_t e = 0; e < E; e++) { r[e] = expf(r[e] - m); s += r[e]; }
        for (uint32_t e = 0; e < E; e++) r[e] /= s;
    }
    float* tw = (float*)malloc((size_t)T * K * sizeof(float));
    int32_t* ti = (int32_t*)malloc((size_t)T * K * sizeof(int32_t));
    for (uint32_t i = 0; i < T; i++) {
        struct { float w; int32_t idx; } best[64];
        int nb = 0;
        for (uint32_t e = 0; e < E; e++) {
            float val = rl[(size_t)i * E + e];
            int pos = nb;
            while (pos > 0 && best[pos - 1].w < val) {
                if (pos < (int)K) best[pos] = best[pos - 1];
                pos--;
            }
            if (pos < (int)K) {
                best[pos].w = val;
                best[pos].idx = (int32_t)e;
                if (nb < (int)K) nb++;
            }
        }
        float sw = 0.0f;
        for (uint32_t k = 0; k < K; k++) sw += best[k].w;
        for (uint32_t k = 0; k < K; k++) {
            tw[(size_t)i * K + k] = best[k].w / sw;
            ti[(size_t)i * K + k] = best[k].idx;
        }
    }
    if (dbg_probs) memcpy(dbg_probs, rl, (size_t)T * E * sizeof(float));
    if (dbg_w) memcpy(dbg_w, tw, (size_t)T * K * sizeof(float));
    if (dbg_idx) memcpy(dbg_idx, ti, (size_t)T * K * sizeof(int32_t));
    float* routed = (float*)calloc((size_t)T * H, sizeof(float));
    float* eo = (float*)malloc(H * sizeof(float));
    for (uint32_t i = 0; i < T; i++)
        for (uint32_t k = 0; k < K; k++) {
            int32_t e = ti[(size_t)i * K + k];
            float wgt = tw[(size_t)i * K + k];
            hyo_swiglu_ffn_f32(x + (size_t)i * H, gu_stacked + (size_t)e * 2 * I * H,
                               dn_stacked + (size_t)e * H * I, eo, 1, H, I);
            for (uint32_t j = 0; j < H; j++) routed[(size_t)i * H + j] += wgt * eo[j];
        }
    for (size_t i = 0; i < (size_t)T * H; i++) out[i] = shared_out[i] + routed[i];
    free(shared_out); free(rl); free(tw); free(ti); free(routed); free(eo);
    return 0;
}

/* ======================================================================
 * (b) q semantics: the GPU path's definition
 * ====================================================================== */

/* exp(x) used by the q semantics (SiLU and the routing softmax), spelled out so the
 * CPU and the GPU evaluate the same operations: Cody-Waite reduction
 * x = n*ln2 + r with ln2 split in a 16-bit head (n*head exact) and a tail, e^r by
 * its Taylor series to degree 7 in Horner form with fmaf (truncation < 6e-9
 * relative on |r| <= ln2/2), then scaling by 2^n with ldexpf. */
float hyo_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.97208404541015625f) return 0.0f;
    const float n = rintf(x * 1.44269504f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.42860682e-6f, r);
    float p = 1.98412698e-4f;           /* 1/7! */
    p = fmaf(p, r, 1.38888889e-3f);     /* 1/6! */
    p = fmaf(p, r, 8.33333377e-3f);     /* 1/5! */
    p = fmaf(p, r, 4.16666679e-2f);     /* 1/4! */
    p = fmaf(p, r, 1.66666672e-1f);     /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

/* 64-lane tree sum (lane l holds v[l], lanes >= n hold 0), the wave reduction order. */
static float hyo_tree_sum64(const float* v, uint32_t n) {
    float p[64];
    for (uint32_t l = 0; l < 64; l++) p[l] = l < n ? v[l] : 0.0f;
    for (int s = 32; s >= 1; s >>= 1)
        for (int l = 0; l < s; l++) p[l] = p[l] + p[l + s];
    return p[0];
}

/* One 64-lane blocked dot in the order the GPU router kernel uses. */
static float hyo_blocked_dot(const float* a, const float* b, uint32_t H) {
    float p[64];
    for (int l = 0; l < 64; l++) p[l] = 0.0f;
    for (uint32_t h0 = 0; h0 < H; h0 += 4) {
        const int l = (int)((h0 / 4) % 64);
        for (uint32_t c = 0; c < 4 && h0 + c < H; c++) p[l] = fmaf(a[h0 + c], b[h0 + c], p[l]);
    }
    for (int s = 32; s >= 1; s >>= 1)
        for (int l = 0; l < s; l++) p[l] = p[l] + p[l + s];
    return p[0];
}

void hyo_router_logits_blocked(const float* x, const float* wr, uint32_t T, uint32_t H,
                               uint32_t E, float* logits) {
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t e = 0; e < E; e++)
            logits[(size_t)t * E + e] = hyo_blocked_dot(x + (size_t)t * H, wr + (size_t)e * H, H);
}

/* One token's routing.  Default: top-K on the logits.  Group-limited greedy
 * (n_group > 0 and topk_group > 0): src/hunyuan_moe_full.cpp:135-178 step by step on
 * the q probabilities.  probs (may be NULL) receives the (masked) probabilities. */
/* q-semantics selection (the GPU's wave_argmax_round): k rounds of the largest
 * untaken value, equal values to the lower index; a NaN ranks below every number and
 * NaNs are taken in index order, so an all-NaN row selects 0..k-1 as the reference's
 * insertion top-k does.  For rows without NaN this is topk_f32
 * (src/hunyuan_moe_full.cpp:56-82) exactly.  n <= 64. */
void hyo_select_q(const float* x, uint32_t n, uint32_t k, float* vals, int32_t* idx) {
    uint8_t taken[64] = {0};
    for (uint32_t r = 0; r < k; r++) {
        int best = -1;
        for (uint32_t i = 0; i < n; i++) {
            if (taken[i] || x[i] != x[i]) continue;
            if (best < 0 || x[i] > x[best]) best = (int)i;
        }
        if (best < 0)
            for (uint32_t i = 0; i < n; i++)
                if (!taken[i]) { best = (int)i; break; }
        taken[best] = 1;
        vals[r] = x[best];
        idx[r] = best;
    }
}

static void hyo_route_one(const float* l, uint32_t E, uint32_t K, int norm, float scale, uint32_t n_group,
                          uint32_t topk_group, float* w, int32_t* idx, float* probs) {
    /* norm 1 renormalises only when K > 1 (src/hunyuan_moe_full.cpp:230, the rule of
     * topkgating_full and so of moe_forward_full); norm 2 at every K
     * (src/attention.cpp:268-275, moe_forward_cpu; topkgating_easy :104-108) */
    const int rn = norm == 2 || (norm != 0 && K > 1);
    float m = l[0]; /* the largest logit (NaN skipped; NaN when every logit is) */
    for (uint32_t e = 1; e < E; e++) m = fmaxf(m, l[e]);
    float ex[64];
    for (uint32_t e = 0; e < E; e++) ex[e] = hyo_expf(l[e] - m);
    const float s = hyo_tree_sum64(ex, E);
    float v[64], ps = 0.0f;
    if (n_group == 0 || topk_group == 0) {
        hyo_select_q(l, E, K, v, idx); /* selection on logits, ties -> lower index */
        float p[64];
        for (uint32_t k = 0; k < K; k++) {
            p[k] = hyo_expf(l[idx[k]] - m) / s;
            ps += p[k];
        }
        if (ps < 1e-8f) ps = 1e-8f;
        for (uint32_t k = 0; k < K; k++) w[k] = rn ? p[k] / ps : p[k] * scale;
        if (probs)
            for (uint32_t e = 0; e < E; e++) probs[e] = hyo_expf(l[e] - m) / s;
        return;
    }
    float p[64];
    for (uint32_t e = 0; e < E; e++) p[e] = hyo_expf(l[e] - m) / s;
    /* group scores: max over the group's experts, from 0 (:139-148).  With
     * E / n_group == 0 (n_group > E) no expert is in a group and nothing is masked. */
    const uint32_t gs = E / n_group;
    float gsc[64], gv[64];
    int32_t gi[64];
    for (uint32_t g = 0; gs > 0 && g < n_group; g++) {
        float mx = 0.0f;
        for (uint32_t j = 0; j < gs; j++)
            if (p[g * gs + j] > mx) mx = p[g * gs + j];
        gsc[g] = mx;
    }
    /* the best topk_group groups; experts of the others are set to 0 (:150-165) */
    if (gs > 0) {
        hyo_topk_f32(gsc, n_group, topk_group, gv, gi);
        uint8_t sel[64] = {0};
        for (uint32_t kg = 0; kg < topk_group; kg++) sel[gi[kg]] = 1;
        for (uint32_t g = 0; g < n_group; g++)
            if (!sel[g])
                for (uint32_t j = 0; j < gs; j++) p[g * gs + j] = 0.0f;
    }
    /* top-K of the masked probabilities (:168-178), weights from them (:229-243) */
    hyo_select_q(p, E, K, v, idx);
    for (uint32_t k = 0; k < K; k++) ps += v[k];
    if (ps < 1e-8f) ps = 1e-8f;
    for (uint32_t k = 0; k < K; k++) w[k] = rn ? v[k] / ps : v[k] * scale;
    if (probs) memcpy(probs, p, E * sizeof(float));
}

void hyo_route_topk(const float* logits, uint32_t T, uint32_t E, uint32_t K, int norm,
                    float scale, float* w, int32_t* idx) {
    for (uint32_t t = 0; t < T; t++)
        hyo_route_one(logits + (size_t)t * E, E, K, norm, scale, 0, 0, w + (size_t)t * K, idx + (size_t)t * K,
                      NULL);
}

void hyo_route_topk_groups(const float* logits, uint32_t T, uint32_t E, uint32_t K, int norm, float scale,
                           uint32_t n_group, uint32_t topk_group, float* w, int32_t* idx, float* probs) {
    for (uint32_t t = 0; t < T; t++)
        hyo_route_one(logits + (size_t)t * E, E, K, norm, scale, n_group, topk_group, w + (size_t)t * K,
                      idx + (size_t)t * K, probs ? probs + (size_t)t * E : NULL);
}

/* src/hunyuan_moe_full.cpp:182-206: the per-token expert mask summed as floats is the
 * exact count; each sum runs over tokens in order, the products are rounded before
 * they are added (no contraction in this build). */
float hyo_aux_loss_q(const float* probs, const int32_t* idx, uint32_t T, uint32_t E, uint32_t K) {
    float l = 0.0f;
    for (uint32_t e = 0; e < E; e++) {
        uint32_t n = 0;
        float r = 0.0f;
        for (uint32_t t = 0; t < T; t++) {
            int hit = 0;
            for (uint32_t k = 0; k < K; k++) hit |= idx[(size_t)t * K + k] == (int32_t)e;
            n += (uint32_t)hit;
            r += probs[(size_t)t * E + e];
        }
        const float tpe = (float)n / (float)T, rpe = r / (float)T;
        l += tpe * rpe;
    }
    return l * (float)(E * E);
}

uint32_t hyo_drop_capacity(uint32_t T, uint32_t E, uint32_t K, float capacity_factor, uint32_t min_capacity) {
    uint32_t c = (uint32_t)(capacity_factor * K * T / E);
    if (c < K) c = K;
    if (c < min_capacity) c = min_capacity;
    return c;
}

void hyo_capacity_keep(const int32_t* idx, uint32_t T, uint32_t E, uint32_t K, uint32_t capacity, uint8_t* keep) {
    uint32_t cnt[64] = {0};
    for (uint32_t k = 0; k < K; k++)
        for (uint32_t t = 0; t < T; t++) {
            const int32_t e = idx[(size_t)t * K + k];
            keep[(size_t)t * K + k] = (uint8_t)(e >= 0 && (uint32_t)e < E && cnt[e]++ < capacity);
        }
}

/* y[r] = row r of W (type wt, n columns) . x ; xq is x quantized to Q8_0 (unused for
 * F32).  Quantized rows: exact int32 block dots s_b (ggml's vec_dot_q8_0_q8_0 /
 * vec_dot_q4_0_q8_0 blocks), accumulated over b ascending as
 * acc = fmaf((float)s_b, d_w*d_x, acc).  F32 rows: acc = fmaf(w_k, x_k, acc), k
 * ascending.  (ggml fixes no float order across its ISAs; this is the one the GPU
 * kernels compute.) */
static float hyo_row_dot(int wt, const void* W, size_t r, size_t n, const float* x, const void* xq) {
    const uint8_t* row = (const uint8_t*)W + r * hyo_type_row_bytes(wt, n);
    float acc = 0.0f;
    switch (wt) {
    case HYO_Q8_0: {
        const hyo_block_q8_0* w = (const hyo_block_q8_0*)row;
        const hyo_block_q8_0* q = (const hyo_block_q8_0*)xq;
        for (size_t b = 0; b < n / HYO_QK; b++) {
            int32_t sb = 0;
            for (int j = 0; j < HYO_QK; j++) sb += (int32_t)w[b].qs[j] * (int32_t)q[b].qs[j];
            acc = fmaf((float)sb, hyo_fp16_to_fp32(w[b].d) * hyo_fp16_to_fp32(q[b].d), acc);
        }
        return acc;
    }
    case HYO_Q4_0: {
        const hyo_block_q4_0* w = (const hyo_block_q4_0*)row;
        const hyo_block_q8_0* q = (const hyo_block_q8_0*)xq;
        for (size_t b = 0; b < n / HYO_QK; b++) {
            int32_t sb = 0;
            for (int j = 0; j < HYO_QK / 2; j++) {
                sb += ((int32_t)(w[b].qs[j] & 0x0f) - 8) * (int32_t)q[b].qs[j];
                sb += ((int32_t)(w[b].qs[j] >> 4) - 8) * (int32_t)q[b].qs[j + HYO_QK / 2];
            }
            acc = fmaf((float)sb, hyo_fp16_to_fp32(w[b].d) * hyo_fp16_to_fp32(q[b].d), acc);
        }
        return acc;
    }
    default: {
        const float* wr = (const float*)row;
        for (size_t k = 0; k < n; k++) acc = fmaf(wr[k], x[k], acc);
        return acc;
    }
    }
}

/* One expert FFN on one token: y = W_d (silu(g) * u), g/u = rows [0,I) / [I,2I) of W_gu x. */
static void hyo_expert_q(int wt, const void* gu, const void* dn, uint32_t H, uint32_t I,
                         const float* x, const void* xq, float* y, float* gbuf, float* hbuf, void* hq) {
    for (uint32_t j = 0; j < 2 * I; j++) gbuf[j] = hyo_row_dot(wt, gu, j, H, x, xq);
    for (uint32_t j = 0; j < I; j++) {
        float g = gbuf[j], u = gbuf[I + j];
        hbuf[j] = g * (1.0f / (1.0f + hyo_expf(-g))) * u;
    }
    if (wt != HYO_F32) hyo_quantize_row_q8_0(hbuf, hq, I);
    for (uint32_t r = 0; r < H; r++) y[r] = hyo_row_dot(wt, dn, r, I, hbuf, hq);
}

static int hyo_check_layer(const hyo_qlayer* L) {
    if (!L || L->H == 0 || L->I == 0 || L->E == 0 || L->K == 0) return -1;
    if (L->K > 64 || L->K > L->E || L->E > 64) return -1;
    if (L->H % HYO_QK || L->I % HYO_QK) return -1;
    if (L->wtype != HYO_F32 && L->wtype != HYO_Q8_0 && L->wtype != HYO_Q4_0) return -1;
    if (L->n_group > 0 && L->topk_group > 64) return -1; /* topk_f32's best[64] */
    return 0;
}

/* Routing of one token: logits (blocked order), then hyo_route_one. */
static void hyo_token_route_q(const hyo_qlayer* L, const float* xt, float* lg, float* w, int32_t* idx,
                              float* probs) {
    const uint32_t H = L->H, E = L->E;
    for (uint32_t e = 0; e < E; e++) lg[e] = hyo_blocked_dot(xt, L->router + (size_t)e * H, H);
    hyo_route_one(lg, E, L->K, L->norm_topk_prob, L->routed_scaling_factor, L->n_group, L->topk_group, w, idx,
                  probs);
}

/* The experts of one routed token: out = shared(x) + sum over its kept pairs with a
 * nonzero weight, in ascending expert order (einsum_combine skips w == 0,
 * src/hunyuan_moe_full.cpp:387-397).  keep may be NULL (all kept). */
static void hyo_token_experts_q(const hyo_qlayer* L, const float* xt, float* ot, const float* wl,
                                const int32_t* il, const uint8_t* keep) {
    const uint32_t H = L->H, I = L->I, E = L->E, K = L->K;
    const int wt = L->wtype;
    void* xq = malloc(hyo_type_row_bytes(HYO_Q8_0, H));
    void* hq = malloc(hyo_type_row_bytes(HYO_Q8_0, I));
    float* gbuf = (float*)malloc(2 * (size_t)I * sizeof(float));
    float* hbuf = (float*)malloc((size_t)I * sizeof(float));
    float* y = (float*)malloc((size_t)H * sizeof(float));
    float* comb = (float*)calloc(H, sizeof(float));
    if (wt != HYO_F32) hyo_quantize_row_q8_0(xt, xq, H);
    const size_t gu_bytes = hyo_type_row_bytes(wt, H) * 2 * I;
    const size_t dn_bytes = hyo_type_row_bytes(wt, I) * H;
    /* routed experts, summed in ascending expert order (einsum_combine order) */
    for (uint32_t e = 0; e < E; e++) {
        int k = -1;
        for (uint32_t j = 0; j < K; j++)
            if (il[j] == (int32_t)e) { k = (int)j; break; }
        if (k < 0 || (keep && !keep[k]) || wl[k] == 0.0f) continue;
        hyo_expert_q(wt, (const uint8_t*)L->gu + e * gu_bytes, (const uint8_t*)L->dn + e * dn_bytes,
                     H, I, xt, xq, y, gbuf, hbuf, hq);
        for (uint32_t r = 0; r < H; r++) comb[r] = fmaf(wl[k], y[r], comb[r]);
    }
    if (L->shared_gu && L->shared_dn) {
        hyo_expert_q(wt, L->shared_gu, L->shared_dn, H, I, xt, xq, y, gbuf, hbuf, hq);
        for (uint32_t r = 0; r < H; r++) ot[r] = y[r] + comb[r];
    } else {
        memcpy(ot, comb, H * sizeof(float));
    }
    free(xq); free(hq); free(gbuf); free(hbuf); free(y); free(comb);
}

static void hyo_token_q(const hyo_qlayer* L, const float* xt, float* ot, float* lg, float* w,
                        int32_t* idx) {
    float lgl[64], wl[64];
    int32_t il[64];
    hyo_token_route_q(L, xt, lg ? lg : lgl, wl, il, NULL);
    if (w) memcpy(w, wl, L->K * sizeof(float));
    if (idx) memcpy(idx, il, L->K * sizeof(int32_t));
    hyo_token_experts_q(L, xt, ot, wl, il, NULL);
}

int hyo_moe_route_q(const hyo_qlayer* L, const float* x, uint32_t T, float* logits, float* w, int32_t* idx,
                    float* probs, uint8_t* keep, int nthreads) {
    if (hyo_check_layer(L) || !w || !idx) return -1;
    const uint32_t E = L->E, K = L->K;
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t t = 0; t < (int64_t)T; t++) {
        float lgl[64];
        hyo_token_route_q(L, x + (size_t)t * L->H, logits ? logits + (size_t)t * E : lgl, w + (size_t)t * K,
                          idx + (size_t)t * K, probs ? probs + (size_t)t * E : NULL);
    }
    (void)nthreads;
    if (keep) {
        if (L->capacity > 0)
            hyo_capacity_keep(idx, T, E, K, L->capacity, keep);
        else
            memset(keep, 1, (size_t)T * K);
    }
    return 0;
}

/* The layer with a capacity: the whole batch is routed first (a pair's slot depends
 * on the earlier tokens), then the tokens' experts.  rows NULL: every token. */
static int hyo_forward_q_capacity(const hyo_qlayer* L, const float* x, uint32_t T, const uint32_t* rows,
                                  uint32_t n_rows, float* out, float* dbg_logits, float* dbg_w, int32_t* dbg_idx,
                                  int nthreads) {
    const uint32_t K = L->K;
    float* w = (float*)malloc((size_t)T * K * sizeof(float));
    int32_t* idx = (int32_t*)malloc((size_t)T * K * sizeof(int32_t));
    uint8_t* keep = (uint8_t*)malloc((size_t)T * K);
    int rc = hyo_moe_route_q(L, x, T, dbg_logits, w, idx, NULL, keep, nthreads);
    if (rc == 0) {
        const int64_t n = rows ? (int64_t)n_rows : (int64_t)T;
#ifdef _OPENMP
        if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
#endif
        for (int64_t i = 0; i < n; i++) {
            const size_t t = rows ? rows[i] : (size_t)i;
            hyo_token_experts_q(L, x + t * L->H, out + (size_t)i * L->H, w + t * K, idx + t * K, keep + t * K);
        }
        if (dbg_w) memcpy(dbg_w, w, (size_t)T * K * sizeof(float));
        if (dbg_idx) memcpy(dbg_idx, idx, (size_t)T * K * sizeof(int32_t));
    }
    free(w); free(idx); free(keep);
    (void)nthreads;
    return rc;
}

int hyo_moe_forward_q_rows(const hyo_qlayer* L, const float* x, uint32_t T,
                           const uint32_t* rows, uint32_t n_rows, float* out, int nthreads) {
    if (hyo_check_layer(L)) return -1;
    for (uint32_t i = 0; i < n_rows; i++)
        if (rows[i] >= T) return -1;
    if (L->capacity > 0) return hyo_forward_q_capacity(L, x, T, rows, n_rows, out, NULL, NULL, NULL, nthreads);
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
#endif
    for (int64_t i = 0; i < (int64_t)n_rows; i++)
        hyo_token_q(L, x + (size_t)rows[i] * L->H, out + (size_t)i * L->H, NULL, NULL, NULL);
    (void)nthreads;
    return 0;
}

int hyo_moe_forward_q(const hyo_qlayer* L, const float* x, uint32_t T, float* out,
                      float* dbg_logits, float* dbg_w, int32_t* dbg_idx, int nthreads) {
    if (hyo_check_layer(L)) return -1;
    if (L->capacity > 0)
        return hyo_forward_q_capacity(L, x, T, NULL, 0, out, dbg_logits, dbg_w, dbg_idx, nthreads);
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
#endif
    for (int64_t t = 0; t < (int64_t)T; t++)
        hyo_token_q(L, x + (size_t)t * L->H, out + (size_t)t * L->H,
                    dbg_logits ? dbg_logits + (size_t)t * L->E : NULL,
                    dbg_w ? dbg_w + (size_t)t * L->K : NULL,
                    dbg_idx ? dbg_idx + (size_t)t * L->K : NULL);
    (void)nthreads;
    return 0;
}

/* RMSNorm, sum of squares in the 64-lane blocked fmaf order shared with the GPU
 * kernel, then x * (1/sqrtf(ss/H + eps)) * w as src/rms_norm.cpp:26-30 (w NULL: unit
 * weight, the last multiply dropped). */
static void hyo_rms_norm_blocked(const float* x, const float* w, float* out, uint32_t H, float eps) {
    float ss = hyo_blocked_dot(x, x, H);
    float rms = 1.0f / sqrtf(ss / (float)H + eps);
    if (w)
        for (uint32_t j = 0; j < H; j++) out[j] = x[j] * rms * w[j];
    else
        for (uint32_t j = 0; j < H; j++) out[j] = x[j] * rms;
}

/* The decoder layer's MoE half (src/decoder_layer.cpp:33-42), stacked: per layer
 * h <- h + MoE(RMSNorm(h) * w_l), w_l = norm_w[l] (NULL array or entry: unit). */
int hyo_moe_stack_qw(const hyo_qlayer* layers, const float* const* norm_w, uint32_t n_layers, const float* x,
                     uint32_t T, float eps, float* out, int nthreads) {
    if (n_layers == 0) return -1;
    const uint32_t H = layers[0].H;
    for (uint32_t l = 0; l < n_layers; l++)
        if (hyo_check_layer(&layers[l]) || layers[l].H != H) return -1;
    float* cur = (float*)malloc((size_t)T * H * sizeof(float));
    float* xn = (float*)malloc((size_t)T * H * sizeof(float));
    float* y = (float*)malloc((size_t)T * H * sizeof(float));
    memcpy(cur, x, (size_t)T * H * sizeof(float));
    for (uint32_t l = 0; l < n_layers; l++) {
        const float* w = norm_w ? norm_w[l] : NULL;
        for (uint32_t t = 0; t < T; t++)
            hyo_rms_norm_blocked(cur + (size_t)t * H, w, xn + (size_t)t * H, H, eps);
        hyo_moe_forward_q(&layers[l], xn, T, y, NULL, NULL, NULL, nthreads);
        for (size_t i = 0; i < (size_t)T * H; i++) cur[i] = cur[i] + y[i];
    }
    memcpy(out, cur, (size_t)T * H * sizeof(float));
    free(cur); free(xn); free(y);
    return 0;
}

/* RMSNorm in the blocked order on T rows (the GPU's rms_norm kernels' restatement). */
void hyo_rms_norm_blocked_rows(const float* x, const float* w, float* out, uint32_t T, uint32_t H, float eps) {
    for (uint32_t t = 0; t < T; t++) hyo_rms_norm_blocked(x + (size_t)t * H, w, out + (size_t)t * H, H, eps);
}

int hyo_moe_stack_q(const hyo_qlayer* layers, uint32_t n_layers, const float* x, uint32_t T,
                    float eps, float* out, int nthreads) {
    return hyo_moe_stack_qw(layers, NULL, n_layers, x, T, eps, out, nthreads);
}
