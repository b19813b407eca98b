/* hy_oracle_attn.c -- CPU restatement of the attention half of a HunyuanImage-3
 * decoder layer.  Test infrastructure only (see hy_oracle_attn.h).  Each function
 * keeps the reference's float operations and their order; built with
 * -ffp-contract=off. */
#include "hy_oracle_attn.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* sequential fp32 dot product, one product then one add per element */
static float seq_dot(const float* a, const float* b, uint32_t n) {
    float s = 0.0f;
    for (uint32_t i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* rotate the interleaved pairs of one head vector by angles ang[d] (cos c[d], sin s[d]) */
static void rotate_pairs(float* v, const float* c, const float* s, uint32_t hd) {
    for (uint32_t d = 0; d < hd / 2; d++) {
        const float a = v[2 * d], b = v[2 * d + 1];
        const float r0 = a * c[d] - b * s[d];
        const float r1 = a * s[d] + b * c[d];
        v[2 * d] = r0;
        v[2 * d + 1] = r1;
    }
}

/* src/rms_norm.cpp:97-152 */
void hyo_rope_f32(float* q, float* k, uint32_t seq, uint32_t n_heads, uint32_t n_kv, uint32_t hd, float theta,
                  const int32_t* positions) {
    float* freq = (float*)malloc(sizeof(float) * (hd / 2));
    float* c = (float*)malloc(sizeof(float) * (hd / 2));
    float* s = (float*)malloc(sizeof(float) * (hd / 2));
    for (uint32_t i = 0; i < hd / 2; i++) freq[i] = 1.0f / powf(theta, (2.0f * (float)i) / (float)hd);
    for (uint32_t t = 0; t < seq; t++) {
        const float pos = positions ? (float)positions[t] : (float)t;
        for (uint32_t d = 0; d < hd / 2; d++) {
            c[d] = cosf(pos * freq[d]);
            s[d] = sinf(pos * freq[d]);
        }
        for (uint32_t h = 0; h < n_heads; h++) rotate_pairs(q + ((size_t)t * n_heads + h) * hd, c, s, hd);
        for (uint32_t h = 0; h < n_kv; h++) rotate_pairs(k + ((size_t)t * n_kv + h) * hd, c, s, hd);
    }
    free(freq);
    free(c);
    free(s);
}

/* src/hunyuan_image_gen.cpp:11-69 */
void hyo_build_2d_rope(uint32_t seq, uint32_t n_elem, uint32_t text_len, uint32_t img_h, uint32_t img_w, float base,
                       float* cos_out, float* sin_out) {
    const uint32_t half = n_elem / 2;
    float* th = (float*)malloc(sizeof(float) * half);
    for (uint32_t i = 0; i < half; i++) th[i] = 1.0f / powf(base, (2.0f * (float)i) / (float)n_elem);
    for (uint32_t p = 0; p < seq; p++) {
        float py, px;
        if (p < text_len) {
            py = (float)p;
            px = (float)p;
        } else {
            const uint32_t idx = p - text_len, row = idx / img_w, col = idx % img_w;
            const float by = (float)text_len + (float)(img_h * img_w - img_h) / 2.0f;
            const float bx = (float)text_len + (float)(img_h * img_w - img_w) / 2.0f;
            py = by + (float)row;
            px = bx + (float)col;
        }
        for (uint32_t d = 0; d < half; d++) {
            const float pos = ((d / 2) % 2 == 0) ? py : px;  /* pairs alternate y, x */
            const float a = pos * th[d];
            const float cv = cosf(a), sv = sinf(a);
            cos_out[(size_t)p * n_elem + 2 * d] = cv;
            cos_out[(size_t)p * n_elem + 2 * d + 1] = cv;
            sin_out[(size_t)p * n_elem + 2 * d] = sv;
            sin_out[(size_t)p * n_elem + 2 * d + 1] = sv;
        }
    }
    free(th);
}

/* src/hunyuan_image_gen.cpp:71-117: the tables hold each pair's value at both of its
 * positions; the rotation reads position 2d */
void hyo_apply_rope_2d_f32(float* q, float* k, const float* cos_t, const float* sin_t, uint32_t n_tokens,
                           uint32_t n_heads, uint32_t n_kv, uint32_t hd) {
    float* c = (float*)malloc(sizeof(float) * (hd / 2));
    float* s = (float*)malloc(sizeof(float) * (hd / 2));
    for (uint32_t t = 0; t < n_tokens; t++) {
        for (uint32_t d = 0; d < hd / 2; d++) {
            c[d] = cos_t[(size_t)t * hd + 2 * d];
            s[d] = sin_t[(size_t)t * hd + 2 * d];
        }
        for (uint32_t h = 0; h < n_heads; h++) rotate_pairs(q + ((size_t)t * n_heads + h) * hd, c, s, hd);
        for (uint32_t h = 0; h < n_kv; h++) rotate_pairs(k + ((size_t)t * n_kv + h) * hd, c, s, hd);
    }
    free(c);
    free(s);
}

/* QKV projection and split into q [T][nh][hd], k, v [T][nkv][hd]
 * (src/attention.cpp:28-81; the cache branch src/hunyuan_extended.cpp:60-88) */
static void project_split(const float* x, const float* qkv_w, uint32_t T, uint32_t H, uint32_t nh, uint32_t nkv,
                          uint32_t hd, float* q, float* k, float* v) {
    const uint32_t nq = nh * hd, nk = nkv * hd;
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t j = 0; j < nq + 2 * nk; j++) {
            const float val = seq_dot(x + (size_t)t * H, qkv_w + (size_t)j * H, H);
            if (j < nq)
                q[(size_t)t * nq + j] = val;
            else if (j < nq + nk)
                k[(size_t)t * nk + (j - nq)] = val;
            else
                v[(size_t)t * nk + (j - nq - nk)] = val;
        }
}

/* per-head RMSNorm.  times_product: x * (rms * w) (the cache branch,
 * src/hunyuan_extended.cpp:99-112); else (x * rms) * w (src/attention.cpp:86-103). */
static void head_norm(float* v, const float* w, uint32_t hd, float eps, int times_product) {
    float ss = 0.0f;
    for (uint32_t d = 0; d < hd; d++) ss += v[d] * v[d];
    const float rms = 1.0f / sqrtf(ss / (float)hd + eps);
    for (uint32_t d = 0; d < hd; d++) v[d] = times_product ? v[d] * (rms * w[d]) : v[d] * rms * w[d];
}

/* softmax-weighted sum of n value rows for one query (src/attention.cpp:121-160):
 * scores = dot * scale, max, expf(s - max), sum, divide, then the sequential sum */
static void attend_one(const float* qh, const float* kbase, const float* vbase, size_t kv_stride, uint32_t n,
                       uint32_t hd, float scale, float* scores, float* out) {
    float mx = -1e30f;
    for (uint32_t j = 0; j < n; j++) {
        scores[j] = seq_dot(qh, kbase + (size_t)j * kv_stride, hd) * scale;
        if (scores[j] > mx) mx = scores[j];
    }
    float sum = 0.0f;
    for (uint32_t j = 0; j < n; j++) {
        scores[j] = expf(scores[j] - mx);
        sum += scores[j];
    }
    for (uint32_t j = 0; j < n; j++) scores[j] /= sum;
    memset(out, 0, sizeof(float) * hd);
    for (uint32_t j = 0; j < n; j++) {
        const float* vh = vbase + (size_t)j * kv_stride;
        for (uint32_t d = 0; d < hd; d++) out[d] += scores[j] * vh[d];
    }
}

/* o_proj: out[t][j] = sequential dot of merged row t with o_w row j (inner length n) */
static void o_project(const float* merged, const float* o_w, uint32_t T, uint32_t H, uint32_t n, float* out) {
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t j = 0; j < H; j++) out[(size_t)t * H + j] = seq_dot(merged + (size_t)t * n, o_w + (size_t)j * n, n);
}

/* src/attention.cpp:10-185 */
void hyo_attention_forward(const float* x, const float* qkv_w, const float* o_w, const float* q_norm,
                           const float* k_norm, uint32_t T, uint32_t H, uint32_t nh, uint32_t nkv, uint32_t hd,
                           float eps, float theta, const int32_t* positions, float* out, float* dbg_q, float* dbg_k,
                           float* dbg_v) {
    const uint32_t nq = nh * hd, nk = nkv * hd, groups = nh / nkv;
    float* q = (float*)malloc(sizeof(float) * (size_t)T * nq);
    float* k = (float*)malloc(sizeof(float) * (size_t)T * nk);
    float* v = (float*)malloc(sizeof(float) * (size_t)T * nk);
    project_split(x, qkv_w, T, H, nh, nkv, hd, q, k, v);
    hyo_rope_f32(q, k, T, nh, nkv, hd, theta, positions);
    for (uint32_t t = 0; t < T; t++) {
        for (uint32_t h = 0; h < nh; h++) head_norm(q + ((size_t)t * nh + h) * hd, q_norm, hd, eps, 0);
        for (uint32_t h = 0; h < nkv; h++) head_norm(k + ((size_t)t * nkv + h) * hd, k_norm, hd, eps, 0);
    }
    if (dbg_q) memcpy(dbg_q, q, sizeof(float) * (size_t)T * nq);
    if (dbg_k) memcpy(dbg_k, k, sizeof(float) * (size_t)T * nk);
    if (dbg_v) memcpy(dbg_v, v, sizeof(float) * (size_t)T * nk);
    const float scale = 1.0f / sqrtf((float)hd);
    float* merged = (float*)malloc(sizeof(float) * (size_t)T * nq);
    float* scores = (float*)malloc(sizeof(float) * (size_t)T);
    for (uint32_t h = 0; h < nh; h++) {
        const uint32_t g = h / groups;
        for (uint32_t t = 0; t < T; t++)  /* causal: keys 0..t */
            attend_one(q + ((size_t)t * nh + h) * hd, k + (size_t)g * hd, v + (size_t)g * hd, nk, t + 1, hd, scale,
                       scores, merged + (size_t)t * nq + (size_t)h * hd);
    }
    o_project(merged, o_w, T, H, nq, out);
    free(q);
    free(k);
    free(v);
    free(merged);
    free(scores);
}

/* src/hunyuan_extended.cpp:52-176 */
int hyo_attention_cached(const float* x, const float* qkv_w, const float* o_w, const float* q_norm,
                         const float* k_norm, uint32_t T, uint32_t H, uint32_t nh, uint32_t nkv, uint32_t hd,
                         float eps, const float* cos_t, const float* sin_t, hyo_kv_cache* cache, float* out) {
    if (cache->cur_len + T > cache->max_len) return -1;
    const uint32_t nq = nh * hd, nk = nkv * hd, groups = nh / nkv;
    float* q = (float*)malloc(sizeof(float) * (size_t)T * nq);
    float* k = (float*)malloc(sizeof(float) * (size_t)T * nk);
    float* v = (float*)malloc(sizeof(float) * (size_t)T * nk);
    project_split(x, qkv_w, T, H, nh, nkv, hd, q, k, v);
    if (cos_t && sin_t) hyo_apply_rope_2d_f32(q, k, cos_t, sin_t, T, nh, nkv, hd);
    for (uint32_t t = 0; t < T; t++) {
        for (uint32_t h = 0; h < nh; h++) head_norm(q + ((size_t)t * nh + h) * hd, q_norm, hd, eps, 1);
        for (uint32_t h = 0; h < nkv; h++) head_norm(k + ((size_t)t * nkv + h) * hd, k_norm, hd, eps, 1);
    }
    const uint32_t pos = cache->cur_len, L = cache->max_len;
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t h = 0; h < nkv; h++) {
            memcpy(cache->k + ((size_t)h * L + pos + t) * hd, k + ((size_t)t * nkv + h) * hd, sizeof(float) * hd);
            memcpy(cache->v + ((size_t)h * L + pos + t) * hd, v + ((size_t)t * nkv + h) * hd, sizeof(float) * hd);
        }
    const uint32_t n = pos + T;
    const float scale = 1.0f / sqrtf((float)hd);
    float* merged = (float*)malloc(sizeof(float) * (size_t)T * nq);
    float* scores = (float*)malloc(sizeof(float) * (size_t)n);
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t h = 0; h < nh; h++) {
            const uint32_t g = h / groups;
            attend_one(q + ((size_t)t * nh + h) * hd, cache->k + (size_t)g * L * hd, cache->v + (size_t)g * L * hd, hd,
                       n, hd, scale, scores, merged + (size_t)t * nq + (size_t)h * hd);
        }
    o_project(merged, o_w, T, H, nq, out);
    cache->cur_len += T;
    free(q);
    free(k);
    free(v);
    free(merged);
    free(scores);
    return 0;
}
