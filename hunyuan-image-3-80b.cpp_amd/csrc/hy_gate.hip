// hy_gate.hip -- GPU kernels behind the reference's dense routing helpers
// (src/hunyuan_moe_full.cpp:56-82 topk_f32, :352-373 einsum_dispatch,
// :379-399 einsum_combine) and RMSNorm with a weight vector (src/rms_norm.cpp:9-33).
// These serve the C++ API that mirrors the reference's header; the fused layer
// forward does not use the dense [T,E,C] representation.
#include "hy_device.hpp"
#include "hy_launch.hpp"

namespace hy {

// Top-k of each row of n values, descending, equal values keep the lower index (the
// insertion order of topk_f32).  One wave per row; lane l owns elements l, l+64, ...
// (n <= 4096, so at most 64 per lane, tracked in a 64-bit taken mask).  k > n pads
// with value 0 / index 0 as the reference's zero-initialised best[] does.  A NaN ranks
// below every number and NaNs are taken in index order (an all-NaN row gives indices
// 0, 1, 2, ... as the reference's insertion does; where NaNs and numbers mix, the
// reference's result depends on their positions and is not reproduced).
__global__ __launch_bounds__(256) void topk_rows_kernel(const float* __restrict__ x, int rows, int n, int k,
                                                        float* __restrict__ vals, int* __restrict__ idx) {
    const int row = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (row >= rows) return;
    const float* xr = x + (size_t)row * n;
    uint64_t taken = 0;
    for (int r = 0; r < k; r++) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        for (int j = 0, i = lane; i < n; j++, i += WAVE) {
            if ((taken >> j) & 1ull) continue;
            const float v = xr[i];
            if (v > bv || (v == bv && i < bi)) {
                bv = v;
                bi = i;
            }
        }
        float m = wave_max(bv);
        int cand = bv == m ? bi : 0x7fffffff;
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) cand = min(cand, __shfl_xor(cand, s, WAVE));
        if (cand == 0x7fffffff && r < n) {
            // only NaNs are left (they rank below every number): the lowest untaken index
            int low = 0x7fffffff;
            for (int j = 0, i = lane; i < n; j++, i += WAVE)
                if (!((taken >> j) & 1ull)) {
                    low = i;
                    break;
                }
#pragma unroll
            for (int s = 32; s >= 1; s >>= 1) low = min(low, __shfl_xor(low, s, WAVE));
            cand = low;
            m = xr[cand];
        }
        if (cand == 0x7fffffff) {  // fewer than k values
            if (lane == 0) {
                vals[(size_t)row * k + r] = 0.0f;
                idx[(size_t)row * k + r] = 0;
            }
            continue;
        }
        if (cand % WAVE == lane) taken |= 1ull << (cand / WAVE);
        if (lane == 0) {
            vals[(size_t)row * k + r] = m;
            idx[(size_t)row * k + r] = cand;
        }
    }
}

hipError_t launch_topk_rows(const float* x, int rows, int n, int k, float* vals, int* idx, hipStream_t s) {
    hipLaunchKernelGGL(topk_rows_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, rows, n, k, vals, idx);
    return hipGetLastError();
}

// disp[e][c][h] = sum over t ascending of x[t][h] where mask[t][e][c] (the reference
// starts from zero and adds in t order).
__global__ void einsum_dispatch_kernel(const float* __restrict__ x, int T, int H, const uint8_t* __restrict__ mask,
                                       int E, int C, float* __restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)E * C * H) return;
    const int h = (int)(idx % H);
    const size_t ec = idx / H;
    float acc = 0.0f;
    for (int t = 0; t < T; t++)
        if (mask[(size_t)t * E * C + ec]) acc = acc + x[(size_t)t * H + h];
    out[idx] = acc;
}

hipError_t launch_einsum_dispatch(const float* x, int T, int H, const uint8_t* mask, int E, int C, float* out,
                                  hipStream_t s) {
    const size_t n = (size_t)E * C * H;
    hipLaunchKernelGGL(einsum_dispatch_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, T, H, mask, E,
                       C, out);
    return hipGetLastError();
}

// out[t][h] = sum over (e, c) ascending, skipping zero weights, of cw[t][e][c] *
// eo[e][c][h] -- mul then add, in the reference's order.
__global__ void einsum_combine_kernel(const float* __restrict__ cw, const float* __restrict__ eo, int T, int H,
                                      int E, int C, float* __restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)T * H) return;
    const int t = (int)(idx / H), h = (int)(idx % H);
    const float* w = cw + (size_t)t * E * C;
    float acc = 0.0f;
    for (int ec = 0; ec < E * C; ec++) {
        const float wv = w[ec];
        if (wv == 0.0f) continue;
        const float p = wv * eo[(size_t)ec * H + h];
        acc = acc + p;
    }
    out[idx] = acc;
}

hipError_t launch_einsum_combine(const float* cw, const float* eo, int T, int H, int E, int C, float* out,
                                 hipStream_t s) {
    const size_t n = (size_t)T * H;
    hipLaunchKernelGGL(einsum_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, cw, eo, T, H, E, C,
                       out);
    return hipGetLastError();
}

// RMSNorm with a weight vector: out = x * rms * w, rms = 1/sqrtf(ss/H + eps), ss in
// the blocked 64-lane order.
__global__ __launch_bounds__(256) void rms_norm_w_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                         int T, int H, float eps, float* __restrict__ out) {
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
    for (int h = lane; h < H; h += WAVE) out[(size_t)row * H + h] = xr[h] * rms * w[h];
}

hipError_t launch_rms_norm_w(const float* x, const float* w, int T, int H, float eps, float* out, hipStream_t s) {
    hipLaunchKernelGGL(rms_norm_w_kernel, dim3((T + 3) / 4), dim3(256), 0, s, x, w, T, H, eps, out);
    return hipGetLastError();
}

}  // namespace hy
