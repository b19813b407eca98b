// hy_ffn.hip -- expert products on the VALU path (small token counts per expert:
// decode batches), plus the combine kernel.
//
// Work item of the "up" kernel: (tile, slab g).  A tile is up to NT tokens routed to
// one expert (or NT consecutive tokens for the shared expert); a slab is 64 packed
// gate_up rows = 32 SiLU rows + the matching 32 linear rows, i.e. one 32-wide block
// of h.  The kernel streams the slab's weights once, forms g and u for the tile's
// tokens, applies h = silu(g) * u (src/hunyuan_moe_full.cpp:479-486) and quantizes h
// to Q8_0 for the down product (ggml quantizes src1 of every quantized matmul).
//
// The "down" kernel's work item is (tile, 64 output rows).  Routed tiles write
// y[pair][row]; shared tiles fuse the combine:
//   out[t] = residual[t] + ( y_shared[t] + sum_{e ascending} w_e * y_e[t] )
// (src/hunyuan_moe_full.cpp:503-515, einsum_combine order :387-397).
//
// Inside a wave, 8 lanes share one weight row: lane s takes blocks s, s+8, ... so the
// 8 lanes read 8 consecutive blocks (256 B for Q8_0) of a row; 8 rows are in flight
// per wave.  Per block the int8 dot is exact (v_dot4_i32_i8) and rescaled in fp32.
#include "hy_device.hpp"
#include "hy_launch.hpp"
#include "hy_layout.hpp"

namespace hy {

constexpr int FFN_THREADS = 256;
constexpr int FFN_ROWS = 64;  // rows per work item

// exact int dot of one Q8_0 weight block with one Q8_0 activation block
__device__ __forceinline__ int dot_q8_block(const int4 w0, const int4 w1, const int4 a0, const int4 a1) {
    int s = dot4(w0.x, a0.x, 0);
    s = dot4(w0.y, a0.y, s);
    s = dot4(w0.z, a0.z, s);
    s = dot4(w0.w, a0.w, s);
    s = dot4(w1.x, a1.x, s);
    s = dot4(w1.y, a1.y, s);
    s = dot4(w1.z, a1.z, s);
    s = dot4(w1.w, a1.w, s);
    return s;
}

// exact int dot of one Q4_0 weight block (16 B, GGUF nibble order) with a Q8_0
// activation block whose int sum is asum: sum (n-8)*x = sum n*x - 8*sum x.
__device__ __forceinline__ int dot_q4_block(const int4 w, const int4 a0, const int4 a1, int asum) {
    const int m = 0x0F0F0F0F;
    int s = dot4(w.x & m, a0.x, 0);
    s = dot4(w.y & m, a0.y, s);
    s = dot4(w.z & m, a0.z, s);
    s = dot4(w.w & m, a0.w, s);
    s = dot4((w.x >> 4) & m, a1.x, s);
    s = dot4((w.y >> 4) & m, a1.y, s);
    s = dot4((w.z >> 4) & m, a1.z, s);
    s = dot4((w.w >> 4) & m, a1.w, s);
    return s - 8 * asum;
}

__device__ int block_dot_q8(const uint8_t* w, const uint8_t* x) {
    const int4* wv = reinterpret_cast<const int4*>(w);
    const int4* xv = reinterpret_cast<const int4*>(x);
    return dot_q8_block(wv[0], wv[1], xv[0], xv[1]);
}

struct TileInfo {
    int e, start, n;
    bool shared;
};

__device__ __forceinline__ bool load_tile(const Routing& R, int tile, int limit_meta_idx, int E, TileInfo& ti) {
    if (tile >= R.meta[limit_meta_idx]) return false;
    ti.e = R.tile_e[tile];
    ti.start = R.tile_start[tile];
    ti.n = R.tile_n[tile];
    ti.shared = ti.e == E;
    return true;
}

// ---------------------------------------------------------------------------- up
template <int WT, int NT>
__global__ __launch_bounds__(FFN_THREADS) void ffn_up_valu_kernel(
    MatView W, Routing R, ActQ X, const float* __restrict__ xf, int T, int H, int I, int E, int K,
    int8_t* __restrict__ hq, float* __restrict__ hd, int* __restrict__ hs, float* __restrict__ hf) {
    extern __shared__ __align__(16) uint8_t smem[];
    TileInfo ti;
    if (!load_tile(R, blockIdx.x, 1, E, ti)) return;
    const int g = blockIdx.y;
    const int nb = H / QK;
    __shared__ int tok_s[NT], slot_s[NT];
    __shared__ float res[FFN_ROWS][NT];
    if (threadIdx.x < NT) {
        const int i = threadIdx.x;
        int tok = 0, slot = 0;
        if (i < ti.n) {
            if (ti.shared) {
                tok = ti.start + i;
                slot = T * K + tok;
            } else {
                slot = R.off[ti.e] + ti.start + i;
                tok = R.srt_tok[slot];
            }
        }
        tok_s[i] = tok;
        slot_s[i] = slot;
    }
    __syncthreads();
    // stage the tile's quantized activations: NT rows of H int8, scales, sums
    int8_t* xs_l = reinterpret_cast<int8_t*>(smem);
    float* xd_l = reinterpret_cast<float*>(smem + (size_t)NT * H);
    int* xsum_l = reinterpret_cast<int*>(smem + (size_t)NT * H + (size_t)NT * nb * 4);
    if (WT != HY_TYPE_F32) {
        const int vec_per_row = H / 16;
        for (int v = threadIdx.x; v < NT * vec_per_row; v += FFN_THREADS) {
            const int i = v / vec_per_row, c = v % vec_per_row;
            int4 val = make_int4(0, 0, 0, 0);
            if (i < ti.n) val = reinterpret_cast<const int4*>(X.q + (size_t)tok_s[i] * H)[c];
            reinterpret_cast<int4*>(xs_l + (size_t)i * H)[c] = val;
        }
        for (int v = threadIdx.x; v < NT * nb; v += FFN_THREADS) {
            const int i = v / nb, b = v % nb;
            xd_l[v] = i < ti.n ? X.d[(size_t)tok_s[i] * nb + b] : 0.0f;
            if (WT == HY_TYPE_Q4_0) xsum_l[v] = i < ti.n ? X.s[(size_t)tok_s[i] * nb + b] : 0;
        }
    }
    __syncthreads();

    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int sub = lane % 8;
    const int e = ti.e;
    for (int pass = 0; pass < 2; pass++) {
        const int lrow = wave * 16 + pass * 8 + lane / 8;  // 0..63 within the slab
        const int prow = g * FFN_ROWS + lrow;               // packed gate_up row
        float acc[NT];
#pragma unroll
        for (int i = 0; i < NT; i++) acc[i] = 0.0f;
        if (WT == HY_TYPE_Q8_0) {
            const uint8_t* wrow = W.qs + (size_t)e * W.qs_stride + (size_t)prow * H;
            const uint16_t* srow = W.sc + (size_t)e * W.sc_stride + (size_t)prow * nb;
            for (int b = sub; b < nb; b += 8) {
                const int4 w0 = reinterpret_cast<const int4*>(wrow + b * QK)[0];
                const int4 w1 = reinterpret_cast<const int4*>(wrow + b * QK)[1];
                const float dw = h2f(srow[b]);
#pragma unroll
                for (int i = 0; i < NT; i++) {
                    if (i < ti.n) {
                        const int4* xb = reinterpret_cast<const int4*>(xs_l + (size_t)i * H + b * QK);
                        const int s = dot_q8_block(w0, w1, xb[0], xb[1]);
                        acc[i] = fmaf((float)s, dw * xd_l[i * nb + b], acc[i]);
                    }
                }
            }
        } else if (WT == HY_TYPE_Q4_0) {
            const uint8_t* wrow = W.qs + (size_t)e * W.qs_stride + (size_t)prow * (H / 2);
            const uint16_t* srow = W.sc + (size_t)e * W.sc_stride + (size_t)prow * nb;
            for (int b = sub; b < nb; b += 8) {
                const int4 w = reinterpret_cast<const int4*>(wrow + b * 16)[0];
                const float dw = h2f(srow[b]);
#pragma unroll
                for (int i = 0; i < NT; i++) {
                    if (i < ti.n) {
                        const int4* xb = reinterpret_cast<const int4*>(xs_l + (size_t)i * H + b * QK);
                        const int s = dot_q4_block(w, xb[0], xb[1], xsum_l[i * nb + b]);
                        acc[i] = fmaf((float)s, dw * xd_l[i * nb + b], acc[i]);
                    }
                }
            }
        } else {
            const float* wrow = reinterpret_cast<const float*>(W.qs + (size_t)e * W.qs_stride) + (size_t)prow * H;
            for (int b = sub; b < nb; b += 8) {
                float4 wv[8];
#pragma unroll
                for (int c = 0; c < 8; c++) wv[c] = reinterpret_cast<const float4*>(wrow + b * QK)[c];
#pragma unroll
                for (int i = 0; i < NT; i++) {
                    if (i < ti.n) {
                        const float4* xv = reinterpret_cast<const float4*>(xf + (size_t)tok_s[i] * H + b * QK);
                        float a = acc[i];
#pragma unroll
                        for (int c = 0; c < 8; c++) {
                            const float4 xx = xv[c];
                            a = fmaf(wv[c].x, xx.x, a);
                            a = fmaf(wv[c].y, xx.y, a);
                            a = fmaf(wv[c].z, xx.z, a);
                            a = fmaf(wv[c].w, xx.w, a);
                        }
                        acc[i] = a;
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NT; i++) {
            float v = acc[i];
            v += shfl_xor(v, 4);
            v += shfl_xor(v, 2);
            v += shfl_xor(v, 1);
            if (sub == 0) res[lrow][i] = v;
        }
    }
    __syncthreads();
    // SwiGLU + Q8_0 quantization of h: half-wave per token, lane j = column
    const int nb_i = I / QK;
    for (int i = threadIdx.x / 32; i < NT; i += FFN_THREADS / 32) {
        if (i >= ti.n) break;  // uniform across the half-wave
        const int j = threadIdx.x % 32;
        const float h = swiglu(res[j][i], res[32 + j][i]);
        const size_t slot = (size_t)slot_s[i];
        if (WT == HY_TYPE_F32) {
            hf[slot * I + (size_t)g * QK + j] = h;
        } else {
            const Q8Result r = quant_q8_0_lane32(h);
            int s = r.q;
#pragma unroll
            for (int m = 16; m >= 1; m >>= 1) s += shfl_xor(s, m, 32);
            hq[slot * I + (size_t)g * QK + j] = r.q;
            if (j == 0) {
                hd[slot * nb_i + g] = h2f(r.dh);
                hs[slot * nb_i + g] = s;
            }
        }
    }
}

// ---------------------------------------------------------------------------- down
// mode 0: routed tiles -> y[pair][row].  mode 1: shared tiles + combine -> out.
template <int WT, int NT>
__global__ __launch_bounds__(FFN_THREADS) void ffn_down_valu_kernel(
    MatView W, Routing R, const int8_t* __restrict__ hq, const float* __restrict__ hd, const int* __restrict__ hs,
    const float* __restrict__ hf, int T, int H, int I, int E, int K, int mode, float* __restrict__ y,
    const float* __restrict__ resid, float* __restrict__ out) {
    extern __shared__ __align__(16) uint8_t smem[];
    TileInfo ti;
    const int tile = (mode == 0) ? (int)blockIdx.x : R.meta[0] + (int)blockIdx.x;
    if (!load_tile(R, tile, mode == 0 ? 0 : 1, E, ti)) return;
    const int r0 = blockIdx.y * FFN_ROWS;
    const int nb = I / QK;
    __shared__ int tok_s[NT], slot_s[NT];
    __shared__ float res[FFN_ROWS][NT];
    if (threadIdx.x < NT) {
        const int i = threadIdx.x;
        int tok = 0, slot = 0;
        if (i < ti.n) {
            if (ti.shared) {
                tok = ti.start + i;
                slot = T * K + tok;
            } else {
                slot = R.off[ti.e] + ti.start + i;
                tok = R.srt_tok[slot];
            }
        }
        tok_s[i] = tok;
        slot_s[i] = slot;
    }
    __syncthreads();
    int8_t* hs_l = reinterpret_cast<int8_t*>(smem);
    float* hd_l = reinterpret_cast<float*>(smem + (size_t)NT * I);
    int* hsum_l = reinterpret_cast<int*>(smem + (size_t)NT * I + (size_t)NT * nb * 4);
    if (WT != HY_TYPE_F32) {
        const int vec_per_row = I / 16;
        for (int v = threadIdx.x; v < NT * vec_per_row; v += FFN_THREADS) {
            const int i = v / vec_per_row, c = v % vec_per_row;
            int4 val = make_int4(0, 0, 0, 0);
            if (i < ti.n) val = reinterpret_cast<const int4*>(hq + (size_t)slot_s[i] * I)[c];
            reinterpret_cast<int4*>(hs_l + (size_t)i * I)[c] = val;
        }
        for (int v = threadIdx.x; v < NT * nb; v += FFN_THREADS) {
            const int i = v / nb, b = v % nb;
            hd_l[v] = i < ti.n ? hd[(size_t)slot_s[i] * nb + b] : 0.0f;
            if (WT == HY_TYPE_Q4_0) hsum_l[v] = i < ti.n ? hs[(size_t)slot_s[i] * nb + b] : 0;
        }
    }
    __syncthreads();
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int sub = lane % 8;
    const int e = ti.e;
    for (int pass = 0; pass < 2; pass++) {
        const int lrow = wave * 16 + pass * 8 + lane / 8;
        const int row = r0 + lrow;
        float acc[NT];
#pragma unroll
        for (int i = 0; i < NT; i++) acc[i] = 0.0f;
        if (row < H) {
            if (WT == HY_TYPE_Q8_0) {
                const uint8_t* wrow = W.qs + (size_t)e * W.qs_stride + (size_t)row * I;
                const uint16_t* srow = W.sc + (size_t)e * W.sc_stride + (size_t)row * nb;
                for (int b = sub; b < nb; b += 8) {
                    const int4 w0 = reinterpret_cast<const int4*>(wrow + b * QK)[0];
                    const int4 w1 = reinterpret_cast<const int4*>(wrow + b * QK)[1];
                    const float dw = h2f(srow[b]);
#pragma unroll
                    for (int i = 0; i < NT; i++) {
                        if (i < ti.n) {
                            const int4* xb = reinterpret_cast<const int4*>(hs_l + (size_t)i * I + b * QK);
                            const int s = dot_q8_block(w0, w1, xb[0], xb[1]);
                            acc[i] = fmaf((float)s, dw * hd_l[i * nb + b], acc[i]);
                        }
                    }
                }
            } else if (WT == HY_TYPE_Q4_0) {
                const uint8_t* wrow = W.qs + (size_t)e * W.qs_stride + (size_t)row * (I / 2);
                const uint16_t* srow = W.sc + (size_t)e * W.sc_stride + (size_t)row * nb;
                for (int b = sub; b < nb; b += 8) {
                    const int4 w = reinterpret_cast<const int4*>(wrow + b * 16)[0];
                    const float dw = h2f(srow[b]);
#pragma unroll
                    for (int i = 0; i < NT; i++) {
                        if (i < ti.n) {
                            const int4* xb = reinterpret_cast<const int4*>(hs_l + (size_t)i * I + b * QK);
                            const int s = dot_q4_block(w, xb[0], xb[1], hsum_l[i * nb + b]);
                            acc[i] = fmaf((float)s, dw * hd_l[i * nb + b], acc[i]);
                        }
                    }
                }
            } else {
                const float* wrow = reinterpret_cast<const float*>(W.qs + (size_t)e * W.qs_stride) + (size_t)row * I;
                for (int b = sub; b < nb; b += 8) {
                    float4 wv[8];
#pragma unroll
                    for (int c = 0; c < 8; c++) wv[c] = reinterpret_cast<const float4*>(wrow + b * QK)[c];
#pragma unroll
                    for (int i = 0; i < NT; i++) {
                        if (i < ti.n) {
                            const float4* xv = reinterpret_cast<const float4*>(hf + (size_t)slot_s[i] * I + b * QK);
                            float a = acc[i];
#pragma unroll
                            for (int c = 0; c < 8; c++) {
                                const float4 xx = xv[c];
                                a = fmaf(wv[c].x, xx.x, a);
                                a = fmaf(wv[c].y, xx.y, a);
                                a = fmaf(wv[c].z, xx.z, a);
                                a = fmaf(wv[c].w, xx.w, a);
                            }
                            acc[i] = a;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NT; i++) {
            float v = acc[i];
            v += shfl_xor(v, 4);
            v += shfl_xor(v, 2);
            v += shfl_xor(v, 1);
            if (sub == 0) res[lrow][i] = v;
        }
    }
    __syncthreads();
    for (int v = threadIdx.x; v < NT * FFN_ROWS; v += FFN_THREADS) {
        const int i = v / FFN_ROWS, lr = v % FFN_ROWS;
        const int row = r0 + lr;
        if (i >= ti.n || row >= H) continue;
        const float val = res[lr][i];
        if (mode == 0) {
            y[(size_t)slot_s[i] * H + row] = val;
        } else {
            const int t = tok_s[i];
            float comb = 0.0f;
            for (int k = 0; k < K; k++)
                comb = fmaf(R.comb_w[t * K + k], y[(size_t)R.comb_pos[t * K + k] * H + row], comb);
            const float o = val + comb;
            out[(size_t)t * H + row] = resid ? resid[(size_t)t * H + row] + o : o;
        }
    }
}

// combine without a shared expert: out[t] = residual[t] + sum_{e ascending} w_e y_e[t]
__global__ __launch_bounds__(256) void combine_kernel(Routing R, const float* __restrict__ y, int T, int H, int K,
                                                      const float* __restrict__ resid, float* __restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)T * H) return;
    const int t = (int)(idx / H), row = (int)(idx % H);
    float comb = 0.0f;
    for (int k = 0; k < K; k++) comb = fmaf(R.comb_w[t * K + k], y[(size_t)R.comb_pos[t * K + k] * H + row], comb);
    out[idx] = resid ? resid[idx] + comb : comb;
}

// ---------------------------------------------------------------------------- launchers
size_t ffn_up_smem(int wtype, int NT, int H) {
    if (wtype == HY_TYPE_F32) return 16;
    return (size_t)NT * H + (size_t)NT * (H / QK) * 8;
}
size_t ffn_down_smem(int wtype, int NT, int I) {
    if (wtype == HY_TYPE_F32) return 16;
    return (size_t)NT * I + (size_t)NT * (I / QK) * 8;
}

template <int NT>
static hipError_t up_dispatch(int wtype, dim3 grid, size_t smem, hipStream_t s, const MatView& W, const Routing& R,
                              const ActQ& X, const float* xf, int T, int H, int I, int E, int K, int8_t* hq,
                              float* hd, int* hs, float* hf) {
    switch (wtype) {
    case HY_TYPE_Q8_0:
        hipLaunchKernelGGL((ffn_up_valu_kernel<HY_TYPE_Q8_0, NT>), grid, dim3(FFN_THREADS), smem, s, W, R, X, xf, T,
                           H, I, E, K, hq, hd, hs, hf);
        break;
    case HY_TYPE_Q4_0:
        hipLaunchKernelGGL((ffn_up_valu_kernel<HY_TYPE_Q4_0, NT>), grid, dim3(FFN_THREADS), smem, s, W, R, X, xf, T,
                           H, I, E, K, hq, hd, hs, hf);
        break;
    default:
        hipLaunchKernelGGL((ffn_up_valu_kernel<HY_TYPE_F32, NT>), grid, dim3(FFN_THREADS), smem, s, W, R, X, xf, T,
                           H, I, E, K, hq, hd, hs, hf);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_ffn_up_valu(int wtype, int NT, int max_tiles, const MatView& W, const Routing& R, const ActQ& X,
                              const float* xf, int T, int H, int I, int E, int K, int8_t* hq, float* hd, int* hs,
                              float* hf, hipStream_t s) {
    dim3 grid(max_tiles, I / QK);
    const size_t smem = ffn_up_smem(wtype, NT, H);
    if (NT == 8) return up_dispatch<8>(wtype, grid, smem, s, W, R, X, xf, T, H, I, E, K, hq, hd, hs, hf);
    return up_dispatch<16>(wtype, grid, smem, s, W, R, X, xf, T, H, I, E, K, hq, hd, hs, hf);
}

template <int NT>
static hipError_t down_dispatch(int wtype, dim3 grid, size_t smem, hipStream_t s, const MatView& W,
                                const Routing& R, const int8_t* hq, const float* hd, const int* hs, const float* hf,
                                int T, int H, int I, int E, int K, int mode, float* y, const float* resid,
                                float* out) {
    switch (wtype) {
    case HY_TYPE_Q8_0:
        hipLaunchKernelGGL((ffn_down_valu_kernel<HY_TYPE_Q8_0, NT>), grid, dim3(FFN_THREADS), smem, s, W, R, hq, hd,
                           hs, hf, T, H, I, E, K, mode, y, resid, out);
        break;
    case HY_TYPE_Q4_0:
        hipLaunchKernelGGL((ffn_down_valu_kernel<HY_TYPE_Q4_0, NT>), grid, dim3(FFN_THREADS), smem, s, W, R, hq, hd,
                           hs, hf, T, H, I, E, K, mode, y, resid, out);
        break;
    default:
        hipLaunchKernelGGL((ffn_down_valu_kernel<HY_TYPE_F32, NT>), grid, dim3(FFN_THREADS), smem, s, W, R, hq, hd,
                           hs, hf, T, H, I, E, K, mode, y, resid, out);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_ffn_down_valu(int wtype, int NT, int n_tiles_bound, int mode, const MatView& W, const Routing& R,
                                const int8_t* hq, const float* hd, const int* hs, const float* hf, int T, int H,
                                int I, int E, int K, float* y, const float* resid, float* out, hipStream_t s) {
    dim3 grid(n_tiles_bound, (H + FFN_ROWS - 1) / FFN_ROWS);
    const size_t smem = ffn_down_smem(wtype, NT, I);
    if (NT == 8)
        return down_dispatch<8>(wtype, grid, smem, s, W, R, hq, hd, hs, hf, T, H, I, E, K, mode, y, resid, out);
    return down_dispatch<16>(wtype, grid, smem, s, W, R, hq, hd, hs, hf, T, H, I, E, K, mode, y, resid, out);
}

hipError_t launch_combine(const Routing& R, const float* y, int T, int H, int K, const float* resid, float* out,
                          hipStream_t s) {
    const size_t n = (size_t)T * H;
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, R, y, T, H, K, resid, out);
    return hipGetLastError();
}

// per-block dots through the VALU routines (parity entry point)
__global__ void block_dots_valu_kernel(int wtype, const uint8_t* __restrict__ w, const uint8_t* __restrict__ x,
                                       int rows, int nb, int* __restrict__ out) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * nb) return;
    const int r = idx / nb, b = idx % nb;
    // GGUF blocks: copy into aligned registers (blocks are 2-byte aligned)
    const uint8_t* xb = x + (size_t)b * 34;
    int xa[8];
    for (int j = 0; j < 8; j++)
        xa[j] = (int)((uint32_t)xb[2 + 4 * j] | ((uint32_t)xb[3 + 4 * j] << 8) | ((uint32_t)xb[4 + 4 * j] << 16) |
                      ((uint32_t)xb[5 + 4 * j] << 24));
    const int4 a0 = make_int4(xa[0], xa[1], xa[2], xa[3]), a1 = make_int4(xa[4], xa[5], xa[6], xa[7]);
    int s;
    if (wtype == HY_TYPE_Q8_0) {
        const uint8_t* wb = w + ((size_t)r * nb + b) * 34;
        int wa[8];
        for (int j = 0; j < 8; j++)
            wa[j] = (int)((uint32_t)wb[2 + 4 * j] | ((uint32_t)wb[3 + 4 * j] << 8) |
                          ((uint32_t)wb[4 + 4 * j] << 16) | ((uint32_t)wb[5 + 4 * j] << 24));
        s = dot_q8_block(make_int4(wa[0], wa[1], wa[2], wa[3]), make_int4(wa[4], wa[5], wa[6], wa[7]), a0, a1);
    } else {
        const uint8_t* wb = w + ((size_t)r * nb + b) * 18;
        int wa[4];
        for (int j = 0; j < 4; j++)
            wa[j] = (int)((uint32_t)wb[2 + 4 * j] | ((uint32_t)wb[3 + 4 * j] << 8) |
                          ((uint32_t)wb[4 + 4 * j] << 16) | ((uint32_t)wb[5 + 4 * j] << 24));
        int asum = 0;
        for (int j = 0; j < 32; j++) asum += (int8_t)xb[2 + j];
        s = dot_q4_block(make_int4(wa[0], wa[1], wa[2], wa[3]), a0, a1, asum);
    }
    out[idx] = s;
}

hipError_t launch_block_dots_valu(int wtype, const uint8_t* w, const uint8_t* x, int rows, int nb, int* out,
                                  hipStream_t s) {
    const int n = rows * nb;
    hipLaunchKernelGGL(block_dots_valu_kernel, dim3((n + 255) / 256), dim3(256), 0, s, wtype, w, x, rows, nb, out);
    return hipGetLastError();
}

}  // namespace hy
