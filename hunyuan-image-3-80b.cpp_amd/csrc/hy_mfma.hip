// hy_mfma.hip -- grouped expert GEMMs on the int8 matrix cores (prefill / image-token
// batches).
//
// Work item = (tile, row block): a tile is up to 64 (token, expert) pairs of one
// expert (or 64 consecutive tokens for the shared expert), a row block is 128 weight
// rows (two 64-row groups of the row-group-interleaved weights).  Each K step stages
// KB = 4 GGUF blocks (128 k) of the 128 weight rows and of the tile's 64 activation
// rows in LDS (double buffered, register staging).  Every
// wave owns 2 x (32 rows x 32 tokens) output tiles and, per 32-wide block, issues
// v_mfma_i32_32x32x32_i8: K = 32 is exactly one GGUF block, so each MFMA result is the
// exact int32 block dot sum_j w_j x_j of ggml's vec_dot, which is then rescaled in
// fp32 with the blocks taken in order: acc = fmaf(float(S), d_w * d_x, acc) -- the
// accumulation the oracle and the decode GEMV use, so all paths agree bit for bit.
//
// MFMA operand / result layout (gfx950, checked on the device): A lane l holds 16
// bytes of row l%32, B lane l 16 bytes of column l%32, both at the same k offset
// 16*(l/32) inside the block; result register v of lane l is row
// 8*(v/4) + 4*(l/32) + v%4, column l%32.
//
// Modes: 0 = gate_up (packed rows: a 128-row block is two 64-row slabs of 32 SiLU +
// 32 linear rows; epilogue h = silu(g) * u and Q8_0 quantization of h per token and
// slab); 1 = down for routed tiles (writes y[pair][row]); 2 = down for shared tiles
// fused with the combine out = resid + (y_shared + sum_{e ascending} w_e y_e).
#include "hy_device.hpp"
#include "hy_launch.hpp"
#include "hy_layout.hpp"

namespace hy {

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef int v16i_t __attribute__((ext_vector_type(16)));

constexpr int MM_ROWS = 128;          // weight rows per work item
constexpr int MM_TOK = 64;            // pairs (tokens) per tile
constexpr int MM_KB = 4;              // GGUF blocks per K step
constexpr int MM_PITCH = MM_KB * 32 + 16;  // LDS row pitch (bytes), padded against bank conflicts
constexpr int MM_THREADS = 256;

struct MmArgs {
    MatView W;
    Routing R;
    const int8_t* aq;   // activations int8 [rows][Kdim] (x for mode 0, h for modes 1/2)
    const float* ad;    // activation scales [rows][Kdim/32]
    int T, H, I, E, K;
    int Kdim;           // reduction length (H for mode 0, I for modes 1/2)
    int8_t* hq;         // mode 0 outputs
    float* hd;
    int* hs;
    float* y;           // mode 1 output / mode 2 input
    const float* resid; // mode 2
    float* out;         // mode 2
};

// Q4_0 nibbles (16 bytes, GGUF order) -> 32 int8 values n-8 in element order.
__device__ __forceinline__ void unpack_q4(const int4 w, int4& lo, int4& hi) {
    const int m = 0x0F0F0F0F;
    auto cv = [](int v) { return ((v | (int)0x80808080) - 0x08080808) ^ (int)0x80808080; };
    lo = make_int4(cv(w.x & m), cv(w.y & m), cv(w.z & m), cv(w.w & m));
    hi = make_int4(cv((w.x >> 4) & m), cv((w.y >> 4) & m), cv((w.z >> 4) & m), cv((w.w >> 4) & m));
}

template <int WT, int MODE>
__global__ __launch_bounds__(MM_THREADS, 2) void moe_mfma_kernel(MmArgs a) {
    __shared__ __align__(16) int8_t As[2][MM_ROWS][MM_PITCH];
    __shared__ __align__(16) int8_t Bs[2][MM_TOK][MM_PITCH];
    __shared__ __align__(16) float Asc[2][MM_KB][MM_ROWS];  // row-contiguous: float4 = 4 rows
    __shared__ __align__(16) float Bsc[2][MM_KB][MM_TOK];
    __shared__ int tok_s[MM_TOK], slot_s[MM_TOK];

    const int tile = (MODE == 2) ? a.R.meta[0] + (int)blockIdx.x : (int)blockIdx.x;
    if (tile >= a.R.meta[MODE == 1 ? 0 : 1]) return;
    const int e = a.R.tile_e[tile], start = a.R.tile_start[tile], n = a.R.tile_n[tile];
    const bool shared = e == a.E;
    const int row0 = blockIdx.y * MM_ROWS;
    const int Kd = a.Kdim;
    const int nb = Kd / QK;
    const int tid = threadIdx.x;

    if (tid < MM_TOK) {
        int tok = 0, slot = 0;
        if (tid < n) {
            if (shared) {
                tok = start + tid;
                slot = a.T * a.K + tok;
            } else {
                slot = a.R.off[e] + start + tid;
                tok = a.R.srt_tok[slot];
            }
        }
        tok_s[tid] = tok;
        slot_s[tid] = slot;
    }
    __syncthreads();

    // ---- global -> register staging
    const uint8_t* wq = a.W.qs + (size_t)e * a.W.qs_stride;
    const uint16_t* wsc = a.W.sc + (size_t)e * a.W.sc_stride;
    constexpr int A_VEC = (WT == HY_TYPE_Q4_0) ? (MM_ROWS * MM_KB) / MM_THREADS       // int4 of nibbles
                                               : (MM_ROWS * MM_KB * 2) / MM_THREADS;  // int4 of int8
    constexpr int B_VEC = (MM_TOK * MM_KB * 2) / MM_THREADS;
    int4 ra[A_VEC], rb[B_VEC];
    float rasc[2], rbsc;
    // activation row of this thread's B loads
    auto act_row = [&](int i) -> int { return (MODE == 0) ? tok_s[i] : slot_s[i]; };

    // weights are row-group interleaved: block b of a 64-row group is one contiguous
    // chunk of 64 * BPB bytes; a stage is 2 groups x MM_KB blocks = 8 chunks
    constexpr int BPB = WT == HY_TYPE_Q4_0 ? 16 : 32;
    const int G0 = row0 / 64;
    auto chunk_base = [&](int chunk, int kb0) -> size_t {
        return (((size_t)(G0 + (chunk >> 2)) * nb + kb0 + (chunk & 3)) * 64) * BPB;
    };
    auto load_stage = [&](int s) {
        const int kb0 = s * MM_KB;
#pragma unroll
        for (int v = 0; v < A_VEC; v++) {
            const int idx = tid + v * MM_THREADS;
            if (WT == HY_TYPE_Q4_0) {  // 64 int4 (rows) per chunk
                ra[v] = *reinterpret_cast<const int4*>(wq + chunk_base(idx >> 6, kb0) + (size_t)(idx & 63) * 16);
            } else {                   // 128 int4 (rows x halves) per chunk
                ra[v] = *reinterpret_cast<const int4*>(wq + chunk_base(idx >> 7, kb0) + (size_t)(idx & 127) * 16);
            }
        }
#pragma unroll
        for (int v = 0; v < 2; v++) {
            const int idx = tid + v * MM_THREADS;  // 8 chunks x 64 rows
            const int chunk = idx >> 6;
            rasc[v] = h2f(wsc[((size_t)(G0 + (chunk >> 2)) * nb + kb0 + (chunk & 3)) * 64 + (idx & 63)]);
        }
#pragma unroll
        for (int v = 0; v < B_VEC; v++) {
            const int idx = tid + v * MM_THREADS;
            const int i = idx / (MM_KB * 2), c = idx % (MM_KB * 2);
            rb[v] = i < n ? *reinterpret_cast<const int4*>(a.aq + (size_t)act_row(i) * Kd + (size_t)kb0 * QK + c * 16)
                          : make_int4(0, 0, 0, 0);
        }
        {
            const int i = tid / MM_KB, b = tid % MM_KB;  // 64 x 4 = 256
            rbsc = i < n ? a.ad[(size_t)act_row(i) * nb + kb0 + b] : 0.0f;
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int v = 0; v < A_VEC; v++) {
            const int idx = tid + v * MM_THREADS;
            if (WT == HY_TYPE_Q4_0) {
                const int chunk = idx >> 6, row = (chunk >> 2) * 64 + (idx & 63), kb = chunk & 3;
                int4 lo, hi;
                unpack_q4(ra[v], lo, hi);
                *reinterpret_cast<int4*>(&As[buf][row][kb * 32]) = lo;
                *reinterpret_cast<int4*>(&As[buf][row][kb * 32 + 16]) = hi;
            } else {
                const int chunk = idx >> 7, w = idx & 127;
                const int row = (chunk >> 2) * 64 + (w >> 1), kb = chunk & 3;
                *reinterpret_cast<int4*>(&As[buf][row][kb * 32 + (w & 1) * 16]) = ra[v];
            }
        }
#pragma unroll
        for (int v = 0; v < 2; v++) {
            const int idx = tid + v * MM_THREADS;
            const int chunk = idx >> 6;
            Asc[buf][chunk & 3][(chunk >> 2) * 64 + (idx & 63)] = rasc[v];
        }
#pragma unroll
        for (int v = 0; v < B_VEC; v++) {
            const int idx = tid + v * MM_THREADS;
            const int i = idx / (MM_KB * 2), c = idx % (MM_KB * 2);
            *reinterpret_cast<int4*>(&Bs[buf][i][c * 16]) = rb[v];
        }
        Bsc[buf][tid % MM_KB][tid / MM_KB] = rbsc;
    };

    const int wave = tid / WAVE, lane = tid % WAVE;
    const int sl = wave & 1;          // 64-row slab within the row block
    const int nh = wave >> 1;         // 32-token half of the tile
    const bool active = nh * 32 < n;  // waves past the tile's last pair skip the math
    const int lr = lane % 32, lg = lane / 32;
    float acc0[16], acc1[16];
#pragma unroll
    for (int v = 0; v < 16; v++) {
        acc0[v] = 0.0f;
        acc1[v] = 0.0f;
    }

    const int nstage = nb / MM_KB;
    load_stage(0);
    store_stage(0);
    __syncthreads();
    for (int s = 0; s < nstage; s++) {
        const int buf = s & 1;
        if (s + 1 < nstage) load_stage(s + 1);
        if (active) {
#pragma unroll
            for (int kb = 0; kb < MM_KB; kb++) {
                const v4i_t A0 = *reinterpret_cast<const v4i_t*>(&As[buf][sl * 64 + lr][kb * 32 + 16 * lg]);
                const v4i_t A1 = *reinterpret_cast<const v4i_t*>(&As[buf][sl * 64 + 32 + lr][kb * 32 + 16 * lg]);
                const v4i_t B = *reinterpret_cast<const v4i_t*>(&Bs[buf][nh * 32 + lr][kb * 32 + 16 * lg]);
                const v16i_t zero = {};
                const v16i_t S0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A0, B, zero, 0, 0, 0);
                const v16i_t S1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A1, B, zero, 0, 0, 0);
                const float dx = Bsc[buf][kb][nh * 32 + lr];
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int r = 8 * g + 4 * lg;
                    const float4 d0 = *reinterpret_cast<const float4*>(&Asc[buf][kb][sl * 64 + r]);
                    const float4 d1 = *reinterpret_cast<const float4*>(&Asc[buf][kb][sl * 64 + 32 + r]);
                    acc0[4 * g + 0] = fmaf((float)S0[4 * g + 0], d0.x * dx, acc0[4 * g + 0]);
                    acc0[4 * g + 1] = fmaf((float)S0[4 * g + 1], d0.y * dx, acc0[4 * g + 1]);
                    acc0[4 * g + 2] = fmaf((float)S0[4 * g + 2], d0.z * dx, acc0[4 * g + 2]);
                    acc0[4 * g + 3] = fmaf((float)S0[4 * g + 3], d0.w * dx, acc0[4 * g + 3]);
                    acc1[4 * g + 0] = fmaf((float)S1[4 * g + 0], d1.x * dx, acc1[4 * g + 0]);
                    acc1[4 * g + 1] = fmaf((float)S1[4 * g + 1], d1.y * dx, acc1[4 * g + 1]);
                    acc1[4 * g + 2] = fmaf((float)S1[4 * g + 2], d1.z * dx, acc1[4 * g + 2]);
                    acc1[4 * g + 3] = fmaf((float)S1[4 * g + 3], d1.w * dx, acc1[4 * g + 3]);
                }
            }
        }
        if (s + 1 < nstage) {
            store_stage(buf ^ 1);
        }
        __syncthreads();
    }

    // ---- epilogues
    const int j = nh * 32 + lr;  // pair index within the tile
    if (!active || j >= n) return;
    if (MODE == 0) {
        // acc0 = gate rows, acc1 = matching up rows of slab (2*blockIdx.y + sl)
        const int slab = 2 * blockIdx.y + sl;
        float h[16];
        float amax = 0.0f;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            h[v] = swiglu(acc0[v], acc1[v]);
            amax = fmaxf(amax, fabsf(h[v]));
        }
        amax = fmaxf(amax, __shfl_xor(amax, 32, WAVE));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        int qsum = 0;
        int packed[4];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t p = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int q = (int)__builtin_roundf(h[4 * g + i] * id);
                qsum += q;
                p |= ((uint32_t)(q & 0xff)) << (8 * i);
            }
            packed[g] = (int)p;
        }
        qsum += __shfl_xor(qsum, 32, WAVE);
        const size_t slot = (size_t)slot_s[j];
        int8_t* dst = a.hq + slot * a.I + (size_t)slab * QK;
#pragma unroll
        for (int g = 0; g < 4; g++) *reinterpret_cast<int*>(dst + 8 * g + 4 * lg) = packed[g];
        if (lg == 0) {
            const size_t nbi = a.I / QK;
            a.hd[slot * nbi + slab] = h2f(f2h(d));
            a.hs[slot * nbi + slab] = qsum;
        }
    } else {
        const int rbase = row0 + sl * 64;
        if (MODE == 1) {
            float* yr = a.y + (size_t)slot_s[j] * a.H;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int r = 8 * g + 4 * lg;
                *reinterpret_cast<float4*>(yr + rbase + r) =
                    make_float4(acc0[4 * g], acc0[4 * g + 1], acc0[4 * g + 2], acc0[4 * g + 3]);
                *reinterpret_cast<float4*>(yr + rbase + 32 + r) =
                    make_float4(acc1[4 * g], acc1[4 * g + 1], acc1[4 * g + 2], acc1[4 * g + 3]);
            }
        } else {
            const int t = tok_s[j];
            float o0[16], o1[16];
#pragma unroll
            for (int v = 0; v < 16; v++) {
                o0[v] = 0.0f;
                o1[v] = 0.0f;
            }
            for (int k = 0; k < a.K; k++) {
                const float w = a.R.comb_w[t * a.K + k];
                const float* yr = a.y + (size_t)a.R.comb_pos[t * a.K + k] * a.H + rbase;
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int r = 8 * g + 4 * lg;
                    const float4 y0 = *reinterpret_cast<const float4*>(yr + r);
                    const float4 y1 = *reinterpret_cast<const float4*>(yr + 32 + r);
                    o0[4 * g] = fmaf(w, y0.x, o0[4 * g]);
                    o0[4 * g + 1] = fmaf(w, y0.y, o0[4 * g + 1]);
                    o0[4 * g + 2] = fmaf(w, y0.z, o0[4 * g + 2]);
                    o0[4 * g + 3] = fmaf(w, y0.w, o0[4 * g + 3]);
                    o1[4 * g] = fmaf(w, y1.x, o1[4 * g]);
                    o1[4 * g + 1] = fmaf(w, y1.y, o1[4 * g + 1]);
                    o1[4 * g + 2] = fmaf(w, y1.z, o1[4 * g + 2]);
                    o1[4 * g + 3] = fmaf(w, y1.w, o1[4 * g + 3]);
                }
            }
            float* orow = a.out + (size_t)t * a.H + rbase;
            const float* rrow = a.resid ? a.resid + (size_t)t * a.H + rbase : nullptr;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int r = 8 * g + 4 * lg;
                float4 v0 = make_float4(acc0[4 * g] + o0[4 * g], acc0[4 * g + 1] + o0[4 * g + 1],
                                        acc0[4 * g + 2] + o0[4 * g + 2], acc0[4 * g + 3] + o0[4 * g + 3]);
                float4 v1 = make_float4(acc1[4 * g] + o1[4 * g], acc1[4 * g + 1] + o1[4 * g + 1],
                                        acc1[4 * g + 2] + o1[4 * g + 2], acc1[4 * g + 3] + o1[4 * g + 3]);
                if (rrow) {
                    const float4 q0 = *reinterpret_cast<const float4*>(rrow + r);
                    const float4 q1 = *reinterpret_cast<const float4*>(rrow + 32 + r);
                    v0 = make_float4(q0.x + v0.x, q0.y + v0.y, q0.z + v0.z, q0.w + v0.w);
                    v1 = make_float4(q1.x + v1.x, q1.y + v1.y, q1.z + v1.z, q1.w + v1.w);
                }
                *reinterpret_cast<float4*>(orow + r) = v0;
                *reinterpret_cast<float4*>(orow + 32 + r) = v1;
            }
        }
    }
}

template <int MODE>
static hipError_t launch_mode(int wtype, dim3 grid, hipStream_t s, const MmArgs& a) {
    if (wtype == HY_TYPE_Q4_0)
        hipLaunchKernelGGL((moe_mfma_kernel<HY_TYPE_Q4_0, MODE>), grid, dim3(MM_THREADS), 0, s, a);
    else
        hipLaunchKernelGGL((moe_mfma_kernel<HY_TYPE_Q8_0, MODE>), grid, dim3(MM_THREADS), 0, s, a);
    return hipGetLastError();
}

bool mfma_path_ok(int wtype, int H, int I) {
    return (wtype == HY_TYPE_Q8_0 || wtype == HY_TYPE_Q4_0) && H % MM_ROWS == 0 && I % MM_ROWS == 0 &&
           (H / QK) % MM_KB == 0 && (I / QK) % MM_KB == 0;
}

int mfma_tile_tokens() { return MM_TOK; }

hipError_t launch_ffn_up_mfma(int wtype, int n_tiles_bound, const MatView& W, const Routing& R, const ActQ& X,
                              int T, int H, int I, int E, int K, int8_t* hq, float* hd, int* hs, hipStream_t s) {
    MmArgs a{W, R, X.q, X.d, T, H, I, E, K, H, hq, hd, hs, nullptr, nullptr, nullptr};
    return launch_mode<0>(wtype, dim3(n_tiles_bound, 2 * I / MM_ROWS), s, a);
}

hipError_t launch_ffn_down_mfma(int wtype, int n_tiles_bound, int mode, const MatView& W, const Routing& R,
                                const int8_t* hq, const float* hd, int T, int H, int I, int E, int K, float* y,
                                const float* resid, float* out, hipStream_t s) {
    MmArgs a{W, R, hq, hd, T, H, I, E, K, I, nullptr, nullptr, nullptr, y, resid, out};
    dim3 grid(n_tiles_bound, H / MM_ROWS);
    return mode == 0 ? launch_mode<1>(wtype, grid, s, a) : launch_mode<2>(wtype, grid, s, a);
}

}  // namespace hy
