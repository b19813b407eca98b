// hy_attn.hip -- the attention half of a HunyuanImage-3 decoder layer on gfx950, in
// fp32 (the reference's precision): attention_forward_cpu (src/attention.cpp:10-185)
// and the KV-cache branch of decoder_layer_extended_f32
// (src/hunyuan_extended.cpp:52-176), with rope_f32 (src/rms_norm.cpp:97-152) and the
// 2D rotary tables (src/hunyuan_image_gen.cpp:11-117).
//
// Kernels:
//  * gemm_nt_f32_lds_kernel / gemm_nt_f32_kernel: C[M][N] = (R[M][N] +) A[M][K] .
//    W[N][K]^T on v_mfma_f32_32x32x2f32 (the QKV and output projections; R is the
//    decoder layer's residual stream when the output projection adds it).  Waves of
//    64 x 64 (2 x 2 MFMA tiles).  Large grids: four waves per 128 x 128 work group,
//    K in stages of 32 (16) floats DMA-copied into a swizzled LDS ring.  Mid-size
//    grids (64..1023 tiles): the same kernel as 512 stream-K work groups that split
//    the tiles' K stages evenly, and gemm_fixup_kernel summing the cut tiles' pieces
//    in K order.  Small grids: one wave per work group, K in steps of 16 straight
//    from global memory into registers.
//  * rope_qknorm_kernel: one wave per (token, head): rotary embedding (1D positions,
//    2D tables or none), per-head RMSNorm, written to q [T][nh][hd] and, for key
//    heads, k / v into a [nkv][L][hd] cache at row pos0 + t.
//  * flash_attn_kernel<HD>: one work group per (32-query tile, kv group), one wave
//    per query head of the group (4 heads share the group's K / V blocks in LDS).
//    Scores are computed transposed, S^T = K Q^T (keys on MFMA rows, queries on the
//    lanes), so a query's online-softmax statistics stay in its lane pair; P^T then
//    feeds O^T += V^T P^T straight from the score registers.
//
// fp32 MFMA layouts (v_mfma_f32_32x32x2f32, checked on the device): A lane l holds
// A[l%32][l/32], B lane l holds B[l/32][l%32], result register v of lane l is
// C[8*(v/4) + 4*(l/32) + v%4][l%32].  Operand k-slots can be any permutation of the
// reduction index as long as A and B use the same one: lane half h takes k = 8h + j
// at step j of a 16-wide chunk, so each lane reads 8 consecutive floats.
#include <utility>

#include "hy_device.hpp"
#include "hy_launch.hpp"
#include "hy_lds.hpp"

namespace hy {

typedef float v16f_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16f_t mfma_f32(float a, float b, v16f_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------- GEMM (NT)
// WM x WN waves per work group, each a 64 x 64 output tile (launched as 1 x 1: the
// grids too small for the LDS-staged kernel below)
template <int WM, int WN>
__global__ __launch_bounds__(WAVE * WM * WN) void gemm_nt_f32_kernel(const float* __restrict__ A,
                                                                    const float* __restrict__ W,
                                                                    const float* __restrict__ R,
                                                                    float* __restrict__ C, int M, int N, int K) {
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int lr = lane % 32, h = lane / 32;
    const int m0 = blockIdx.y * (64 * WM) + (wave / WN) * 64, n0 = blockIdx.x * (64 * WN) + (wave % WN) * 64;
    // operand rows of this lane (clamped for loads; the stores are guarded)
    const float* pa[2];
    const float* pb[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int r = min(m0 + 32 * i + lr, M - 1), c = min(n0 + 32 * i + lr, N - 1);
        pa[i] = A + (size_t)r * K + 8 * h;
        pb[i] = W + (size_t)c * K + 8 * h;
    }
    v16f_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = v16f_t{};
    float4 a[2][2], b[2][2];  // [tile][lo/hi 4 floats]
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            a[i][0] = *reinterpret_cast<const float4*>(pa[i] + k0);
            a[i][1] = *reinterpret_cast<const float4*>(pa[i] + k0 + 4);
            b[i][0] = *reinterpret_cast<const float4*>(pb[i] + k0);
            b[i][1] = *reinterpret_cast<const float4*>(pb[i] + k0 + 4);
        }
    };
    load(0);
    for (int k0 = 0; k0 < K; k0 += 16) {
        float av[2][8], bv[2][8];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const float4 x0 = a[i][0], x1 = a[i][1], y0 = b[i][0], y1 = b[i][1];
            av[i][0] = x0.x; av[i][1] = x0.y; av[i][2] = x0.z; av[i][3] = x0.w;
            av[i][4] = x1.x; av[i][5] = x1.y; av[i][6] = x1.z; av[i][7] = x1.w;
            bv[i][0] = y0.x; bv[i][1] = y0.y; bv[i][2] = y0.z; bv[i][3] = y0.w;
            bv[i][4] = y1.x; bv[i][5] = y1.y; bv[i][6] = y1.z; bv[i][7] = y1.w;
        }
        if (k0 + 16 < K) load(k0 + 16);
#pragma unroll
        for (int j = 0; j < 8; j++)
#pragma unroll
            for (int ti = 0; ti < 2; ti++)
#pragma unroll
                for (int tj = 0; tj < 2; tj++) acc[ti][tj] = mfma_f32(av[ti][j], bv[tj][j], acc[ti][tj]);
    }
#pragma unroll
    for (int ti = 0; ti < 2; ti++)
#pragma unroll
        for (int tj = 0; tj < 2; tj++) {
            const int col = n0 + 32 * tj + lr;
            if (col >= N) continue;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = m0 + 32 * ti + 8 * (v / 4) + 4 * h + v % 4;
                if (row >= M) continue;
                const size_t o = (size_t)row * N + col;
                C[o] = R ? R[o] + acc[ti][tj][v] : acc[ti][tj][v];  // optional residual: R + A.W^T
            }
        }
}

// LDS-staged GEMM for large grids: a 128 x 128 tile per work group of 4 waves (2 x 2,
// 64 x 64 each).  K advances in stages of KC floats: each wave DMA-copies 32 rows of
// A and 32 rows of W (KC floats each) global -> LDS into a RING-deep ring, so every
// operand element is fetched once per work group (the register kernel above fetches
// it once per wave) and no VGPRs hold copies in flight.  Rows sit in LDS as 16-byte
// chunks whose position is XOR-swizzled by the row (gemm_swz), so the ds_read_b128
// of 32 consecutive rows at one logical chunk spreads over all banks.
template <int KC>
struct GemmLds {
    static constexpr int ROWB = KC * 4;                // bytes of one operand row in a stage
    static constexpr int OPB = 128 * ROWB;             // one operand tile
    static constexpr int BYTES = 2 * OPB;              // A tile, then W tile
    static constexpr int CPO = 32 * ROWB / 1024;       // 1 KB copies per wave and operand
    static constexpr int LOADS = 2 * CPO;              // copies per wave and stage
    static_assert(KC == 16 || KC == 32, "stages of 16 or 32 floats");
};

// chunk swizzle of LDS row r: chunk c sits at position c ^ gemm_swz(r).  Any 8 (and
// any 16) consecutive rows read at one logical chunk land in distinct 16-byte bank
// groups of the 128-byte (256-byte) window.
template <int KC>
__device__ __forceinline__ int gemm_swz(int r) {
    if constexpr (KC == 16)
        return (((r >> 2) & 1) << 1) | (((r >> 1) ^ (r >> 3)) & 1);
    else
        return (((r >> 2) & 1) << 2) | (((r >> 1) & 1) << 1) | ((r ^ (r >> 3)) & 1);
}

struct GemmArgs {
    const float* A;
    const float* W;
    const float* R;  // optional residual (C = R + A.W^T)
    float* C;
    int M, N, K;
    int mtiles;      // 128-row tiles of M
    int tiles;
    int G;           // 0: one tile per work group; else the stream-K work-group count
    float* part;     // stream-K partial tiles: 2 G slots of 128 x 128 floats
};

// first row / column of tile t: N varies fastest, so consecutive work groups share
// the A rows of one row of tiles (measured ~3 % faster than M-fastest at 4096 tokens)
__device__ __forceinline__ int tile_m0(const GemmArgs& p, int t) { return 128 * (t / (p.tiles / p.mtiles)); }
__device__ __forceinline__ int tile_n0(const GemmArgs& p, int t) { return 128 * (t % (p.tiles / p.mtiles)); }

// Stream-K split: the tiles x (K / KC) stage units are cut into G equal contiguous
// ranges, work group g taking units [g U / G, (g + 1) U / G).  A tile whose units all
// fall in one range is written directly; the pieces of a tile cut between ranges are
// written to partial slots (slot 2 g for the range's first piece, 2 g + 1 for its
// last) and summed in K order by gemm_fixup_kernel.
__device__ __forceinline__ long sk_lo(long g, long U, int G) { return g * U / G; }
__device__ __forceinline__ int sk_owner(long u, long U, int G) { return (int)(((u + 1) * G - 1) / U); }

template <int KC, int RING, int WG_PER_CU>
__global__ __launch_bounds__(256, WG_PER_CU) void gemm_nt_f32_lds_kernel(GemmArgs p) {
    using G = GemmLds<KC>;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[RING][G::BYTES];
    const int tid = threadIdx.x, lane = tid % WAVE;
    const int wv = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int lr = lane % 32, h = lane / 32;
    const int M = p.M, N = p.N, K = p.K;
    const int nstage = K / KC;

    // copy lanes: lane l of copy i lands at byte 16 l of the wave's 1 KB piece i, i.e.
    // row 32 wv + (1024 i + 16 l) / ROWB, position q = l % (ROWB / 16), and fetches
    // the chunk stored there, q ^ gemm_swz(row).  Rows past M / N re-read the last
    // row (in bounds; their results are never stored).
    int crow[G::CPO], ccol[G::CPO];
#pragma unroll
    for (int i = 0; i < G::CPO; i++) {
        const int o = 1024 * i + 16 * lane;
        crow[i] = 32 * wv + o / G::ROWB;
        ccol[i] = 4 * ((o % G::ROWB) / 16 ^ gemm_swz<KC>(crow[i]));
    }
    // operand reads: A rows 64 wm + 32 ti + lr, W rows 64 wn + 32 tj + lr; sub-step u
    // (16 floats) takes floats 16 u + 8 h .. + 7 of the row as two chunks
    const int wm = wv / 2, wn = wv % 2;
    const int sw = gemm_swz<KC>(lr);  // rows 32 t + lr share the swizzle of lr
    uint32_t ra[KC / 16][2], rw[KC / 16][2];
#pragma unroll
    for (int u = 0; u < KC / 16; u++)
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int pos = 16 * ((4 * u + 2 * h + t) ^ sw);
            ra[u][t] = (uint32_t)((64 * wm + lr) * G::ROWB + pos);
            rw[u][t] = (uint32_t)(G::OPB + (64 * wn + lr) * G::ROWB + pos);
        }
    const uint32_t ring0 = lds_off(ring[0]);

    // stages [s0, s1) of tile t into acc
    auto segment = [&](int t, int s0, int s1, v16f_t (&acc)[2][2]) {
        const int mt = tile_m0(p, t), nt = tile_n0(p, t);
        const float* a_base = p.A + (size_t)mt * K;
        const float* w_base = p.W + (size_t)nt * K;
        uint32_t a_off[G::CPO], w_off[G::CPO];
#pragma unroll
        for (int i = 0; i < G::CPO; i++) {
            a_off[i] = (uint32_t)((min(mt + crow[i], M - 1) - mt) * K + ccol[i]) * 4u;
            w_off[i] = (uint32_t)((min(nt + crow[i], N - 1) - nt) * K + ccol[i]) * 4u;
        }
        auto issue = [&](int s) {
            uint8_t* st = ring[(s - s0) % RING];
            const uint8_t* ab = reinterpret_cast<const uint8_t*>(a_base + (size_t)s * KC);
            const uint8_t* wb = reinterpret_cast<const uint8_t*>(w_base + (size_t)s * KC);
#pragma unroll
            for (int i = 0; i < G::CPO; i++) {
                g2l16(ab + a_off[i], st + 32 * wv * G::ROWB + 1024 * i);
                g2l16(wb + w_off[i], st + G::OPB + 32 * wv * G::ROWB + 1024 * i);
            }
        };
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[i][j] = v16f_t{};
#pragma unroll
        for (int s = 0; s < RING - 1; s++)
            if (s0 + s < s1) issue(s0 + s);
        for (int s = s0; s < s1; s++) {
            wait_copies<G::LOADS, RING - 2>(s1 - 1 - s);
            __syncthreads();
            if (s + RING - 1 < s1) issue(s + RING - 1);  // refills the slot read at s - 1
            const uint32_t st = ring0 + (uint32_t)(((s - s0) % RING) * G::BYTES);
            v4i_t a[KC / 16][2][2], b[KC / 16][2][2];  // [u][tile][chunk]
#pragma unroll
            for (int u = 0; u < KC / 16; u++)
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    a[u][0][q] = lds_b128_at<0>(st + ra[u][q]);
                    a[u][1][q] = lds_b128_at<32 * G::ROWB>(st + ra[u][q]);
                    b[u][0][q] = lds_b128_at<0>(st + rw[u][q]);
                    b[u][1][q] = lds_b128_at<32 * G::ROWB>(st + rw[u][q]);
                }
            lds_wait();
#pragma unroll
            for (int u = 0; u < KC / 16; u++)
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        lds_pin(a[u][i][q]);
                        lds_pin(b[u][i][q]);
                    }
#pragma unroll
            for (int u = 0; u < KC / 16; u++)
#pragma unroll
                for (int j = 0; j < 8; j++)
#pragma unroll
                    for (int ti = 0; ti < 2; ti++)
#pragma unroll
                        for (int tj = 0; tj < 2; tj++)
                            // (__int_as_float: this hipcc miscompiles __builtin_bit_cast of
                            // a vector element into a read of element 0)
                            acc[ti][tj] = mfma_f32(__int_as_float(a[u][ti][j / 4][j % 4]),
                                                   __int_as_float(b[u][tj][j / 4][j % 4]), acc[ti][tj]);
        }
        __syncthreads();  // every wave is done with the ring before it is refilled
    };
    auto store = [&](int t, const v16f_t (&acc)[2][2]) {
        const int m0 = tile_m0(p, t) + 64 * wm, n0 = tile_n0(p, t) + 64 * wn;
#pragma unroll
        for (int ti = 0; ti < 2; ti++)
#pragma unroll
            for (int tj = 0; tj < 2; tj++) {
                const int col = n0 + 32 * tj + lr;
                if (col >= N) continue;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int row = m0 + 32 * ti + 8 * (v / 4) + 4 * h + v % 4;
                    if (row >= M) continue;
                    const size_t o = (size_t)row * N + col;
                    p.C[o] = p.R ? p.R[o] + acc[ti][tj][v] : acc[ti][tj][v];  // R + A.W^T
                }
            }
    };

    v16f_t acc[2][2];
    if (p.G == 0) {
        segment(blockIdx.x, 0, nstage, acc);
        store(blockIdx.x, acc);
        return;
    }
    const long U = (long)p.tiles * nstage;
    const int g = blockIdx.x;
    const long lo = sk_lo(g, U, p.G), hi = sk_lo(g + 1, U, p.G);
    for (long u = lo; u < hi;) {
        const int t = (int)(u / nstage);
        const int s0 = (int)(u - (long)t * nstage);
        const int s1 = (int)min((long)nstage, s0 + (hi - u));
        segment(t, s0, s1, acc);
        if (s0 == 0 && s1 == nstage) {
            store(t, acc);
        } else {
            float* slot = p.part + (size_t)(2 * g + (u == lo ? 0 : 1)) * (128 * 128) + wv * 4096 + lane;
#pragma unroll
            for (int ti = 0; ti < 2; ti++)
#pragma unroll
                for (int tj = 0; tj < 2; tj++)
#pragma unroll
                    for (int v = 0; v < 16; v++) slot[((ti * 2 + tj) * 16 + v) * 64] = acc[ti][tj][v];
        }
        u += s1 - s0;
    }
}

// Sum of the stream-K pieces of every cut tile, in K order (+ R): work group (t, y)
// takes values 4 y .. 4 y + 3 of every thread of tile t (tiles written directly return
// at once).  Thread layout and slot layout are the GEMM's: wave w, lane l, value
// q = (2 ti + tj) 16 + v at slot + 4096 w + 64 q + l.
constexpr int FIX_Q = 4;
__global__ __launch_bounds__(256) void gemm_fixup_kernel(GemmArgs p, int nstage) {
    const int t = blockIdx.x;
    const long U = (long)p.tiles * nstage;
    const long u0 = (long)t * nstage, u1 = u0 + nstage - 1;
    const int g0 = sk_owner(u0, U, p.G), g1 = sk_owner(u1, U, p.G);
    if (g0 == g1) return;
    const int tid = threadIdx.x, wv = tid / WAVE, lane = tid % WAVE;
    const int lr = lane % 32, h = lane / 32, wm = wv / 2, wn = wv % 2;
    const int m0 = tile_m0(p, t) + 64 * wm, n0 = tile_n0(p, t) + 64 * wn;
    // the first piece is g0's last one unless g0's range starts at this tile
    const int slot0 = 2 * g0 + (sk_lo(g0, U, p.G) == u0 ? 0 : 1);
    const float* __restrict__ part = p.part;
    const size_t base = (size_t)wv * 4096 + (size_t)blockIdx.y * FIX_Q * 64 + lane;
    float sum[FIX_Q];
#pragma unroll
    for (int j = 0; j < FIX_Q; j++) sum[j] = part[(size_t)slot0 * (128 * 128) + base + 64 * j];
    for (int g = g0 + 1; g <= g1; g++) {
        float x[FIX_Q];
#pragma unroll
        for (int j = 0; j < FIX_Q; j++) x[j] = part[(size_t)(2 * g) * (128 * 128) + base + 64 * j];
#pragma unroll
        for (int j = 0; j < FIX_Q; j++) sum[j] += x[j];
    }
#pragma unroll
    for (int j = 0; j < FIX_Q; j++) {
        const int q = blockIdx.y * FIX_Q + j, ti = q / 32, tj = (q / 16) % 2, v = q % 16;
        const int col = n0 + 32 * tj + lr, row = m0 + 32 * ti + 8 * (v / 4) + 4 * h + v % 4;
        if (col < p.N && row < p.M) {
            const size_t o = (size_t)row * p.N + col;
            p.C[o] = p.R ? p.R[o] + sum[j] : sum[j];
        }
    }
}

// Decode-sized products (M <= 16 rows of A): C = (R +) A . W^T is a stream over W.
// One wave owns GV_RPW consecutive W rows; lane l takes floats 4 l + 256 c .. + 3 of
// every row (chunk c), so each W load is a contiguous 1 KB per wave and each A float4
// (the same for all waves: L1 hits) feeds GV_RPW rows.  Loads are unconditional from
// clamped addresses and software-pipelined GV_D chunks deep; a chunk past K is masked
// by a select.  The 64 lane partials of every output fold level by level at the end.
constexpr int GV_RPW = 2;  // two rows per wave: 4 KB in flight per wave at depth 4 (swept 1..8)
template <int MB, int GV_D>
__global__ __launch_bounds__(256) void gemv_nt_f32_kernel(const float* __restrict__ A, const float* __restrict__ W,
                                                         const float* __restrict__ R, float* __restrict__ C, int M,
                                                         int N, int K) {
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
    const int n0 = (blockIdx.x * 4 + wave) * GV_RPW;
    if (n0 >= N) return;
    const int nch = (K + 4 * WAVE - 1) / (4 * WAVE);
    const float* wrow[GV_RPW];
    const float* arow[MB];
#pragma unroll
    for (int r = 0; r < GV_RPW; r++) wrow[r] = W + (size_t)min(n0 + r, N - 1) * K;
#pragma unroll
    for (int m = 0; m < MB; m++) arow[m] = A + (size_t)min(m, M - 1) * K;
    float acc[GV_RPW][MB];
#pragma unroll
    for (int r = 0; r < GV_RPW; r++)
#pragma unroll
        for (int m = 0; m < MB; m++) acc[r][m] = 0.0f;
    v4f_t wb[GV_D][GV_RPW], ab[GV_D][MB];
    auto load = [&](int c, v4f_t* wd, v4f_t* ad) {
        const int k = min(4 * lane + 4 * WAVE * c, K - 4);  // in bounds (K % 4 == 0)
#pragma unroll
        for (int r = 0; r < GV_RPW; r++) wd[r] = *reinterpret_cast<const v4f_t*>(wrow[r] + k);
#pragma unroll
        for (int m = 0; m < MB; m++) ad[m] = *reinterpret_cast<const v4f_t*>(arow[m] + k);
    };
#pragma unroll
    for (int d = 0; d < GV_D - 1; d++) load(d, wb[d], ab[d]);
    for (int c0 = 0; c0 < nch; c0 += GV_D) {
#pragma unroll
        for (int d = 0; d < GV_D; d++) {
            const int c = c0 + d;
            load(c + GV_D - 1, wb[(d + GV_D - 1) % GV_D], ab[(d + GV_D - 1) % GV_D]);
            __builtin_amdgcn_sched_barrier(0);  // keep the refill ahead of the math
            const bool ok = c < nch && 4 * lane + 4 * WAVE * c < K;
#pragma unroll
            for (int r = 0; r < GV_RPW; r++)
#pragma unroll
                for (int m = 0; m < MB; m++) {
                    const v4f_t w = wb[d][r], x = ab[d][m];
                    float s = acc[r][m];
                    s = fmaf(w[0], x[0], s);
                    s = fmaf(w[1], x[1], s);
                    s = fmaf(w[2], x[2], s);
                    s = fmaf(w[3], x[3], s);
                    acc[r][m] = ok ? s : acc[r][m];
                }
        }
    }
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1)
#pragma unroll
        for (int r = 0; r < GV_RPW; r++)
#pragma unroll
            for (int m = 0; m < MB; m++) acc[r][m] += shfl_down(acc[r][m], sh);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < GV_RPW; r++)
#pragma unroll
            for (int m = 0; m < MB; m++) {
                const int n = n0 + r;
                if (n < N && m < M) {
                    const size_t o = (size_t)m * N + n;
                    C[o] = R ? R[o] + acc[r][m] : acc[r][m];
                }
            }
    }
}

size_t gemm_nt_f32_ws_bytes() { return (size_t)2 * GEMM_SK_GROUPS * 128 * 128 * 4; }

// fewer 128 x 128 tiles than two full rounds of resident work groups (but enough to
// split): stream-K over all of them, two 64 KB-LDS work groups per CU
bool gemm_nt_f32_uses_ws(int M, int N, int K) {
    const long tiles = (long)((M + 127) / 128) * ((N + 127) / 128);
    return K % 32 == 0 && tiles >= 64 && tiles < 2 * GEMM_SK_GROUPS && tiles * (K / 32) >= 4 * GEMM_SK_GROUPS;
}

hipError_t launch_gemm_nt_f32(const float* A, const float* W, const float* R, float* C, int M, int N, int K,
                              hipStream_t s, float* ws) {
    const int mtiles = (M + 127) / 128, tiles = mtiles * ((N + 127) / 128);
    GemmArgs p{A, W, R, C, M, N, K, mtiles, tiles, 0, ws};
    if (M <= 16) {
        const dim3 grid((unsigned)((N + 4 * GV_RPW - 1) / (4 * GV_RPW)));
        // rows 8.. go through a second pass over W (M <= 16 keeps it at two)
        for (int m0 = 0; m0 < M; m0 += 8) {
            const int mb = min(M - m0, 8);
            const float* a = A + (size_t)m0 * K;
            const float* r = R ? R + (size_t)m0 * N : nullptr;
            float* c = C + (size_t)m0 * N;
            if (mb == 1)
                hipLaunchKernelGGL((gemv_nt_f32_kernel<1, 4>), grid, dim3(256), 0, s, a, W, r, c, mb, N, K);
            else if (mb == 2)
                hipLaunchKernelGGL((gemv_nt_f32_kernel<2, 4>), grid, dim3(256), 0, s, a, W, r, c, mb, N, K);
            else if (mb <= 4)
                hipLaunchKernelGGL((gemv_nt_f32_kernel<4, 4>), grid, dim3(256), 0, s, a, W, r, c, mb, N, K);
            else
                hipLaunchKernelGGL((gemv_nt_f32_kernel<8, 3>), grid, dim3(256), 0, s, a, W, r, c, mb, N, K);
        }
        return hipGetLastError();
    }
    if (ws && gemm_nt_f32_uses_ws(M, N, K)) {
        p.G = GEMM_SK_GROUPS;
        hipLaunchKernelGGL((gemm_nt_f32_lds_kernel<32, 2, 2>), dim3(p.G), dim3(256), 0, s, p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(gemm_fixup_kernel, dim3(tiles, 64 / FIX_Q), dim3(256), 0, s, p, K / 32);
    } else if (tiles >= 512) {
        if (K % 32 == 0)
            hipLaunchKernelGGL((gemm_nt_f32_lds_kernel<32, 2, 2>), dim3(tiles), dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL((gemm_nt_f32_lds_kernel<16, 3, 3>), dim3(tiles), dim3(256), 0, s, p);
    } else {
        const dim3 grid((N + 63) / 64, (M + 63) / 64);
        hipLaunchKernelGGL((gemm_nt_f32_kernel<1, 1>), grid, dim3(64), 0, s, A, W, R, C, M, N, K);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- RoPE + QK-norm
// One wave per (token, group of RQ_HEADS heads): the rotation angles depend on
// (token, pair) only, so each wave computes them once for its group.  Lane l owns
// pairs l and l + 64 (head_dim <= 256) and moves them as float2.  Key heads also copy
// their value row.
constexpr int RQ_HEADS = 4;
__global__ __launch_bounds__(256) void rope_qknorm_kernel(RopeNormArgs a) {
    const int heads = a.nh + a.nkv;
    const int groups = (heads + RQ_HEADS - 1) / RQ_HEADS;
    const int wid = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (wid >= a.T * groups) return;
    const int t = wid / groups, h0 = (wid % groups) * RQ_HEADS;
    const int hd = a.hd, npair = hd / 2;
    const float pos = a.positions ? (float)a.positions[t] : (float)t;
    constexpr int MAXP = 2;  // pairs per lane: hd <= 256
    float cs[MAXP], sn[MAXP];
#pragma unroll
    for (int i = 0; i < MAXP; i++) {
        const int d = lane + WAVE * i;
        cs[i] = 1.0f;
        sn[i] = 0.0f;
        if (d >= npair) continue;
        if (a.mode == ROPE_1D) {
            const float freq = 1.0f / powf(a.theta, (2.0f * (float)d) / (float)hd);
            cs[i] = cosf(pos * freq);
            sn[i] = sinf(pos * freq);
        } else if (a.mode == ROPE_TABLE) {
            cs[i] = a.cos_t[(size_t)t * hd + 2 * d];
            sn[i] = a.sin_t[(size_t)t * hd + 2 * d];
        }
    }
    const bool rot = a.mode != ROPE_NONE;
    // the group's rows, loaded together
    float2 x[RQ_HEADS][MAXP];
#pragma unroll
    for (int j = 0; j < RQ_HEADS; j++)
#pragma unroll
        for (int i = 0; i < MAXP; i++) {
            const int d = lane + WAVE * i, hh = h0 + j;
            x[j][i] = (d < npair && hh < heads)
                          ? *reinterpret_cast<const float2*>(a.qkv + (size_t)t * a.nqkv + (size_t)hh * hd + 2 * d)
                          : make_float2(0.0f, 0.0f);
        }
#pragma unroll
    for (int j = 0; j < RQ_HEADS; j++) {
        const int hh = h0 + j;
        if (hh >= heads) break;  // wave-uniform
        const bool is_q = hh < a.nh;
        float r0[MAXP], r1[MAXP];
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < MAXP; i++) {
            const float x0 = x[j][i].x, x1 = x[j][i].y;
            r0[i] = rot ? x0 * cs[i] - x1 * sn[i] : x0;
            r1[i] = rot ? x0 * sn[i] + x1 * cs[i] : x1;
            ss += r0[i] * r0[i];
            ss += r1[i] * r1[i];
        }
        ss = wave_sum(ss);
        const float rms = 1.0f / sqrtf(ss / (float)hd + a.eps);
        const float* w = is_q ? a.q_norm : a.k_norm;
        float* dst = is_q ? a.q + ((size_t)t * a.nh + hh) * hd : a.k + ((size_t)(hh - a.nh) * a.L + a.pos0 + t) * hd;
#pragma unroll
        for (int i = 0; i < MAXP; i++) {
            const int d = lane + WAVE * i;
            if (d >= npair) continue;
            const float2 wv = *reinterpret_cast<const float2*>(w + 2 * d);
            // (x * rms) * w as attention_forward_cpu; x * (rms * w) as the cache branch
            const float o0 = a.norm_assoc ? r0[i] * (rms * wv.x) : r0[i] * rms * wv.x;
            const float o1 = a.norm_assoc ? r1[i] * (rms * wv.y) : r1[i] * rms * wv.y;
            *reinterpret_cast<float2*>(dst + 2 * d) = make_float2(o0, o1);
        }
        if (!is_q) {  // the value row of this kv head, unchanged
            const float* vs = a.qkv + (size_t)t * a.nqkv + (size_t)(a.nh + a.nkv) * hd + (size_t)(hh - a.nh) * hd;
            float* vd = a.v + ((size_t)(hh - a.nh) * a.L + a.pos0 + t) * hd;
            for (int d = 2 * lane; d < hd; d += 2 * WAVE)
                *reinterpret_cast<float2*>(vd + d) = *reinterpret_cast<const float2*>(vs + d);
        }
    }
}

hipError_t launch_rope_qknorm(const RopeNormArgs& a, hipStream_t s) {
    const int waves = a.T * ((a.nh + a.nkv + RQ_HEADS - 1) / RQ_HEADS);
    hipLaunchKernelGGL(rope_qknorm_kernel, dim3((waves + 3) / 4), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------- 2D rotary tables
// build_2d_rope (src/hunyuan_image_gen.cpp:11-69): one thread per (position, pair).
__global__ void rope2d_table_kernel(int seq, int n_elem, int text_len, int img_h, int img_w, float base,
                                    float* __restrict__ cos_out, float* __restrict__ sin_out) {
    const int half = n_elem / 2;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= seq * half) return;
    const int p = idx / half, d = idx % half;
    float py, px;
    if (p < text_len) {
        py = (float)p;
        px = (float)p;
    } else {
        const int i = p - text_len, row = i / img_w, col = i % img_w;
        py = (float)text_len + (float)(img_h * img_w - img_h) / 2.0f + (float)row;
        px = (float)text_len + (float)(img_h * img_w - img_w) / 2.0f + (float)col;
    }
    const float th = 1.0f / powf(base, (2.0f * (float)d) / (float)n_elem);
    const float ang = (((d / 2) % 2) == 0 ? py : px) * th;
    const float c = cosf(ang), sn = sinf(ang);
    cos_out[(size_t)p * n_elem + 2 * d] = c;
    cos_out[(size_t)p * n_elem + 2 * d + 1] = c;
    sin_out[(size_t)p * n_elem + 2 * d] = sn;
    sin_out[(size_t)p * n_elem + 2 * d + 1] = sn;
}

hipError_t launch_rope2d_table(int seq, int n_elem, int text_len, int img_h, int img_w, float base, float* cos_out,
                               float* sin_out, hipStream_t s) {
    const int n = seq * (n_elem / 2);
    hipLaunchKernelGGL(rope2d_table_kernel, dim3((n + 255) / 256), dim3(256), 0, s, seq, n_elem, text_len, img_h,
                       img_w, base, cos_out, sin_out);
    return hipGetLastError();
}

// ---------------------------------------------------------------- flash attention
// LDS row pitches (floats): K rows are read 16 B per lane by 32 rows (pitch = 4 mod
// 64 banks: 16 consecutive rows hit 16 distinct bank quads); V rows 4 B per lane by
// two rows 4 apart per instruction (pitch = 8 mod 16: the two half-waves land on
// opposite bank halves).
// K / V blocks of 32 keys reach LDS by DMA (global_load_lds_dwordx4) into a 2-deep
// ring: the next block's copies are in flight during a block's math, no registers
// hold them, and one barrier per block suffices.  Rows are HD floats (HD / 4 16-byte
// chunks), unpadded; chunk c of K row r sits at position c ^ (r & 15) and chunk c of V
// row r at c ^ 8 ((r >> 2) & 1).  Then the K reads of 16 consecutive rows at one
// logical chunk (QK^T) and the V reads of rows key and key + 4 by the two half-waves
// (PV) fall on distinct bank groups.  Each lane of a copy fetches the chunk that
// belongs at its position.
template <int HD>
struct FaShape {
    static constexpr int ROWB = HD * 4;         // bytes per row
    static constexpr int BLK = 32 * ROWB;       // one K (or V) block
    static constexpr int BUF = 2 * BLK;         // K block, then V block
    static constexpr int CPW = BLK / 1024 / 4;  // 1 KB copies per wave for K (and for V)
    static constexpr int RPC = 1024 / ROWB;     // rows per copy
    static_assert(CPW >= 1 && HD / 4 >= 16, "head_dim 64 or 128");
};
__device__ __forceinline__ int fa_swz_k(int r) { return r & 15; }
__device__ __forceinline__ int fa_swz_v(int r) { return 8 * ((r >> 2) & 1); }

template <int HD>
__global__ __launch_bounds__(256, 2) void flash_attn_kernel(FlashArgs a) {
    using S = FaShape<HD>;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[2][S::BUF];
    const int tid = threadIdx.x, lane = tid % WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int lr = lane % 32, h = lane / 32;
    const int n_qt = (a.T + 31) / 32;
    // chunk-major, and inside a chunk the longest (causal) query tiles first
    const int per_chunk = n_qt * a.nkv;
    const int chunk = (int)blockIdx.x / per_chunk, rem = (int)blockIdx.x % per_chunk;
    const int qt = n_qt - 1 - rem / a.nkv;
    const int g = rem % a.nkv;
    const int q0 = qt * 32;
    const int head = g * 4 + wave;  // 4 query heads per kv group
    const int qrow = min(q0 + lr, a.T - 1);

    // visible keys: all kv_len, or (causal) keys <= q_pos0 + q
    const int last_q = min(q0 + 31, a.T - 1);
    const int key_end = a.causal ? min(a.kv_len, a.q_pos0 + last_q + 1) : a.kv_len;
    const int nblk = (key_end + 31) / 32;
    // this work group's key blocks: all of them, or chunk `chunk` of cb blocks
    const int nc = a.cb ? (nblk + a.cb - 1) / a.cb : 1;
    if (chunk >= nc) return;  // whole work group: the tile has fewer chunks
    const int kb0 = a.cb ? chunk * a.cb : 0, kb1 = a.cb ? min(nblk, kb0 + a.cb) : nblk;

    // copies: copy q of this wave moves rows (wave CPW + q) RPC .. + RPC - 1 of the
    // block; lane l lands at byte 16 l of it: row + l / (ROWB / 16), position
    // l % (ROWB / 16), fetching the chunk stored there
    const float* kg = a.k + (size_t)g * a.L * HD;
    const float* vg = a.v + (size_t)g * a.L * HD;
    int crow[S::CPW], kchunk[S::CPW], vchunk[S::CPW];
#pragma unroll
    for (int q = 0; q < S::CPW; q++) {
        crow[q] = (wave * S::CPW + q) * S::RPC + lane / (S::ROWB / 16);
        const int pos = lane % (S::ROWB / 16);
        kchunk[q] = 4 * (pos ^ fa_swz_k(crow[q]));
        vchunk[q] = 4 * (pos ^ fa_swz_v(crow[q]));
    }
    auto issue = [&](int kb) {
        uint8_t* buf = ring[(kb - kb0) & 1];
#pragma unroll
        for (int q = 0; q < S::CPW; q++) {
            const size_t row = (size_t)min(kb * 32 + crow[q], a.kv_len - 1) * HD;  // in bounds
            g2l16(kg + row + kchunk[q], buf + (wave * S::CPW + q) * 1024);
            g2l16(vg + row + vchunk[q], buf + S::BLK + (wave * S::CPW + q) * 1024);
        }
    };
    issue(kb0);

    // Q resident: lane (query lr, half h) holds Q[q][16c + 8h + j], pre-multiplied by
    // scale * log2(e): the scores come out in the base-2 domain, where the softmax uses
    // the hardware 2^x (v_exp_f32; 2^-inf = 0 serves the masked keys)
    const float qscale = a.scale * 1.4426950408889634f;
    float qv[HD / 2];
    {
        const float* qp = a.q + ((size_t)qrow * a.nh + head) * HD + 8 * h;
#pragma unroll
        for (int c = 0; c < HD / 16; c++) {
            const v4f_t x0 = *reinterpret_cast<const v4f_t*>(qp + 16 * c);
            const v4f_t x1 = *reinterpret_cast<const v4f_t*>(qp + 16 * c + 4);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                qv[8 * c + j] = x0[j] * qscale;
                qv[8 * c + 4 + j] = x1[j] * qscale;
            }
        }
    }
    // LDS read offsets inside a buffer: K row lr at logical chunk 4c + 2h + t; V rows
    // 8 i + 4 h + j at float 32 c + lr (the row part 8 i + j is an immediate)
    const int swk = fa_swz_k(lr);
    uint32_t voff[HD / 32];
#pragma unroll
    for (int c = 0; c < HD / 32; c++) voff[c] = (uint32_t)(S::BLK + 4 * h * S::ROWB + 128 * (c ^ h) + 4 * lr);
    const uint32_t ring0 = lds_off(ring[0]);

    v16f_t o[HD / 32];
#pragma unroll
    for (int c = 0; c < HD / 32; c++) o[c] = v16f_t{};
    float m_run = -INFINITY, l_run = 0.0f;
    const int my_q = a.q_pos0 + q0 + lr;  // key index of this lane's query (causal bound)

    for (int kb = kb0; kb < kb1; kb++) {
        MM_WAIT_VM_LGKM(0);  // this wave's copies of block kb have landed
        __syncthreads();     // everyone's have, and block kb - 1's buffer is free
        if (kb + 1 < kb1) issue(kb + 1);
        const uint32_t base = ring0 + (uint32_t)(((kb - kb0) & 1) * S::BUF);
        // S^T[key][q] = sum_d K[key][d] Q[q][d]: all K reads of the block in flight,
        // consumed in order
        const uint32_t krow = base + (uint32_t)(lr * S::ROWB);
        v4i_t kr[HD / 16][2];
#pragma unroll
        for (int c = 0; c < HD / 16; c++)
#pragma unroll
            for (int t = 0; t < 2; t++) kr[c][t] = lds_b128_at<0>(krow + 16u * (uint32_t)((4 * c + 2 * h + t) ^ swk));
        v16f_t s = v16f_t{};
        [&]<int... C>(std::integer_sequence<int, C...>) {
            (
                [&] {
                    lds_wait_upto<HD / 8 - 2 - 2 * C>();
                    lds_pin(kr[C][0]);
                    lds_pin(kr[C][1]);
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        s = mfma_f32(__int_as_float(kr[C][j / 4][j % 4]), qv[8 * C + j], s);
                }(),
                ...);
        }(std::make_integer_sequence<int, HD / 16>{});
        // mask (only blocks that reach past the tile's first query or past kv_len),
        // online softmax over this lane pair's 32 keys
        const bool need_mask = kb * 32 + 31 >= a.kv_len || (a.causal && kb * 32 + 31 > a.q_pos0 + q0);
        if (need_mask) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int key = kb * 32 + 8 * (v / 4) + 4 * h + v % 4;
                if (key >= a.kv_len || (a.causal && key > my_q)) s[v] = -INFINITY;
            }
        }
        float mloc = s[0];
#pragma unroll
        for (int v = 1; v < 16; v++) mloc = fmaxf(mloc, s[v]);
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, WAVE));
        // every processed block leaves at least one visible key per query, so m_new is
        // finite
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 for the first block
        float psum = 0.0f;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float p = __builtin_amdgcn_exp2f(s[v] - m_new);
            s[v] = p;
            psum += p;
        }
        psum += __shfl_xor(psum, 32, WAVE);
        l_run = l_run * alpha + psum;
        m_run = m_new;
        if (__ballot(alpha != 1.0f)) {  // the running max moved for some query
#pragma unroll
            for (int c = 0; c < HD / 32; c++) o[c] *= alpha;
        }
        // O^T[d][q] += sum_key V[key][d] P^T[key][q]: per 32 dims, the 16 key values
        // of the lane in two groups of 8 reads
#pragma unroll
        for (int c = 0; c < HD / 32; c++) {
            const uint32_t vb = base + voff[c];
            uint32_t vv[16];
            [&]<int... V>(std::integer_sequence<int, V...>) {
                ((vv[V] = lds_b32_at<(8 * (V / 4) + V % 4) * S::ROWB>(vb)), ...);
            }(std::make_integer_sequence<int, 16>{});
            lds_wait_upto<8>();
#pragma unroll
            for (int v = 0; v < 8; v++) {
                lds_pin(vv[v]);
                o[c] = mfma_f32(__uint_as_float(vv[v]), s[v], o[c]);
            }
            lds_wait_upto<0>();
#pragma unroll
            for (int v = 8; v < 16; v++) {
                lds_pin(vv[v]);
                o[c] = mfma_f32(__uint_as_float(vv[v]), s[v], o[c]);
            }
        }
    }
    if (nc > 1) {
        // partial result of this chunk: unnormalised O^T, running max and sum
        float* pp = a.part + ((size_t)((qt * a.nch + chunk) * a.nkv + g) * 4 + wave) * (HD * 32 + 128);
#pragma unroll
        for (int c = 0; c < HD / 32; c++)
#pragma unroll
            for (int v = 0; v < 16; v++) pp[(c * 16 + v) * 64 + lane] = o[c][v];
        pp[HD * 32 + lane] = m_run;
        pp[HD * 32 + 64 + lane] = l_run;
        return;
    }
    if (q0 + lr >= a.T) return;
    const float inv = 1.0f / l_run;
    float* op = a.out + ((size_t)(q0 + lr) * a.nh + head) * HD;
#pragma unroll
    for (int c = 0; c < HD / 32; c++)
#pragma unroll
        for (int v4 = 0; v4 < 4; v4++) {
            const int d = 32 * c + 8 * v4 + 4 * h;
            *reinterpret_cast<float4*>(op + d) = make_float4(o[c][4 * v4] * inv, o[c][4 * v4 + 1] * inv,
                                                             o[c][4 * v4 + 2] * inv, o[c][4 * v4 + 3] * inv);
        }
}

// Join the chunks of every split query tile: work group (tile x kv group, piece y)
// takes 4 of the output values of every thread of the attention kernel's layout
// (y = 4 cc + v4: dims 32 cc + 8 v4 + 4 h .. + 3 of query lr).  With M = max_c m_c,
// O = sum_c 2^(m_c - M) O_c and l = sum_c 2^(m_c - M) l_c in chunk order; out = O / l.
template <int HD>
__global__ __launch_bounds__(256) void flash_merge_kernel(FlashArgs a) {
    const int qt = (int)blockIdx.x / a.nkv, g = (int)blockIdx.x % a.nkv;
    const int q0 = qt * 32;
    const int last_q = min(q0 + 31, a.T - 1);
    const int key_end = a.causal ? min(a.kv_len, a.q_pos0 + last_q + 1) : a.kv_len;
    const int nblk = (key_end + 31) / 32;
    const int nc = (nblk + a.cb - 1) / a.cb;
    if (nc <= 1) return;  // written directly by the attention kernel
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int lr = lane % 32, h = lane / 32;
    if (q0 + lr >= a.T) return;
    const int head = g * 4 + wave;
    const int cc = (int)blockIdx.y / 4, v4 = (int)blockIdx.y % 4;
    const float* __restrict__ base = a.part + ((size_t)(qt * a.nch * a.nkv + g) * 4 + wave) * (HD * 32 + 128);
    const size_t cstride = (size_t)a.nkv * 4 * (HD * 32 + 128);  // chunk c + 1 of the same tile
    // the chunks' running maxima are in the base-2 domain of the attention kernel
    float mx = -INFINITY;
    for (int c = 0; c < nc; c++) mx = fmaxf(mx, base[c * cstride + HD * 32 + lane]);
    float l = 0.0f, r0 = 0.0f, r1 = 0.0f, r2 = 0.0f, r3 = 0.0f;
    for (int c = 0; c < nc; c++) {
        const float* pp = base + c * cstride;
        const float mc = pp[HD * 32 + lane], lc = pp[HD * 32 + 64 + lane];
        const float* ov = pp + (cc * 16 + 4 * v4) * 64 + lane;
        const float o0 = ov[0], o1 = ov[64], o2 = ov[128], o3 = ov[192];
        const float wgt = __builtin_amdgcn_exp2f(mc - mx);
        l += wgt * lc;
        r0 += wgt * o0;
        r1 += wgt * o1;
        r2 += wgt * o2;
        r3 += wgt * o3;
    }
    const float inv = 1.0f / l;
    const int d = 32 * cc + 8 * v4 + 4 * h;
    *reinterpret_cast<float4*>(a.out + ((size_t)(q0 + lr) * a.nh + head) * HD + d) =
        make_float4(r0 * inv, r1 * inv, r2 * inv, r3 * inv);
}

// ---------------------------------------------------------------- decode (T <= 8)
// A few new tokens against a long cache: the 4 query heads of a kv group times the T
// tokens pack into one 32-row tile (row r: token r / 4, head 4 g + r % 4), so a single
// wave covers the whole group for a block of keys, and the keys spread over as many
// waves as the chip holds.  Every wave is a work group of its own and takes cb
// consecutive key blocks of one group: K and V of a block reach its own LDS buffer by
// DMA, in the prompt kernel's swizzled layout, read by the same MFMA steps.  The wave
// writes unnormalised O, running max and sum of its 4T live rows;
// flash_decode_merge_kernel joins the waves of a group.
template <int HD>
__global__ __launch_bounds__(64) void flash_decode_kernel(FlashArgs a) {
    using S = FaShape<HD>;
    constexpr int NCP = S::BLK / 1024;  // 1 KB copies per block of K (and of V)
    __shared__ __attribute__((aligned(1024))) uint8_t buf[S::BUF];
    const int lane = threadIdx.x, lr = lane % 32, h = lane / 32;
    const int g = (int)blockIdx.x / a.nch, w = (int)blockIdx.x % a.nch;
    const int t = min(lr / 4, a.T - 1), head = g * 4 + lr % 4;
    const int key_end = a.causal ? min(a.kv_len, a.q_pos0 + a.T) : a.kv_len;
    const int nblk = (key_end + 31) / 32;
    const int kb0 = w * a.cb, kb1 = min(nblk, kb0 + a.cb);  // kb0 < nblk: nch = ceil(nblk / cb)

    const float* kg = a.k + (size_t)g * a.L * HD;
    const float* vg = a.v + (size_t)g * a.L * HD;
    const int pos = lane % (S::ROWB / 16);
    // K copies of a block, then its V copies (copies complete in issue order): QK^T
    // starts once K has landed, while V is still on its way
    auto issue = [&](int kb, const float* src, int (*swz)(int), int off) {
#pragma unroll
        for (int q = 0; q < NCP; q++) {
            const int r = q * S::RPC + lane / (S::ROWB / 16);
            const size_t row = (size_t)min(kb * 32 + r, a.kv_len - 1) * HD;  // in bounds
            g2l16(src + row + 4 * (pos ^ swz(r)), buf + off + q * 1024);
        }
    };
    // Q first: its loads then complete ahead of the block copies issued after them
    const float qscale = a.scale * 1.4426950408889634f;
    float qv[HD / 2];
    {
        const float* qp = a.q + ((size_t)t * a.nh + head) * HD + 8 * h;
#pragma unroll
        for (int c = 0; c < HD / 16; c++) {
            const v4f_t x0 = *reinterpret_cast<const v4f_t*>(qp + 16 * c);
            const v4f_t x1 = *reinterpret_cast<const v4f_t*>(qp + 16 * c + 4);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                qv[8 * c + j] = x0[j] * qscale;
                qv[8 * c + 4 + j] = x1[j] * qscale;
            }
        }
    }
    issue(kb0, kg, fa_swz_k, 0);
    issue(kb0, vg, fa_swz_v, S::BLK);
    MM_WAIT_VM_LGKM(2 * NCP);  // Q has landed (older than the copies): nothing of it is pending in the loop

    const int swk = fa_swz_k(lr);
    uint32_t voff[HD / 32];
#pragma unroll
    for (int c = 0; c < HD / 32; c++) voff[c] = (uint32_t)(S::BLK + 4 * h * S::ROWB + 128 * (c ^ h) + 4 * lr);
    const uint32_t base = lds_off(buf);

    v16f_t o[HD / 32];
#pragma unroll
    for (int c = 0; c < HD / 32; c++) o[c] = v16f_t{};
    float m_run = -INFINITY, l_run = 0.0f;
    const int my_q = a.q_pos0 + t;

    for (int kb = kb0; kb < kb1; kb++) {
        MM_WAIT_VM_LGKM(NCP);  // K of block kb is in LDS
        const uint32_t krow = base + (uint32_t)(lr * S::ROWB);
        v4i_t kr[HD / 16][2];
#pragma unroll
        for (int c = 0; c < HD / 16; c++)
#pragma unroll
            for (int u = 0; u < 2; u++) kr[c][u] = lds_b128_at<0>(krow + 16u * (uint32_t)((4 * c + 2 * h + u) ^ swk));
        v16f_t s = v16f_t{};
        [&]<int... C>(std::integer_sequence<int, C...>) {
            (
                [&] {
                    lds_wait_upto<HD / 8 - 2 - 2 * C>();
                    lds_pin(kr[C][0]);
                    lds_pin(kr[C][1]);
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        s = mfma_f32(__int_as_float(kr[C][j / 4][j % 4]), qv[8 * C + j], s);
                }(),
                ...);
        }(std::make_integer_sequence<int, HD / 16>{});
        // every K read has returned: the K half of the buffer takes the next block's K
        const bool more = kb + 1 < kb1;
        if (more) issue(kb + 1, kg, fa_swz_k, 0);
        const bool need_mask = kb * 32 + 31 >= a.kv_len || (a.causal && kb * 32 + 31 > a.q_pos0);
        if (need_mask) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int key = kb * 32 + 8 * (v / 4) + 4 * h + v % 4;
                if (key >= a.kv_len || (a.causal && key > my_q)) s[v] = -INFINITY;
            }
        }
        float mloc = s[0];
#pragma unroll
        for (int v = 1; v < 16; v++) mloc = fmaxf(mloc, s[v]);
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, WAVE));
        // a wave's blocks may hide every key from a causal row (the cache's last block
        // against an earlier new token): its max stays -inf, its weights 0
        const float m_new = fmaxf(m_run, mloc);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        float psum = 0.0f;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float p = __builtin_amdgcn_exp2f(s[v] - m_use);
            s[v] = p;
            psum += p;
        }
        psum += __shfl_xor(psum, 32, WAVE);
        l_run = l_run * alpha + psum;
        m_run = m_new;
        if (__ballot(alpha != 1.0f)) {
#pragma unroll
            for (int c = 0; c < HD / 32; c++) o[c] *= alpha;
        }
        if (more)  // V of block kb landed; the next block's K may still be in flight
            MM_WAIT_VM_LGKM(NCP);
        else
            MM_WAIT_VM_LGKM(0);
#pragma unroll
        for (int c = 0; c < HD / 32; c++) {
            const uint32_t vb = base + voff[c];
            uint32_t vv[16];
            [&]<int... V>(std::integer_sequence<int, V...>) {
                ((vv[V] = lds_b32_at<(8 * (V / 4) + V % 4) * S::ROWB>(vb)), ...);
            }(std::make_integer_sequence<int, 16>{});
            lds_wait_upto<8>();
#pragma unroll
            for (int v = 0; v < 8; v++) {
                lds_pin(vv[v]);
                o[c] = mfma_f32(__uint_as_float(vv[v]), s[v], o[c]);
            }
            lds_wait_upto<0>();
#pragma unroll
            for (int v = 8; v < 16; v++) {
                lds_pin(vv[v]);
                o[c] = mfma_f32(__uint_as_float(vv[v]), s[v], o[c]);
            }
        }
        // every V read has returned (lgkmcnt 0): the V half takes the next block's V
        if (more) issue(kb + 1, vg, fa_swz_v, S::BLK);
    }
    if (lr >= 4 * a.T) return;
    // partial of wave w of group g: O rows [32][HD], then m [32], l [32]
    float* pp = a.part + (size_t)blockIdx.x * (32 * HD + 64);
#pragma unroll
    for (int c = 0; c < HD / 32; c++)
#pragma unroll
        for (int v4 = 0; v4 < 4; v4++) {
            const int d = 32 * c + 8 * v4 + 4 * h;
            *reinterpret_cast<v4f_t*>(pp + lr * HD + d) =
                v4f_t{o[c][4 * v4], o[c][4 * v4 + 1], o[c][4 * v4 + 2], o[c][4 * v4 + 3]};
        }
    if (h == 0) {
        pp[32 * HD + lr] = m_run;
        pp[32 * HD + 32 + lr] = l_run;
    }
}

// The same for T <= 4 (16 live rows): 16 x 16 x 4 fp32 MFMA tiles, half the matrix
// work of the 32-row tile.  Lane l: kq = l % 16, kk = l / 16.
//   S^T[key][q] (two halves of 16 keys): step j takes d = (HD / 4) kk + j, lane
//     supplying K[16 hf + kq][d] and Q[kq][d]; lane l ends with S of query l % 16 and
//     keys 16 hf + 4 (l / 16) + v.
//   O^T[d][q] (HD / 16 tiles of 16 dims): step j takes keys 16 (j / 4) + 4 kk + j % 4,
//     lane supplying V[key][16 dt + kq] and its own P; lane l ends with O of query
//     l % 16, dims 16 dt + 4 (l / 16) + v.
// V sits at chunk position c ^ (8 ((r >> 2) & 1) + 4 ((r >> 3) & 1)): the four key rows
// of one read (4 kk + const) fall on four different 16-chunk bank groups.
__device__ __forceinline__ int fa_swz_vd(int r) { return 8 * ((r >> 2) & 1) + 4 * ((r >> 3) & 1); }

template <int HD>
__global__ __launch_bounds__(64) void flash_decode16_kernel(FlashArgs a) {
    using S = FaShape<HD>;
    constexpr int NCP = S::BLK / 1024;
    constexpr int KR = HD / 16;  // 16-byte K reads per half
    __shared__ __attribute__((aligned(1024))) uint8_t buf[S::BUF];
    const int lane = threadIdx.x, kq = lane % 16, kk = lane / 16;
    const int g = (int)blockIdx.x / a.nch, w = (int)blockIdx.x % a.nch;
    const int key_end = a.causal ? min(a.kv_len, a.q_pos0 + a.T) : a.kv_len;
    const int nblk = (key_end + 31) / 32;
    const int kb0 = w * a.cb, kb1 = min(nblk, kb0 + a.cb);

    const float* kg = a.k + (size_t)g * a.L * HD;
    const float* vg = a.v + (size_t)g * a.L * HD;
    const int pos = lane % (S::ROWB / 16);
    auto issue = [&](int kb, const float* src, int (*swz)(int), int off) {
#pragma unroll
        for (int q = 0; q < NCP; q++) {
            const int r = q * S::RPC + lane / (S::ROWB / 16);
            const size_t row = (size_t)min(kb * 32 + r, a.kv_len - 1) * HD;  // in bounds
            g2l16(src + row + 4 * (pos ^ swz(r)), buf + off + q * 1024);
        }
    };
    // Q first: its loads then complete ahead of the block copies issued after them
    const float qscale = a.scale * 1.4426950408889634f;
    float qv[HD / 4];
    {
        const int t = min(kq / 4, a.T - 1), head = g * 4 + kq % 4;
        const float* qp = a.q + ((size_t)t * a.nh + head) * HD + (HD / 4) * kk;
#pragma unroll
        for (int c = 0; c < HD / 16; c++) {
            const v4f_t x = *reinterpret_cast<const v4f_t*>(qp + 4 * c);
#pragma unroll
            for (int j = 0; j < 4; j++) qv[4 * c + j] = x[j] * qscale;
        }
    }
    issue(kb0, kg, fa_swz_k, 0);
    issue(kb0, vg, fa_swz_vd, S::BLK);
    MM_WAIT_VM_LGKM(2 * NCP);  // Q has landed (older than the copies): nothing of it is pending in the loop

    const uint32_t base = lds_off(buf);
    // K: row 16 hf + kq, logical chunks (HD / 16) kk + m at position ^ kq
    const uint32_t krow = base + (uint32_t)(kq * S::ROWB);
    // V: rows 4 kk (+ 16 hf + v, immediate), logical chunk 4 dt + kq / 4 at position
    // 4 (dt ^ sv) + kq / 4 with sv = the row's swizzle / 4 (dt = 4 dh + dl: dh immediate)
    const int sv = fa_swz_vd(4 * kk) / 4;
    uint32_t voff[4];
#pragma unroll
    for (int dl = 0; dl < 4; dl++)
        voff[dl] = base + (uint32_t)(S::BLK + 4 * kk * S::ROWB + 64 * (dl ^ sv) + 4 * kq);

    v4f_t o[HD / 16];
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++) o[dt] = v4f_t{};
    float m_run = -INFINITY, l_run = 0.0f;
    const int my_q = a.q_pos0 + min(kq / 4, a.T - 1);  // lane's query: l % 16

    for (int kb = kb0; kb < kb1; kb++) {
        MM_WAIT_VM_LGKM(NCP);  // K of block kb is in LDS
        v4i_t kr[2][KR];
#pragma unroll
        for (int hf = 0; hf < 2; hf++)
#pragma unroll
            for (int m = 0; m < KR; m++)
                kr[hf][m] = lds_b128_at<0>(krow + (uint32_t)(16 * hf * S::ROWB) +
                                           16u * (uint32_t)(((HD / 16) * kk + m) ^ kq));
        v4f_t sc[2] = {v4f_t{}, v4f_t{}};
        [&]<int... I>(std::integer_sequence<int, I...>) {
            (
                [&] {
                    constexpr int hf = I / KR, m = I % KR;
                    lds_wait_upto<2 * KR - 1 - I>();
                    lds_pin(kr[hf][m]);
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        sc[hf] = __builtin_amdgcn_mfma_f32_16x16x4f32(__int_as_float(kr[hf][m][j]), qv[4 * m + j],
                                                                    sc[hf], 0, 0, 0);
                }(),
                ...);
        }(std::make_integer_sequence<int, 2 * KR>{});
        const bool more = kb + 1 < kb1;
        if (more) issue(kb + 1, kg, fa_swz_k, 0);
        const bool need_mask = kb * 32 + 31 >= a.kv_len || (a.causal && kb * 32 + 31 > a.q_pos0);
        if (need_mask) {
#pragma unroll
            for (int hf = 0; hf < 2; hf++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int key = kb * 32 + 16 * hf + 4 * kk + v;
                    if (key >= a.kv_len || (a.causal && key > my_q)) sc[hf][v] = -INFINITY;
                }
        }
        float mloc = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                           fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16, WAVE));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, WAVE));
        const float m_new = fmaxf(m_run, mloc);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        float psum = 0.0f;
#pragma unroll
        for (int hf = 0; hf < 2; hf++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float p = __builtin_amdgcn_exp2f(sc[hf][v] - m_use);
                sc[hf][v] = p;
                psum += p;
            }
        psum += __shfl_xor(psum, 16, WAVE);
        psum += __shfl_xor(psum, 32, WAVE);
        l_run = l_run * alpha + psum;
        m_run = m_new;
        if (__ballot(alpha != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < HD / 16; dt++) o[dt] *= alpha;
        }
        if (more)
            MM_WAIT_VM_LGKM(NCP);
        else
            MM_WAIT_VM_LGKM(0);
        // two dim tiles at a time: 16 reads in flight, consumed 8 and 8
        [&]<int... DP>(std::integer_sequence<int, DP...>) {
            (
                [&] {
                    constexpr int dt = 2 * DP;
                    uint32_t vv[2][8];
                    [&]<int... V>(std::integer_sequence<int, V...>) {
                        ((vv[V / 8][V % 8] = lds_b32_at<(16 * ((V % 8) / 4) + (V % 8) % 4) * S::ROWB +
                                                        256 * ((dt + V / 8) / 4)>(voff[(dt + V / 8) % 4])),
                         ...);
                    }(std::make_integer_sequence<int, 16>{});
                    lds_wait_upto<8>();
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        lds_pin(vv[0][j]);
                        o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(vv[0][j]), sc[j / 4][j % 4],
                                                                     o[dt], 0, 0, 0);
                    }
                    lds_wait_upto<0>();
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        lds_pin(vv[1][j]);
                        o[dt + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(vv[1][j]), sc[j / 4][j % 4],
                                                                         o[dt + 1], 0, 0, 0);
                    }
                }(),
                ...);
        }(std::make_integer_sequence<int, HD / 32>{});
        if (more) issue(kb + 1, vg, fa_swz_vd, S::BLK);
    }
    if (kq >= 4 * a.T) return;
    float* pp = a.part + (size_t)blockIdx.x * (32 * HD + 64);
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++) *reinterpret_cast<v4f_t*>(pp + kq * HD + 16 * dt + 4 * kk) = o[dt];
    if (kk == 0) {
        pp[32 * HD + kq] = m_run;
        pp[32 * HD + 32 + kq] = l_run;
    }
}

// Join the nch waves of a group for one row (work group = group x row): with
// M = max_w m_w, O = sum_w 2^(m_w - M) O_w and l likewise; out = O / l.  The work
// group's 1024 threads form 1024 / (HD / 4) teams of HD / 4 (one float4 of the row
// each); team j folds waves j, j + teams, ... in one pass with a running max, and the
// teams' results are joined in team order.
constexpr int FDM_THREADS = 1024;
template <int HD>
__global__ __launch_bounds__(FDM_THREADS) void flash_decode_merge_kernel(FlashArgs a) {
    constexpr int TPR = HD / 4, TEAMS = FDM_THREADS / TPR;
    constexpr size_t STRIDE = 32 * HD + 64;
    __shared__ v4f_t team_o[TEAMS][TPR];
    __shared__ float team_m[TEAMS], team_l[TEAMS];
    const int rows = 4 * a.T;
    const int g = (int)blockIdx.x / rows, r = (int)blockIdx.x % rows;
    const float* __restrict__ base = a.part + (size_t)g * a.nch * STRIDE;
    const int j = (int)threadIdx.x / TPR, d4 = (int)threadIdx.x % TPR;
    v4f_t acc = v4f_t{};
    float mt = -INFINITY, lt = 0.0f;
#pragma unroll 2
    for (int w = j; w < a.nch; w += TEAMS) {
        const float* pp = base + w * STRIDE;
        const float mw = pp[32 * HD + r], lw = pp[32 * HD + 32 + r];
        const v4f_t ov = *reinterpret_cast<const v4f_t*>(pp + r * HD + 4 * d4);
        const float m_new = fmaxf(mt, mw);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;  // a wave may see no key of this row
        const float a0 = __builtin_amdgcn_exp2f(mt - m_use), a1 = __builtin_amdgcn_exp2f(mw - m_use);
        acc = acc * a0 + ov * a1;
        lt = lt * a0 + lw * a1;
        mt = m_new;
    }
    team_o[j][d4] = acc;
    if (d4 == 0) {
        team_m[j] = mt;
        team_l[j] = lt;
    }
    __syncthreads();
    if (j != 0) return;
    float mx = team_m[0];
#pragma unroll
    for (int u = 1; u < TEAMS; u++) mx = fmaxf(mx, team_m[u]);  // finite: key 0 is visible to every row
    v4f_t sum = v4f_t{};
    float lsum = 0.0f;
#pragma unroll
    for (int u = 0; u < TEAMS; u++) {
        const float wgt = __builtin_amdgcn_exp2f(team_m[u] - mx);  // 0 for a team without waves
        sum += team_o[u][d4] * wgt;
        lsum += team_l[u] * wgt;
    }
    const float inv = 1.0f / lsum;
    const int tok = r / 4, head = g * 4 + r % 4;
    *reinterpret_cast<v4f_t*>(a.out + ((size_t)tok * a.nh + head) * HD + 4 * d4) = sum * inv;
}

int flash_attn_ws_slots(int max_tokens, int max_keys, int nkv) {
    const long n = (long)((max_tokens + 31) / 32) * ((max_keys + 31) / 32) * nkv;
    return (int)min(n, (long)FA_SPLIT_SLOTS);
}
size_t flash_attn_ws_floats(int hd, int slots) { return (size_t)slots * 4 * (hd * 32 + 128); }

hipError_t launch_flash_attn(const FlashArgs& a_in, hipStream_t s, float* ws, int ws_slots, int max_waves) {
    FlashArgs a = a_in;
    const int n_qt = (a.T + 31) / 32, base = n_qt * a.nkv;
    const int max_keys = a.causal ? min(a.kv_len, a.q_pos0 + a.T) : a.kv_len;
    const int max_nblk = (max_keys + 31) / 32;
    a.part = nullptr;
    a.cb = 0;
    a.nch = 1;
    // Split the keys of each query tile into chunks of cb blocks when that shortens the
    // launch.  Cost model, in units of one key block of one work group (~6.8 us at two
    // work groups per CU):
    //   whole tiles (longest first):  max(longest tile, all blocks / resident groups) + 1
    //   chunks of cb:                 rounds x (cb + 1) + partial-tile traffic
    // (+1: the ramp of a round; the partials are written and read back by the merge at
    // ~5 TB/s, ~34 MB per unit of time).  Short prompts, causal tiles of very different
    // lengths and decode against a long cache split; long prompts fill the chip with
    // whole tiles.
    if (a.T <= 8 && ws && max_nblk >= 2) {
        // decode: one wave per cb key blocks of a group, at most half as many waves as
        // are resident (LDS: 32 KB a wave at head_dim 128, 5 a CU; 16 KB at 64, 10 a
        // CU), or the caller's cap.  Two blocks a wave beat one (T=1 against 4,116
        // positions: 15.3-15.9 us for 520 waves, 18.9 us for 1,032): the second
        // block's K copy overlaps the first block's PV, and half the partials remain.
        const int resident = 256 * (a.hd == 128 ? 5 : 10);
        const int target = max_waves > 0 ? min(max_waves, resident) : resident / 2;
        int cb = (int)max(1L, ((long)max_nblk * a.nkv + target - 1) / target);
        int nw = (max_nblk + cb - 1) / cb;
        const size_t cap = flash_attn_ws_floats(a.hd, ws_slots);
        while (nw > 1 && (size_t)a.nkv * nw * (32 * a.hd + 64) > cap) nw = (max_nblk + ++cb - 1) / cb;
        a.cb = cb;
        a.nch = nw;
        a.part = ws;
        const dim3 grid((unsigned)(a.nkv * nw)), mgrid((unsigned)(a.nkv * 4 * a.T));
        if (a.T <= 4) {
            if (a.hd == 128)
                hipLaunchKernelGGL(flash_decode16_kernel<128>, grid, dim3(64), 0, s, a);
            else if (a.hd == 64)
                hipLaunchKernelGGL(flash_decode16_kernel<64>, grid, dim3(64), 0, s, a);
            else
                return hipErrorInvalidValue;
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            if (a.hd == 128)
                hipLaunchKernelGGL(flash_decode_merge_kernel<128>, mgrid, dim3(FDM_THREADS), 0, s, a);
            else
                hipLaunchKernelGGL(flash_decode_merge_kernel<64>, mgrid, dim3(FDM_THREADS), 0, s, a);
        } else if (a.hd == 128) {
            hipLaunchKernelGGL(flash_decode_kernel<128>, grid, dim3(64), 0, s, a);
            hipLaunchKernelGGL(flash_decode_merge_kernel<128>, mgrid, dim3(FDM_THREADS), 0, s, a);
        } else if (a.hd == 64) {
            hipLaunchKernelGGL(flash_decode_kernel<64>, grid, dim3(64), 0, s, a);
            hipLaunchKernelGGL(flash_decode_merge_kernel<64>, mgrid, dim3(FDM_THREADS), 0, s, a);
        } else {
            return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    const int slots = 256 * (a.hd == 128 ? 2 : 3);  // resident work groups (occupancy)
    if (ws && max_nblk >= 2) {
        auto tile_blocks = [&](int t) {
            const int kend = a.causal ? min(a.kv_len, a.q_pos0 + min(32 * t + 31, a.T - 1) + 1) : a.kv_len;
            return (kend + 31) / 32;
        };
        long total = 0;
        for (int t = 0; t < n_qt; t++) total += tile_blocks(t);
        total *= a.nkv;
        const double part_units = 2.0 * 4 * (a.hd * 32 + 128) * 4 / 34e6;  // per split unit
        double best = (double)max((long)max_nblk, (total + slots - 1) / slots) + 1;
        int best_cb = 0;
        for (int cb = 1; cb < max_nblk; cb++) {
            const int nch = (max_nblk + cb - 1) / cb;
            if ((long)n_qt * nch * a.nkv > ws_slots) continue;
            long units = 0;
            for (int t = 0; t < n_qt; t++) units += (tile_blocks(t) + cb - 1) / cb;
            units *= a.nkv;
            const double cost = (double)((units + slots - 1) / slots) * (cb + 1) + units * part_units;
            if (cost < best) {
                best = cost;
                best_cb = cb;
            }
        }
        if (best_cb) {
            a.cb = best_cb;
            a.nch = (max_nblk + best_cb - 1) / best_cb;
            a.part = ws;
        }
    }
    const dim3 grid((unsigned)(base * a.nch));
    if (a.hd == 128)
        hipLaunchKernelGGL(flash_attn_kernel<128>, grid, dim3(256), 0, s, a);
    else if (a.hd == 64)
        hipLaunchKernelGGL(flash_attn_kernel<64>, grid, dim3(256), 0, s, a);
    else
        return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !a.cb) return e;
    if (a.hd == 128)
        hipLaunchKernelGGL(flash_merge_kernel<128>, dim3((unsigned)base, 128 / 8), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(flash_merge_kernel<64>, dim3((unsigned)base, 64 / 8), dim3(256), 0, s, a);
    return hipGetLastError();
}

// rope_f32 (src/rms_norm.cpp:97-152) / apply_rope_2d_f32 (src/hunyuan_image_gen.cpp:71-117)
// in place on x [T][heads][hd]: one thread per interleaved pair
__global__ void rope_apply_kernel(float* __restrict__ x, int T, int heads, int hd, int mode,
                                  const int* __restrict__ positions, float theta, const float* __restrict__ cos_t,
                                  const float* __restrict__ sin_t) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int np = hd / 2;
    if (idx >= (size_t)T * heads * np) return;
    const int d = (int)(idx % np);
    const int t = (int)(idx / ((size_t)np * heads));
    float c, sn;
    if (mode == ROPE_1D) {
        const float pos = positions ? (float)positions[t] : (float)t;
        const float freq = 1.0f / powf(theta, (2.0f * (float)d) / (float)hd);
        c = cosf(pos * freq);
        sn = sinf(pos * freq);
    } else {
        c = cos_t[(size_t)t * hd + 2 * d];
        sn = sin_t[(size_t)t * hd + 2 * d];
    }
    float* v = x + (idx / np) * hd + 2 * d;
    const float x0 = v[0], x1 = v[1];
    v[0] = x0 * c - x1 * sn;
    v[1] = x0 * sn + x1 * c;
}

hipError_t launch_rope_apply(float* x, int T, int heads, int hd, int mode, const int* positions, float theta,
                             const float* cos_t, const float* sin_t, hipStream_t s) {
    const size_t n = (size_t)T * heads * (hd / 2);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_apply_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, T, heads, hd, mode,
                       positions, theta, cos_t, sin_t);
    return hipGetLastError();
}

// embedding_lookup_f32 (src/hunyuan_full_model.cpp:276-290): row ids[t] of the table;
// an id outside the vocabulary gives a zero row instead of an out-of-bounds read
__global__ void embed_kernel(const int* __restrict__ ids, const float* __restrict__ table, int T, int H, int vocab,
                             float* __restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // float4 index
    const int h4 = H / 4;
    if (idx >= (size_t)T * h4) return;
    const int t = (int)(idx / h4), c = (int)(idx % h4);
    const int id = ids[t];
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (id >= 0 && id < vocab) v = reinterpret_cast<const float4*>(table + (size_t)id * H)[c];
    reinterpret_cast<float4*>(out)[idx] = v;
}

hipError_t launch_embed(const int* ids, const float* table, int T, int H, int vocab, float* out, hipStream_t s) {
    const size_t n = (size_t)T * (H / 4);
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, ids, table, T, H, vocab,
                       out);
    return hipGetLastError();
}

__global__ void fill_f32_kernel(float* __restrict__ out, size_t n, float v) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < n) out[idx] = v;
}

hipError_t launch_fill_f32(float* out, size_t n, float v, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, n, v);
    return hipGetLastError();
}

// k / v rows of the [nkv][L][hd] buffers back to the reference's [T][nkv][hd] layout
__global__ void gather_kv_kernel(const float* __restrict__ src, int nkv, int L, int pos0, int T, int hd,
                                 float* __restrict__ dst) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)T * nkv * hd) return;
    const int d = (int)(idx % hd), g = (int)((idx / hd) % nkv), t = (int)(idx / ((size_t)hd * nkv));
    dst[idx] = src[((size_t)g * L + pos0 + t) * hd + d];
}

hipError_t launch_gather_kv(const float* src, int nkv, int L, int pos0, int T, int hd, float* dst, hipStream_t s) {
    const size_t n = (size_t)T * nkv * hd;
    hipLaunchKernelGGL(gather_kv_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, nkv, L, pos0, T, hd,
                       dst);
    return hipGetLastError();
}

}  // namespace hy
