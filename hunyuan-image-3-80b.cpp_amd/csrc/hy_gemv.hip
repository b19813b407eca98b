// hy_gemv.hip -- expert products for decode-sized batches: a dequant-GEMV that
// streams each expert's weights once from HBM, plus the combine kernel.
//
// One wave owns one 64-row group of the row-group-interleaved weights: lane l owns
// row l and walks the blocks b = 0, 1, ... in order, so per block the wave reads one
// contiguous 64-row chunk (2 KB Q8_0 / 1 KB Q4_0 / 8 KB F32) plus 128 B of fp16
// scales, and every output accumulates its blocks in the order the oracle does:
//   acc = fmaf((float)s_b, d_w * d_x, acc)   (s_b = exact int32 block dot, dot4)
//   acc = fmaf(w_k, x_k, acc)                (F32 rows)
// The tile's activation rows sit in LDS and are read as broadcasts.
//
// Work item of the up kernel: (tile, 4 row groups).  A tile is up to NT tokens
// routed to one expert (or NT consecutive tokens for the shared expert).  gate_up
// rows are packed so a 64-row group is 32 SiLU rows + the matching 32 linear rows:
// lanes 0..31 hold g, lanes 32..63 the matching u, and h = silu(g) * u
// (src/hunyuan_moe_full.cpp:479-486) is quantized to Q8_0 by the 32 gate lanes
// (ggml quantizes src1 of every quantized matmul).
// The down kernel's work item is (tile, 4 groups of 64 output rows); every tile
// (routed and shared, one launch) writes y[slot][row], then the combine kernel forms
//   out[t] = residual[t] + ( y_shared[t] + sum_{e ascending} w_e * y_e[t] )
// (src/hunyuan_moe_full.cpp:503-515, einsum_combine order :387-397).
#include <utility>

#include "hy_device.hpp"
#include "hy_launch.hpp"
#include "hy_layout.hpp"
#include "hy_lds.hpp"

namespace hy {

constexpr int GV_WAVES = 4;
constexpr int GV_THREADS = GV_WAVES * WAVE;
constexpr int GV_UNROLL = 8;  // blocks per register set (two sets in flight)

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

// exact int dot of one Q4_0 weight block (16 B, GGUF nibble order: byte j = element
// j | element j+16 << 4) with a Q8_0 activation block whose int sum is asum:
// sum (n-8)*x = sum n*x - 8*sum x.
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

struct GvArgs {
    MatView W;
    Routing R;
    const int8_t* aq;   // activations int8: x [T][H] (mode 0); h block-major [I/32][slots][32] (mode 1)
    const float* ad;    // their scales: x [T][H/32]; h [I/32][slots]
    const int* as;      // their block sums, laid out as the scales
    const float* af;    // f32 activations (F32 weights): x or hf
    int T, H, I, E, K;
    int Kd;             // reduction length
    int n_groups;       // 64-row groups of the weight matrix
    int nx;             // activation rows staged per tile (min(NT, T)): sizes the LDS
    int8_t* hq;         // mode 0 outputs
    float* hd;
    int* hs;
    float* hf;
    float* y;           // mode 1 output
    Route1Out r1;       // one-token batches routed inside the gate/up GEMV (launch_gemv_up_route1)
};

// rows of the block-major h planes: every routed pair's slot and the shared expert's T
__device__ __forceinline__ int h_slots(const GvArgs& a) { return a.T * a.K + a.T; }

template <int WT, int NT, int MODE>
__global__ __launch_bounds__(GV_THREADS) void gemv_kernel(GvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int tok_s[NT], slot_s[NT];
    // mode 1 covers every tile, routed and shared
    // grid (row-group quads, tiles), dispatched tile by tile from the last tile (the
    // shared expert's, with the most tokens) as the ring kernel's
    const int tile = (int)gridDim.y - 1 - (int)blockIdx.y;
    if (tile >= a.R.meta[1]) return;
    const int e = a.R.tile_e[tile], start = a.R.tile_start[tile], n = a.R.tile_n[tile];
    const bool shared = e == a.E;
    const int Kd = a.Kd, nb = Kd / QK;
    if (threadIdx.x < NT) {
        const int i = threadIdx.x;
        int tok = 0, slot = 0;
        if (i < n) {
            if (shared) {
                tok = start + i;
                slot = a.T * a.K + tok;
            } else {
                slot = a.R.off[e] + start + i;
                tok = a.R.srt_tok[slot];
            }
        }
        tok_s[i] = tok;
        slot_s[i] = slot;
    }
    __syncthreads();
    // stage the tile's quantized activation rows (int8), scales and block sums
    int8_t* xs_l = reinterpret_cast<int8_t*>(smem);
    float* xd_l = reinterpret_cast<float*>(smem + (size_t)NT * Kd);
    int* xsum_l = reinterpret_cast<int*>(smem + (size_t)NT * Kd + (size_t)NT * nb * 4);
    if (WT != HY_TYPE_F32) {
        const int vec_per_row = Kd / 16;
        for (int v = threadIdx.x; v < NT * vec_per_row; v += GV_THREADS) {
            const int i = v / vec_per_row, c = v % vec_per_row;
            int4 val = make_int4(0, 0, 0, 0);
            if (i < n) {
                const int row = MODE == 0 ? tok_s[i] : slot_s[i];
                val = MODE == 0 ? reinterpret_cast<const int4*>(a.aq + (size_t)row * Kd)[c]
                                : reinterpret_cast<const int4*>(a.aq + ((size_t)(c / 2) * h_slots(a) + row) * QK)[c % 2];
            }
            reinterpret_cast<int4*>(xs_l + (size_t)i * Kd)[c] = val;
        }
        for (int v = threadIdx.x; v < NT * nb; v += GV_THREADS) {
            const int i = v / nb, b = v % nb;
            const int row = MODE == 0 ? tok_s[i] : slot_s[i];
            const size_t si = MODE == 0 ? (size_t)row * nb + b : (size_t)b * h_slots(a) + row;
            xd_l[v] = i < n ? a.ad[si] : 0.0f;
            if (WT == HY_TYPE_Q4_0) xsum_l[v] = i < n ? a.as[si] : 0;
        }
    }
    __syncthreads();

    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int G = blockIdx.x * GV_WAVES + wave;
    if (G >= a.n_groups) return;
    float acc[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) acc[i] = 0.0f;

    if (WT == HY_TYPE_F32) {
        // quad-major blocks: quad c of this lane's row at c * 256 + 4 lane floats; the
        // next block's 8 loads are in flight while this block is consumed
        const float* wbase = reinterpret_cast<const float*>(a.W.qs + (size_t)e * a.W.qs_stride) +
                             (size_t)G * nb * 64 * QK + 4 * lane;
        v4f_t w[2][8];
        auto load = [&](int set, int b) {
            const float* p = wbase + (size_t)min(b, nb - 1) * 64 * QK;  // in bounds
#pragma unroll
            for (int c = 0; c < 8; c++) w[set][c] = __builtin_nontemporal_load(reinterpret_cast<const v4f_t*>(p + c * 256));
        };
        auto consume = [&](int set, int b) {
#pragma unroll
            for (int i = 0; i < NT; i++) {
                if (i < n) {
                    const int row = MODE == 0 ? tok_s[i] : slot_s[i];
                    const float4* xv = reinterpret_cast<const float4*>(a.af + (size_t)row * Kd + (size_t)b * QK);
                    float s = acc[i];
#pragma unroll
                    for (int c = 0; c < 8; c++) {
                        const float4 xx = xv[c];
                        s = fmaf(w[set][c][0], xx.x, s);
                        s = fmaf(w[set][c][1], xx.y, s);
                        s = fmaf(w[set][c][2], xx.z, s);
                        s = fmaf(w[set][c][3], xx.w, s);
                    }
                    acc[i] = s;
                }
            }
        };
        load(0, 0);
        for (int b = 0; b < nb; b += 2) {
            load(1, b + 1);
            consume(0, b);
            if (b + 1 >= nb) break;
            load(0, b + 2);
            consume(1, b + 1);
        }
    } else {
        constexpr int BPB = WT == HY_TYPE_Q8_0 ? 32 : 16;
        const uint8_t* wbase = a.W.qs + (size_t)e * a.W.qs_stride + ((size_t)G * nb * 64 + lane) * BPB;
        const uint16_t* sbase = a.W.sc + (size_t)e * a.W.sc_stride + (size_t)G * nb * 64 + lane;
        // two register sets of GV_UNROLL blocks: the next chunk's loads are in flight
        // while the current chunk is consumed (software pipelining)
        int4 w0[2][GV_UNROLL], w1[2][GV_UNROLL];
        float dw[2][GV_UNROLL];
        auto load = [&](int set, int b0) {
#pragma unroll
            for (int u = 0; u < GV_UNROLL; u++) {
                const int b = b0 + u;
                if (b < nb) {
                    const int4* p = reinterpret_cast<const int4*>(wbase + (size_t)b * 64 * BPB);
                    w0[set][u] = p[0];
                    if (WT == HY_TYPE_Q8_0) w1[set][u] = p[1];
                    dw[set][u] = h2f(sbase[(size_t)b * 64]);
                }
            }
        };
        auto consume = [&](int set, int b0) {
#pragma unroll
            for (int u = 0; u < GV_UNROLL; u++) {
                const int b = b0 + u;
                if (b >= nb) break;
#pragma unroll
                for (int i = 0; i < NT; i++) {
                    if (i < n) {
                        const int4* xb = reinterpret_cast<const int4*>(xs_l + (size_t)i * Kd + b * QK);
                        const int s = WT == HY_TYPE_Q8_0
                                          ? dot_q8_block(w0[set][u], w1[set][u], xb[0], xb[1])
                                          : dot_q4_block(w0[set][u], xb[0], xb[1], xsum_l[i * nb + b]);
                        acc[i] = fmaf((float)s, dw[set][u] * xd_l[i * nb + b], acc[i]);
                    }
                }
            }
        };
        load(0, 0);
        for (int b0 = 0; b0 < nb; b0 += 2 * GV_UNROLL) {
            if (b0 + GV_UNROLL < nb) load(1, b0 + GV_UNROLL);
            consume(0, b0);
            if (b0 + GV_UNROLL >= nb) break;
            if (b0 + 2 * GV_UNROLL < nb) load(0, b0 + 2 * GV_UNROLL);
            consume(1, b0 + GV_UNROLL);
        }
    }

    if (MODE == 0) {
        // lanes 0..31: gate rows 32G+lane, lanes 32..63: the matching up rows
#pragma unroll
        for (int i = 0; i < NT; i++) {
            if (i >= n) break;
            const float u = __shfl(acc[i], (lane + 32) % WAVE, WAVE);
            const float h = swiglu(acc[i], u);
            const size_t slot = (size_t)slot_s[i];
            if (WT == HY_TYPE_F32) {
                if (lane < 32) a.hf[slot * a.I + (size_t)G * QK + lane] = h;
            } else {
                const Q8Result r = quant_q8_0_lane32(h);
                int s = r.q;
#pragma unroll
                for (int m = 16; m >= 1; m >>= 1) s += shfl_xor(s, m, 32);
                if (lane < 32) {
                    const size_t hi = (size_t)G * h_slots(a) + slot;  // block-major h
                    a.hq[hi * QK + lane] = r.q;
                    if (lane == 0) {
                        a.hd[hi] = h2f(r.dh);
                        a.hs[hi] = s;
                    }
                }
            }
        }
    } else {
        const int row = G * 64 + lane;
#pragma unroll
        for (int i = 0; i < NT; i++) {
            if (i >= n) break;
            a.y[(size_t)slot_s[i] * a.H + row] = acc[i];
        }
    }
}

// Quantized weights (Q8_0 / Q4_0): the same per-row block-sequential accumulation as
// gemv_kernel, with the operand streams decoupled from the arithmetic.  Each work
// group is one wave owning one 64-row group of one tile (<= NT tokens).  A private LDS
// ring holds NSTEP steps; a step is U consecutive blocks (8, or 4 or 2 when a launch's
// waves outnumber the LDS slots of the larger steps):
//   weights  U x (64 rows x 16 B / 32 B)      one DMA per block (two for Q8_0)
//   scales   U x 64 fp16                      one DMA (contiguous in the plane)
//   x        NT tokens x U x 32 B int8        one DMA (token = lane / (2 U))
//   x scales / block sums  NT x U x 4 B       one DMA (lanes 0..NT U-1 / NT U..2 NT U-1)
// Token slots past the tile's n read token 0's row (valid, never used), so every
// step issues the same number of copies and the vmcnt waits are constants.  Copies
// complete in order; no barrier is needed because a wave only reads what it copied.
// The weight stream starts before the routing lookups of the tile (expert id read
// speculatively and clamped into the resident table), so their latency overlaps the
// first copies; the first activation copies follow, and one full wait joins both.
// The last NSTEP steps are consumed by an unrolled tail whose waits count down to
// zero: the wave leaves no copy in flight.
constexpr int GQ_U = 8;       // blocks per step
constexpr int GQ_U_SMALL = 4;  // ... for launches whose waves only 4-block steps keep resident
constexpr int GQ_U_TINY = 2;   // ... only 2-block steps
constexpr int GQ_WAVES = 1;   // one wave per work group: work groups spread over every CU
constexpr int GQ_THREADS = GQ_WAVES * WAVE;

// Ring depth: Q4_0 3 steps of 8 blocks (31 KB of LDS, 5 waves a CU), Q8_0 2 (37 KB, 4 a
// CU); copies in flight <= 36 < 64 (vmcnt).  A launch with more waves than the deeper
// ring leaves resident takes 2 steps for Q4_0 (21 KB, 7 a CU): one round of waves
// instead of a second, short one (T=2: 15 tiles x 96 row groups = 1,440 waves for 1,280
// slots); larger launches take 2 steps of 4 blocks (Q4_0 10 KB, 15 a CU) or 2 blocks
// (5 KB, 31 a CU) when that keeps every wave resident (gemv_launch).
template <int WT>
struct GqSteps {
    static constexpr int value = WT == HY_TYPE_Q4_0 ? 3 : 2;
};

template <int WT, int NT, int U>
struct GqSlot {
    static constexpr int BPB = WT == HY_TYPE_Q4_0 ? 16 : 32;
    static constexpr int W = 0;                             // weights
    static constexpr int S = W + U * 64 * BPB;              // weight scales
    static constexpr int X = S + U * 64 * 2;                // activation quants
    static constexpr int XD = X + NT * U * QK;              // activation scales, then block sums
    static constexpr int BYTES = XD + 2 * NT * U * 4;
    static constexpr int LOADS = U * (WT == HY_TYPE_Q4_0 ? 1 : 2) + 1 + 1 + 1;
    // lanes that carry a copy: weight scales (16 B each), activations (16 B each), their
    // scales and block sums (4 B each); the other lanes are masked
    static constexpr int SC_LANES = U * 64 * 2 / 16, X_LANES = NT * U * QK / 16, XD_LANES = 2 * NT * U;
    static_assert(U == 2 || U == 4 || U == 8, "steps of 2, 4 or 8 blocks");
    static_assert(SC_LANES <= WAVE && X_LANES <= WAVE && XD_LANES <= WAVE, "one copy per lane moves each part");
    static_assert(X_LANES % NT == 0, "whole token rows per copy");
};

// One-token routing inside the gate/up GEMV (launch_gemv_up_route1): the wave selects
// the top-k of logits[E] exactly as the decode routing pass does (topk_wave), and its
// tile is the tile-th selected expert in ascending order (each selected expert has
// the token's one pair: one tile, slot = rank); tile K is the shared expert's, which
// needs no routing.  The writer wave (tile 0, row group 0) also stores every routing
// product that pass stores for T = 1, for the down GEMV, the combine and the caller:
// top-k weights and ids, per-expert counts and offsets, the sorted token list, pair
// positions, the combine list in ascending expert order, the tiles and meta.
__device__ __forceinline__ int route1_tile(const GvArgs& a, int tile, int lane, bool writer) {
    const Route1Out& r = a.r1;
    const int E = a.E, K = a.K;
    if (tile >= K && !writer) return E;
    __shared__ float selw_s[MAX_K];
    __shared__ int seli_s[MAX_K];
    const float lv = lane < E ? r.logits[lane] : 0.0f;
    topk_wave(lv, E, K, r.norm, r.scale, lane, selw_s, seli_s);
    __syncthreads();
    int kq = -1;  // this lane's expert's rank in the top-k, -1 if not selected
    for (int k = 0; k < K; k++) kq = seli_s[k] == lane ? k : kq;
    const bool sel = kq >= 0;
    const int rank = __popcll(__ballot(sel) & ((1ull << lane) - 1ull));  // selected experts below this one
    if (writer) {
        if (lane < K) {
            r.topw[lane] = selw_s[lane];
            r.topi[lane] = seli_s[lane];
            r.srt_tok[lane] = 0;
        }
        if (lane < E) {
            r.cnt[lane] = sel ? 1 : 0;
            r.off[lane] = rank;
            r.meta[META_TILE_OFF + lane] = rank;
        }
        if (sel) {
            r.pair_pos[kq] = rank;
            r.comb_pos[rank] = rank;
            r.comb_w[rank] = selw_s[kq];
            r.tile_e[rank] = lane;
            r.tile_start[rank] = 0;
            r.tile_n[rank] = 1;
        }
        if (lane == 0) {
            const int all = K + r.has_shared;
            r.off[E] = K;
            r.meta[0] = K;
            r.meta[1] = all;
            r.meta[2] = K;
            r.meta[3] = 1;
            r.meta[META_TILE_OFF + E] = K;
            r.meta[META_TILE_OFF + E + 1] = all;
            if (r.has_shared) {
                r.tile_e[K] = E;
                r.tile_start[K] = 0;
                r.tile_n[K] = 1;
            }
        }
    }
    if (tile >= K) return E;
    return (int)__builtin_ctzll(__ballot(sel && rank == tile));
}

// consume the last NSTEP steps: before step base + J, wait until at most the
// NSTEP - 1 - J younger steps' copies are outstanding
template <int J, int NSTEP, int LOADS, class F>
__device__ __forceinline__ void gemv_tail(F& step, int base) {
    if constexpr (J < NSTEP) {
        MM_WAIT_VM_LGKM((NSTEP - 1 - J) * LOADS);
        step(base + J);
        gemv_tail<J + 1, NSTEP, LOADS>(step, base);
    }
}

template <int WT, int NT, int MODE, int NSTEP, bool R1 = false, int U = GQ_U>
__global__ __launch_bounds__(GQ_THREADS) void gemv_q_kernel(GvArgs a) {
    static_assert(!R1 || MODE == 0, "routing inside the launch: gate/up only");
    static_assert(MODE == 0 || MODE == 1, "routed/shared products only (the combine runs separately)");
    using SL = GqSlot<WT, NT, U>;
    constexpr bool Q4 = WT == HY_TYPE_Q4_0;
    constexpr int BPB = SL::BPB;
    constexpr int WBYTES = 64 * BPB;  // one block of a 64-row group
    extern __shared__ __align__(16) uint8_t ring[];
    __shared__ int tok_s[NT], slot_s[NT];
    const int lane = threadIdx.x;
    // grid (row groups, tiles), dispatched tile by tile from the last tile: the shared
    // expert's tiles (the list's last, and with the most tokens) start first, so
    // their heavier waves do not form the launch's tail
    const int G = blockIdx.x;  // 64-row group (grid.x == n_groups)
    const int tile = (int)gridDim.y - 1 - (int)blockIdx.y;
    const int Kd = a.Kd, nb = Kd / QK, nsteps = nb / U;

    // start the weight stream first: tile_e[tile] is in the arena for every launched
    // tile; a stale entry (tile past this call's count) is clamped into the table and
    // its copies are drained before the work group exits.  R1: the wave routes the
    // token itself (the shared tile starts at once).
    int e;
    if constexpr (R1) {
        e = route1_tile(a, tile, lane, tile == 0 && G == 0);
        e = e < 0 ? 0 : (e >= a.W.n_mats ? a.W.n_mats - 1 : e);  // in the table whatever the logits hold
    } else {
        e = a.R.tile_e[tile];
        e = e < 0 ? 0 : (e >= a.W.n_mats ? a.W.n_mats - 1 : e);
    }
    const uint8_t* wq = a.W.qs + (size_t)e * a.W.qs_stride + (size_t)G * nb * WBYTES + lane * 16;
    const uint16_t* wsc = a.W.sc + (size_t)e * a.W.sc_stride + (size_t)G * nb * 64 + lane * 8;
    auto issue_w = [&](int st_i) {
        uint8_t* st = ring + (st_i % NSTEP) * SL::BYTES;
        const uint8_t* src = wq + (size_t)st_i * U * WBYTES;
#pragma unroll
        for (int u = 0; u < U; u++) {
            g2l16_nt(src + u * WBYTES, st + SL::W + u * WBYTES);
            if (!Q4) g2l16_nt(src + u * WBYTES + 1024, st + SL::W + u * WBYTES + 1024);
        }
        if (SL::SC_LANES == WAVE || lane < SL::SC_LANES) g2l16_nt(wsc + (size_t)st_i * U * 64, st + SL::S);
    };
#pragma unroll
    for (int s = 0; s < NSTEP; s++) issue_w(s);

    if (!R1 && tile >= a.R.meta[1]) {
        MM_WAIT_VM_LGKM(0);
        return;
    }
    // R1: one pair per tile (the routed tile's slot is its rank, tile; the shared
    // tile's is T * K)
    const int start = R1 ? 0 : a.R.tile_start[tile], n = R1 ? 1 : a.R.tile_n[tile];
    const bool shared = e == a.E;
    if (lane < NT) {
        int tok = 0, slot = 0;
        if (lane < n) {
            if (shared) {
                tok = start + lane;
                slot = a.T * a.K + tok;
            } else if (R1) {
                slot = tile;
            } else {
                slot = a.R.off[e] + start + lane;
                tok = a.R.srt_tok[slot];
            }
        }
        tok_s[lane] = tok;
        slot_s[lane] = slot;
    }
    __syncthreads();
    // this lane's activation sources: x piece (token lane / PPT, 16 B piece lane % PPT
    // of the step's U * 32 B per token) and the scale (lanes < NT * U) or block sum
    // (lanes NT * U .. 2 NT * U - 1) of token (lane % NT * U) / U, block lane % U; token
    // slots >= n read token 0's row, lanes past a part's copy read in-range sources
    constexpr int PPT = U * QK / 16, NTU = NT * U;
    const int xt = lane / PPT;
    const bool is_sum = lane >= NTU;
    const int sidx = lane % NTU, st_tok = sidx / U;
    const int xrow = MODE == 0 ? tok_s[xt < n ? xt : 0] : slot_s[xt < n ? xt : 0];
    const int srow = MODE == 0 ? tok_s[st_tok < n ? st_tok : 0] : slot_s[st_tok < n ? st_tok : 0];
    // mode 1 reads h block-major: block b of slot r at (b * slots + r) * 32, its scale and
    // sum at b * slots + r; a step advances U block planes
    const size_t hs_n = MODE == 0 ? 1 : (size_t)h_slots(a);
    const int8_t* xsrc = MODE == 0 ? a.aq + (size_t)xrow * Kd + (lane % PPT) * 16
                                   : a.aq + ((size_t)((lane % PPT) / 2) * hs_n + xrow) * QK + (lane % 2) * 16;
    const size_t sofs = MODE == 0 ? (size_t)srow * nb + sidx % U : (size_t)(sidx % U) * hs_n + srow;
    const void* ssrc = !is_sum ? (const void*)(a.ad + sofs)
                               : (Q4 ? (const void*)(a.as + sofs) : (const void*)(a.ad + sofs));
    const size_t x_step = (size_t)U * QK * hs_n, s_step = (size_t)U * 4 * hs_n;  // bytes per step
    auto issue_x = [&](int st_i) {
        uint8_t* st = ring + (st_i % NSTEP) * SL::BYTES;
        if (SL::X_LANES == WAVE || lane < SL::X_LANES) g2l16(xsrc + (size_t)st_i * x_step, st + SL::X);
        if (SL::XD_LANES == WAVE || lane < SL::XD_LANES)
            __builtin_amdgcn_global_load_lds(static_cast<const uint8_t*>(ssrc) + (size_t)st_i * s_step, st + SL::XD, 4,
                                             0, 0);
    };
#pragma unroll
    for (int s = 0; s < NSTEP; s++) issue_x(s);
    MM_WAIT_VM_LGKM(0);  // the first NSTEP steps have landed

    float acc[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) acc[i] = 0.0f;
    // one step: the step's weights and scales, then per token its activation blocks, one
    // wait per token, then the blocks in order
    auto step = [&](int st_i) {
        const uint32_t st = lds_off(ring + (st_i % NSTEP) * SL::BYTES);
        const uint32_t wrow = st + SL::W + lane * BPB;
        const uint32_t srow_l = st + SL::S + lane * 2;
        v4i_t w0[U], w1[U], wlo[U], whi[U];
        uint32_t dwb[U];
        float dwf[U];
        [&]<int... UU>(std::integer_sequence<int, UU...>) {
            ((w0[UU] = lds_b128_at<UU * WBYTES>(wrow)), ...);
            if constexpr (!Q4) ((w1[UU] = lds_b128_at<UU * WBYTES + 16>(wrow)), ...);
            ((dwb[UU] = lds_u16_at<UU * 128>(srow_l)), ...);
        }(std::make_integer_sequence<int, U>{});
#pragma unroll
        for (int i = 0; i < NT; i++) {
            if (i < n) {
                const uint32_t xb = st + SL::X + i * U * QK;
                const uint32_t db = st + SL::XD + i * U * 4;
                v4i_t x0[U], x1[U];
                uint32_t xdb[U], xsb[U];
                [&]<int... UU>(std::integer_sequence<int, UU...>) {
                    ((x0[UU] = lds_b128_at<UU * QK>(xb)), ...);
                    ((x1[UU] = lds_b128_at<UU * QK + 16>(xb)), ...);
                    ((xdb[UU] = lds_b32_at<UU * 4>(db)), ...);
                    if constexpr (Q4) ((xsb[UU] = lds_b32_at<NTU * 4 + UU * 4>(db)), ...);
                }(std::make_integer_sequence<int, U>{});
                lds_wait();
                if (i == 0) {
                    // weight-side work shared by the tile's tokens: Q4_0 nibbles unpacked
                    // and fp16 scales converted once per block
#pragma unroll
                    for (int u = 0; u < U; u++) {
                        lds_pin(w0[u]);
                        if (!Q4) lds_pin(w1[u]);
                        lds_pin(dwb[u]);
                        dwf[u] = h2f((uint16_t)dwb[u]);
                        if (Q4) {
                            const int m = 0x0F0F0F0F;
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                wlo[u][j] = w0[u][j] & m;
                                whi[u][j] = (w0[u][j] >> 4) & m;
                            }
                        }
                    }
                }
#pragma unroll
                for (int u = 0; u < U; u++) {
                    lds_pin(x0[u]);
                    lds_pin(x1[u]);
                    lds_pin(xdb[u]);
                    if (Q4) lds_pin(xsb[u]);
                    int sdot;
                    if (Q4) {
                        // sum (n - 8) x = sum n x - 8 sum x, from the activation block's sum
                        sdot = -8 * (int)xsb[u];
#pragma unroll
                        for (int j = 0; j < 4; j++) sdot = dot4(wlo[u][j], x0[u][j], sdot);
#pragma unroll
                        for (int j = 0; j < 4; j++) sdot = dot4(whi[u][j], x1[u][j], sdot);
                    } else {
                        const int4 W0 = make_int4(w0[u][0], w0[u][1], w0[u][2], w0[u][3]);
                        const int4 W1 = make_int4(w1[u][0], w1[u][1], w1[u][2], w1[u][3]);
                        const int4 X0 = make_int4(x0[u][0], x0[u][1], x0[u][2], x0[u][3]);
                        const int4 X1 = make_int4(x1[u][0], x1[u][1], x1[u][2], x1[u][3]);
                        sdot = dot_q8_block(W0, W1, X0, X1);
                    }
                    acc[i] = fmaf((float)sdot, dwf[u] * __builtin_bit_cast(float, xdb[u]), acc[i]);
                }
                pin_f32(acc[i]);  // token i done before token i+1's reads
            }
        }
    };
    for (int s = 0; s < nsteps - NSTEP; s++) {
        MM_WAIT_VM_LGKM((NSTEP - 1) * SL::LOADS);  // step s landed (copies complete in order)
        step(s);
        issue_w(s + NSTEP);                        // refill the slot just read
        issue_x(s + NSTEP);
    }
    gemv_tail<0, NSTEP, SL::LOADS>(step, nsteps - NSTEP);

    if (MODE == 0) {
        // lanes 0..31: gate rows 32G+lane, lanes 32..63: the matching up rows
#pragma unroll
        for (int i = 0; i < NT; i++) {
            if (i >= n) break;
            const float u = __shfl(acc[i], (lane + 32) % WAVE, WAVE);
            const float h = swiglu(acc[i], u);
            const size_t slot = (size_t)slot_s[i];
            const Q8Result r = quant_q8_0_lane32(h);
            int s = r.q;
#pragma unroll
            for (int m = 16; m >= 1; m >>= 1) s += shfl_xor(s, m, 32);
            if (lane < 32) {
                const size_t hi = (size_t)G * h_slots(a) + slot;  // block-major h
                a.hq[hi * QK + lane] = r.q;
                if (lane == 0) {
                    a.hd[hi] = h2f(r.dh);
                    a.hs[hi] = s;
                }
            }
        }
    } else {
        const int row = G * 64 + lane;
#pragma unroll
        for (int i = 0; i < NT; i++) {
            if (i >= n) break;
            a.y[(size_t)slot_s[i] * a.H + row] = acc[i];
        }
    }
}

// combine: out[t] = residual[t] + ( y_shared[t] + sum_{e ascending} w_e y_e[t] ), the
// shared expert's output at slot T*K + t when has_shared.  A pair with w_e == 0 (a
// dropped pair, or a zero gate) adds nothing, as einsum_combine skips it
// (src/hunyuan_moe_full.cpp:387-397); its y row is read but not used.  One thread per 4 outputs
// (16-byte loads of the y rows); each output keeps the scalar fmaf order.  The token's
// list entries are taken KMAX at a time (one pass for K <= KMAX; indices clamped to
// K - 1): a chunk's entries and then its y rows are all loaded before its first fmaf,
// so a thread waits for two rounds of loads per chunk, not 2 K.
template <int KMAX>
__global__ __launch_bounds__(256) void combine_kernel(Routing R, const float* __restrict__ y, int T, int H, int K,
                                                      int has_shared, const float* __restrict__ resid,
                                                      float* __restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // group of 4 outputs
    const int H4 = H / 4;
    if (idx >= (size_t)T * H4) return;
    const int t = (int)(idx / H4), r4 = (int)(idx % H4);
    // the shared expert's row and the residual do not depend on the lists: their loads
    // are issued first, so they overlap the list and y-row round trips instead of
    // following them
    v4f_t u = {0.f, 0.f, 0.f, 0.f}, q = {0.f, 0.f, 0.f, 0.f};
    if (has_shared) u = __builtin_nontemporal_load(reinterpret_cast<const v4f_t*>(y + ((size_t)T * K + t) * H) + r4);
    if (resid) q = reinterpret_cast<const v4f_t*>(resid + (size_t)t * H)[r4];
    float4 c = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k0 = 0; k0 < K; k0 += KMAX) {
        int pos[KMAX];
        float w[KMAX];
#pragma unroll
        for (int k = 0; k < KMAX; k++) {
            const int kk = min(k0 + k, K - 1);
            pos[k] = R.comb_pos[t * K + kk];
            w[k] = R.comb_w[t * K + kk];
        }
        v4f_t v[KMAX];
#pragma unroll
        for (int k = 0; k < KMAX; k++) v[k] = __builtin_nontemporal_load(reinterpret_cast<const v4f_t*>(y + (size_t)pos[k] * H) + r4);
#pragma unroll
        for (int k = 0; k < KMAX; k++)
            if (k0 + k < K && w[k] != 0.0f)
                c = make_float4(fmaf(w[k], v[k][0], c.x), fmaf(w[k], v[k][1], c.y), fmaf(w[k], v[k][2], c.z),
                                fmaf(w[k], v[k][3], c.w));
    }
    float4 o = c;
    if (has_shared) o = make_float4(u[0] + c.x, u[1] + c.y, u[2] + c.z, u[3] + c.w);
    if (resid) o = make_float4(q[0] + o.x, q[1] + o.y, q[2] + o.z, q[3] + o.w);
    reinterpret_cast<float4*>(out + (size_t)t * H)[r4] = o;
}

// ---------------------------------------------------------------------------- launchers
int gemv_tile_tokens() { return GEMV_NT; }

size_t gemv_smem(int wtype, int Kd) {
    if (wtype == HY_TYPE_F32) return 16;
    return (size_t)GEMV_NT * Kd + (size_t)GEMV_NT * (Kd / QK) * 8;
}

// LDS of gemv_q_kernel: a ring of NSTEP steps
template <int WT, int U = GQ_U>
static size_t gemv_q_smem(int nstep) {
    return (size_t)nstep * GqSlot<WT, GEMV_NT, U>::BYTES;
}

template <int WT, int U = GQ_U>
static bool gemv_q_fits(int Kd) {
    const int nb = Kd / QK;
    return nb % U == 0 && nb / U >= GqSteps<WT>::value;
}

// resident one-wave work groups per CU at this LDS footprint (160 KB of LDS a CU)
static int gemv_q_slots(size_t smem) {
    const int per_cu = (int)((160u * 1024u) / smem);
    return 256 * (per_cu < 32 ? per_cu : 32);  // at most 32 one-wave work groups a CU (8 waves a SIMD)
}

template <int MODE>
static hipError_t gemv_launch(int wtype, int tiles, hipStream_t s, GvArgs a) {
    a.nx = a.T < GEMV_NT ? a.T : GEMV_NT;
    const dim3 grid_v((a.n_groups + GV_WAVES - 1) / GV_WAVES, tiles);
    const dim3 grid_q(a.n_groups, tiles);
    // tiles is the host's bound on the routed + shared tiles.  Steps of 4 or 2 blocks (2x /
    // 4x the resident waves) when the smaller steps, and not the larger ones, hold the
    // whole launch at once (Q4_0 steps: T=4 125.4-127.7 -> 119.3-120.2 us, T=6 161.5-165.1
    // -> 154.3-157.5, T=8 184.0-192.9 -> 174.6-181.9); a launch too large for every size
    // stays on 8-block steps (T=8 on 4-block steps: 185.9-189.7 against 184.8-186.5 us)
    const long waves = (long)tiles * a.n_groups;
    auto small_steps = [&](auto wt) {
        constexpr int WT = decltype(wt)::value;
        return gemv_q_fits<WT, GQ_U_SMALL>(a.Kd) && waves > gemv_q_slots(gemv_q_smem<WT>(2)) &&
               waves <= gemv_q_slots(gemv_q_smem<WT, GQ_U_SMALL>(2));
    };
    auto tiny_steps = [&](auto wt) {
        constexpr int WT = decltype(wt)::value;
        return gemv_q_fits<WT, GQ_U_TINY>(a.Kd) && waves > gemv_q_slots(gemv_q_smem<WT, GQ_U_SMALL>(2)) &&
               waves <= gemv_q_slots(gemv_q_smem<WT, GQ_U_TINY>(2));
    };
    switch (wtype) {
    case HY_TYPE_Q8_0:
        if (tiny_steps(std::integral_constant<int, HY_TYPE_Q8_0>{}))
            hipLaunchKernelGGL((gemv_q_kernel<HY_TYPE_Q8_0, GEMV_NT, MODE, 2, false, GQ_U_TINY>), grid_q,
                               dim3(GQ_THREADS), (gemv_q_smem<HY_TYPE_Q8_0, GQ_U_TINY>(2)), s, a);
        else if (small_steps(std::integral_constant<int, HY_TYPE_Q8_0>{}))
            hipLaunchKernelGGL((gemv_q_kernel<HY_TYPE_Q8_0, GEMV_NT, MODE, 2, false, GQ_U_SMALL>), grid_q,
                               dim3(GQ_THREADS), (gemv_q_smem<HY_TYPE_Q8_0, GQ_U_SMALL>(2)), s, a);
        else if (gemv_q_fits<HY_TYPE_Q8_0>(a.Kd))
            hipLaunchKernelGGL((gemv_q_kernel<HY_TYPE_Q8_0, GEMV_NT, MODE, 2>), grid_q, dim3(GQ_THREADS),
                               gemv_q_smem<HY_TYPE_Q8_0>(2), s, a);
        else
            hipLaunchKernelGGL((gemv_kernel<HY_TYPE_Q8_0, GEMV_NT, MODE>), grid_v, dim3(GV_THREADS),
                               gemv_smem(wtype, a.Kd), s, a);
        break;
    case HY_TYPE_Q4_0:
        if (tiny_steps(std::integral_constant<int, HY_TYPE_Q4_0>{})) {
            hipLaunchKernelGGL((gemv_q_kernel<HY_TYPE_Q4_0, GEMV_NT, MODE, 2, false, GQ_U_TINY>), grid_q,
                               dim3(GQ_THREADS), (gemv_q_smem<HY_TYPE_Q4_0, GQ_U_TINY>(2)), s, a);
        } else if (small_steps(std::integral_constant<int, HY_TYPE_Q4_0>{})) {
            hipLaunchKernelGGL((gemv_q_kernel<HY_TYPE_Q4_0, GEMV_NT, MODE, 2, false, GQ_U_SMALL>), grid_q,
                               dim3(GQ_THREADS), (gemv_q_smem<HY_TYPE_Q4_0, GQ_U_SMALL>(2)), s, a);
        } else if (gemv_q_fits<HY_TYPE_Q4_0>(a.Kd)) {
            // the deeper ring for gate/up when every launched wave is resident at once; the
            // down products take 2 steps (T=2: 23.9 -> 22.8 us, T=1 and T=4 unchanged)
            if (MODE == 0 && waves <= gemv_q_slots(gemv_q_smem<HY_TYPE_Q4_0>(3)))
                hipLaunchKernelGGL((gemv_q_kernel<HY_TYPE_Q4_0, GEMV_NT, MODE, 3>), grid_q, dim3(GQ_THREADS),
                                   gemv_q_smem<HY_TYPE_Q4_0>(3), s, a);
            else
                hipLaunchKernelGGL((gemv_q_kernel<HY_TYPE_Q4_0, GEMV_NT, MODE, 2>), grid_q, dim3(GQ_THREADS),
                                   gemv_q_smem<HY_TYPE_Q4_0>(2), s, a);
        } else {
            hipLaunchKernelGGL((gemv_kernel<HY_TYPE_Q4_0, GEMV_NT, MODE>), grid_v, dim3(GV_THREADS),
                               gemv_smem(wtype, a.Kd), s, a);
        }
        break;
    default:
        hipLaunchKernelGGL((gemv_kernel<HY_TYPE_F32, GEMV_NT, MODE>), grid_v, dim3(GV_THREADS),
                           gemv_smem(wtype, a.Kd), s, a);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_gemv_up(int wtype, int max_tiles, const MatView& W, const Routing& R, const ActQ& X, const float* xf,
                          int T, int H, int I, int E, int K, int8_t* hq, float* hd, int* hs, float* hf,
                          hipStream_t s) {
    GvArgs a{W, R, X.q, X.d, X.s, xf, T, H, I, E, K, H, 2 * I / 64, 0, hq, hd, hs, hf, nullptr};
    return gemv_launch<0>(wtype, max_tiles, s, a);
}

bool gemv_route1_ok(int wtype, int H) {
    return (wtype == HY_TYPE_Q8_0 && gemv_q_fits<HY_TYPE_Q8_0>(H)) || (wtype == HY_TYPE_Q4_0 && gemv_q_fits<HY_TYPE_Q4_0>(H));
}

hipError_t launch_gemv_up_route1(int wtype, const MatView& W, const Route1Out& r, const ActQ& X, int H, int I, int E,
                                 int K, int8_t* hq, float* hd, int* hs, hipStream_t s) {
    if (!gemv_route1_ok(wtype, H) || K < 1 || K > E || E > MAX_E) return hipErrorInvalidValue;
    GvArgs a{W, Routing{}, X.q, X.d, X.s, nullptr, 1, H, I, E, K, H, 2 * I / 64, 1, hq, hd, hs, nullptr, nullptr, r};
    const dim3 grid((unsigned)a.n_groups, (unsigned)(K + r.has_shared));
    // one token: K + 1 tiles x row groups, a 2-step ring for both types (at T = 1 with
    // E = 64, K = 8, H = 4096, Q4_0, the 3-step ring, every wave still resident, was
    // 1 % slower: gate/up 27.6-27.7 against 27.4 us)
    if (wtype == HY_TYPE_Q8_0)
        hipLaunchKernelGGL((gemv_q_kernel<HY_TYPE_Q8_0, GEMV_NT, 0, 2, true>), grid, dim3(GQ_THREADS),
                           gemv_q_smem<HY_TYPE_Q8_0>(2), s, a);
    else
        hipLaunchKernelGGL((gemv_q_kernel<HY_TYPE_Q4_0, GEMV_NT, 0, 2, true>), grid, dim3(GQ_THREADS),
                           gemv_q_smem<HY_TYPE_Q4_0>(2), s, a);
    return hipGetLastError();
}

hipError_t launch_gemv_down(int wtype, int n_tiles_bound, const MatView& W, const Routing& R, const int8_t* hq,
                            const float* hd, const int* hs, const float* hf, int T, int H, int I, int E, int K,
                            float* y, hipStream_t s) {
    GvArgs a{W, R, hq, hd, hs, hf, T, H, I, E, K, I, H / 64, 0, nullptr, nullptr, nullptr, nullptr, y};
    return gemv_launch<1>(wtype, n_tiles_bound, s, a);
}

hipError_t launch_combine(const Routing& R, const float* y, int T, int H, int K, int has_shared, const float* resid,
                          float* out, hipStream_t s) {
    const size_t n = (size_t)T * (H / 4);
    const dim3 grid((unsigned)((n + 255) / 256));
    if (K <= 4)
        hipLaunchKernelGGL(combine_kernel<4>, grid, dim3(256), 0, s, R, y, T, H, K, has_shared, resid, out);
    else if (K <= 8)
        hipLaunchKernelGGL(combine_kernel<8>, grid, dim3(256), 0, s, R, y, T, H, K, has_shared, resid, out);
    else  // 16 pairs per chunk (larger K loops over chunks)
        hipLaunchKernelGGL(combine_kernel<16>, grid, dim3(256), 0, s, R, y, T, H, K, has_shared, resid, out);
    return hipGetLastError();
}

// per-block dots through the GEMV dot routines (parity entry point); GGUF blocks in,
// one thread per (row, block)
__global__ void block_dots_valu_kernel(int wtype, const uint8_t* __restrict__ w, const uint8_t* __restrict__ x,
                                       int rows, int nb, int* __restrict__ out) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * nb) return;
    const int r = idx / nb, b = idx % nb;
    // GGUF blocks are only 2-byte aligned: assemble the dwords bytewise
    auto dword = [](const uint8_t* p) {
        return (int)((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24));
    };
    const uint8_t* xb = x + (size_t)b * 34 + 2;
    const int4 a0 = make_int4(dword(xb), dword(xb + 4), dword(xb + 8), dword(xb + 12));
    const int4 a1 = make_int4(dword(xb + 16), dword(xb + 20), dword(xb + 24), dword(xb + 28));
    int s;
    if (wtype == HY_TYPE_Q8_0) {
        const uint8_t* wb = w + ((size_t)r * nb + b) * 34 + 2;
        s = dot_q8_block(make_int4(dword(wb), dword(wb + 4), dword(wb + 8), dword(wb + 12)),
                         make_int4(dword(wb + 16), dword(wb + 20), dword(wb + 24), dword(wb + 28)), a0, a1);
    } else {
        const uint8_t* wb = w + ((size_t)r * nb + b) * 18 + 2;
        int asum = 0;
        for (int j = 0; j < 32; j++) asum += (int8_t)xb[j];
        s = dot_q4_block(make_int4(dword(wb), dword(wb + 4), dword(wb + 8), dword(wb + 12)), a0, a1, asum);
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
