// hy_mfma.hip -- grouped expert GEMMs on the int8 matrix cores (prefill / image-token
// batches).
//
// Work item = (tile, row block): a tile is up to TOK (token, expert) pairs of one
// expert (or TOK consecutive tokens for the shared expert), a row block is ROWS weight
// rows (ROWS/64 row groups of the row-group-interleaved weights).  Each K step copies
// KB GGUF blocks of the ROWS weight rows and of the tile's TOK activation rows
// straight from global memory into an LDS ring of stages; the activations (the gathered
// x, and h) are block-major in pair-slot order, so a tile's rows of one block are one
// contiguous run.  Two shapes, picked per call
// from the mean pairs per expert:
//   wide  (ROWS 128, TOK 128, KB 2): four waves, 2 row slabs x 2 token halves, each
//         wave 2 x 2 output tiles (64 rows x 64 tokens: one LDS read of each A and B
//         operand serves two tiles), a 2-stage ring (one stage in flight while one is
//         consumed), three work groups per CU (at most 168 VGPRs);
//   tall  (ROWS 256, TOK  64, KB 2): eight waves, 4 row slabs x 2 token halves, each
//         wave 2 x 1 tiles, a 3-stage ring, two work groups per CU -- keeps the waves
//         busy when experts see ~64 pairs.
// Every wave owns 2 (or 2 x 2) output tiles of 32 rows x 32 tokens and, per 32-wide
// block and 32 tokens, issues
// v_mfma_i32_32x32x32_i8: K = 32 is exactly one GGUF block, so each MFMA result is the
// exact int32 block dot sum_j w_j x_j of ggml's vec_dot, which is then rescaled in
// fp32 with the blocks taken in order: acc = fmaf(float(S), d_w * d_x, acc) -- the
// accumulation the oracle and the decode GEMV use, so all paths agree bit for bit.
// The 32x32 scale products d_w * d_x come from a rank-1 f16 MFMA (exact), which
// takes 16 multiplies per tile and block off the vector ALUs.
//
// MFMA operand / result layout (gfx950, checked on the device): A lane l holds 16
// bytes of row l%32, B lane l 16 bytes of column l%32, both at the same k offset
// 16*(l/32) inside the block; result register v of lane l is row
// 8*(v/4) + 4*(l/32) + v%4, column l%32.
//
// Modes: 0 = gate_up (packed rows: every 64-row slab holds 32 SiLU rows and the 32
// matching linear rows; epilogue h = silu(g) * u and Q8_0 quantization of h per token and
// slab); 1 = down for every tile, routed and shared (writes y[slot][row]; the combine
// kernel then forms out = resid + (y_shared + sum_{e ascending} w_e y_e)).
//
// Scheduling: work items are dealt to the 8 XCDs in tile groups (work-group ids go
// round robin over the XCDs); each XCD's last two rounds of items are claimed at run
// time through per-XCD counters, so an XCD that runs ahead takes over the others'
// tail (moe_mfma_kernel).
#include <utility>

#include "hy_device.hpp"
#include "hy_launch.hpp"
#include "hy_layout.hpp"
#include "hy_lds.hpp"

namespace hy {

typedef int v16i_t __attribute__((ext_vector_type(16)));
typedef float v16f_t __attribute__((ext_vector_type(16)));
typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));

constexpr int MM_XCD = 8;                  // XCDs of the device (work-group round robin)
constexpr int MM_CU_PER_XCD = 32;          // CUs per XCD (256 in all)
constexpr int MM_CTR_STRIDE = 32;          // ints between two work counters (one 128-byte line each)
constexpr int MM_CTR_INTS = 2 * MM_XCD * MM_CTR_STRIDE;  // [mode][XCD] counters of the grouped GEMM

// Tile shape.  LDS stage layout (bytes): A = CHUNKS (row group x block) chunks of
// 64 rows x 32 B int8 (Q4_0: 64 rows x 16 B raw nibbles); B = KB blocks of TOK tokens
// x 32 B; A scales = CHUNKS x 64 fp16; B scales = TOK tokens x KB f32.
//
// Bank swizzle of the 32-byte operand rows (A rows and B token rows): the two 16-byte
// halves of row r sit in swapped order when bit 3 of r is set.  An MFMA operand read
// (lane l: row l%32, half l/32) then touches 64 distinct banks per 16 lanes; without
// the swap rows r and r+8 share banks and every read takes two passes.  The copies
// keep their contiguous LDS destinations and fetch the swapped halves instead.
//
// WAVES waves per work group (one 64-row slab x 32 * TT tokens each); RING LDS stage
// slots (one computed, RING - 1 in flight).  8-wave shapes run two work groups per
// CU, the 4-wave 2 x 2 shape three, a 16-wave shape one.
template <int ROWS_, int TOK_, int KB_, int WAVES_ = 8, int RING_ = 3, int TT_ = 1, int GROUP_ = 1>
struct MmShape {
    static constexpr int ROWS = ROWS_, TOK = TOK_, KB = KB_, WAVES = WAVES_, RING = RING_;
    static constexpr int TT = TT_;                   // 32-token tiles per wave (1 or 2)
    static constexpr int GROUP = GROUP_;             // consecutive tiles scheduled together on one XCD
    static constexpr int THREADS = WAVES * WAVE;
    static constexpr int WG_PER_CU = WAVES == 16 ? 1 : (TT == 2 ? 3 : 2);
    static constexpr int SLABS = ROWS / 64;          // 64-row slabs (one per row group)
    static constexpr int TQ = WAVES / SLABS;         // column groups of 32 * TT tokens
    static constexpr int CHUNKS = SLABS * KB;
    static constexpr int ST_A = CHUNKS * 64 * 32;
    static constexpr int ST_AR = CHUNKS * 64 * 16;
    static constexpr int ST_B = TOK * KB * 32;
    static constexpr int ST_AS = CHUNKS * 64 * 2;
    static constexpr int ST_BS = TOK * KB * 4;
    // B rows: wave w copies block w % KB of TPW tokens x 32 B with 16-byte lanes
    static constexpr int TPW = TOK * KB / WAVES;
    static constexpr int B_LANES = TPW * 2;
    static constexpr int B_LOADS = (B_LANES + WAVE - 1) / WAVE;
    static constexpr int WPC = WAVES / CHUNKS;        // waves sharing one A chunk's copies
    static_assert(CHUNKS * WPC == WAVES && (WPC == 1 || WPC == 2), "A chunks split evenly over the waves");
    static_assert(WAVES == 8 || WAVES == 16 || (WAVES == 4 && TT == 2), "work group shapes");
    static_assert(RING >= 2, "at least one stage in flight while one is consumed");
    static_assert(TQ * 32 * TT == TOK, "token groups must cover the tile");
    static_assert(B_LANES % WAVE == 0 || B_LOADS == 1, "partial B loads only as a single load");
    static_assert(KB == 2 || KB == 1, "B-scale copy: one 4-byte piece per (token, block)");
    static_assert(WAVES % KB == 0 && TPW % 2 == 0, "B copies: whole token rows per wave");
};
using ShapeWide = MmShape<128, 128, 2, 4, 2, 2, 4>;
using ShapeTall = MmShape<256, 64, 2>;

struct MmArgs {
    MatView W;
    Routing R;
    const int8_t* aq;   // activations int8, block-major in slot order [Kdim/32][slots][32]: the
                        // gathered x (mode 0, gather_act_kernel) or h (mode 1)
    const float* ad;    // their scales (exact fp16 values) [Kdim/32][slots]
    int T, H, I, E, K;
    int Kdim;           // reduction length (H for mode 0, I for modes 1/2)
    int nrb;            // row blocks of the weight matrix
    int tiles_pad;      // tile bound rounded up to a multiple of MM_XCD x the shape's GROUP (sizes the grid)
    int8_t* hq;         // mode 0 outputs
    float* hd;
    int* hs;
    float* y;           // mode 1 output
    int* ctr;           // MM_CTR_INTS work counters, zeroed by gather_act_kernel before the gate/up launch
};

// Byte offset, inside a 32-byte operand row, of the row's 16-byte half h: the halves
// are swapped when bit 3 of the row is set (conflict-free MFMA operand reads).
__device__ __forceinline__ int swz_half(int row, int h) { return 16 * (h ^ ((row >> 3) & 1)); }

// Offset, inside a 32-row operand tile of 32-byte rows, of the 16 bytes MFMA lane
// (lr = l % 32, lg = l / 32) reads: row lr, half lg.
__device__ __forceinline__ int operand_lane_off(int lr, int lg) { return lr * 32 + swz_half(lr, lg); }

// Q4_0 unpack of one 64-row chunk by one wave, as contiguous 16-byte stores: lane l
// writes pieces l and 64 + l of the chunk's int8 operand rows (32 bytes each, halves
// swizzled by swz_half).  Piece d is half h = (d % 2) ^ (bit 3 of row d / 2) of row
// d / 2: the values n - 8 of the low (h = 0, elements 0-15) or high (h = 1, elements
// 16-31) nibbles of the row's 16 stored bytes; lanes 2j and 2j + 1 read the same
// nibble row.  nib = the chunk's nibble rows + 16 * (l / 2), dst = its int8 rows + 16 l,
// sh = 4 h (the same for rows l / 2 and 32 + l / 2).
__device__ __forceinline__ void unpack_q4_chunk_at(uint32_t nib, uint32_t dst, uint32_t sh) {
    v4i_t w0 = lds_b128_at<0>(nib);
    v4i_t w1 = lds_b128_at<512>(nib);
    lds_wait(w0, w1);
    auto cv = [sh](int v) {
        const uint32_t x = ((uint32_t)v >> sh) & 0x0F0F0F0Fu;
        return (int)(((x | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
    };
    lds_st128_at<0>(dst, v4i_t{cv(w0[0]), cv(w0[1]), cv(w0[2]), cv(w0[3])});
    lds_st128_at<1024>(dst, v4i_t{cv(w1[0]), cv(w1[1]), cv(w1[2]), cv(w1[3])});
}
__device__ __forceinline__ uint32_t unpack_q4_shift(int lane) { return 4u * (uint32_t)((lane & 1) ^ ((lane >> 4) & 1)); }

// The exact int32 dots of one 32-wide GGUF block over a 32x32 tile (K = 32 is one
// block): v_mfma_i32_32x32x32_i8 with a zero accumulator.
__device__ __forceinline__ v16i_t block_dot_tile(v4i_t A, v4i_t B) {
    const v16i_t zero = {};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, zero, 0, 0, 0);
}

// Per-block scale products c[row][tok] = d_w[row] * d_x[tok] for a 32x32 tile from one
// f16 MFMA: A holds d_w in k-slot 0 of lane group 0, B holds d_x in the same slot,
// every other slot is zero.  The product of two fp16 values is exact in fp32, so c
// equals the float multiply d_w * d_x bit for bit.
__device__ __forceinline__ v16f_t scale_outer(_Float16 dw, _Float16 dx, int lg) {
    v8h_t a = {}, b = {};
    if (lg == 0) {
        a[0] = dw;
        b[0] = dx;
    }
    const v16f_t zero = {};
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, zero, 0, 0, 0);
}


template <int WT, int MODE, class SH>
__global__ __launch_bounds__(SH::THREADS, SH::WG_PER_CU) void moe_mfma_kernel(MmArgs a) {
    constexpr int MM_ROWS = SH::ROWS, MM_TOK = SH::TOK, MM_KB = SH::KB, MM_SLABS = SH::SLABS;
    constexpr int MM_WAVES = SH::WAVES, MM_THREADS = SH::THREADS, MM_RING = SH::RING;
    constexpr bool Q4 = WT == HY_TYPE_Q4_0;
    // stage slot: A (int8, or Q4_0 nibbles), B, A scales, B scales, then a zero area
    // the upper lane half reads its rank-1 scale operands from
    constexpr int ZBYTES = 512;
    constexpr int STAGE = SH::ST_A * (Q4 ? 0 : 1) + (Q4 ? SH::ST_AR : 0) + SH::ST_B + SH::ST_AS + SH::ST_BS + ZBYTES;
    __shared__ __align__(16) uint8_t ring[MM_RING][STAGE];
    // Q4_0: the unpacked int8 A of a stage, double-buffered (stage s in aun[s & 1])
    __shared__ __align__(16) int8_t aun[Q4 ? 2 : 1][Q4 ? SH::ST_A : 16];
    static_assert(!Q4 || (SH::WPC == 1 && SH::CHUNKS * 64 == SH::THREADS),
                  "Q4_0: each wave copies whole nibble chunks and unpacks exactly the chunk it copied");
    static_assert((MM_RING * STAGE + (Q4 ? 2 * SH::ST_A : 16) + 8 * MM_TOK) * SH::WG_PER_CU <= 160 * 1024,
                  "the work groups of a CU fit its 160 KB of LDS");
    __shared__ int slot_s[MM_TOK];
    constexpr int OFF_A = 0;                                  // Q8_0: int8 A; Q4_0: raw nibbles
    constexpr int OFF_B = Q4 ? SH::ST_AR : SH::ST_A;
    constexpr int OFF_AS = OFF_B + SH::ST_B;
    constexpr int OFF_BS = OFF_AS + SH::ST_AS;
    constexpr int OFF_Z = OFF_BS + SH::ST_BS;
    static_assert(MM_KB * 128 <= ZBYTES, "scale offsets of the upper lanes stay in the zero area");
    // copies per wave per stage (every wave issues the same number; vmcnt counts them)
    constexpr int WPC = SH::WPC;
    constexpr int A_LOADS = Q4 ? 1 : 2 / WPC;
    constexpr int LOADS = A_LOADS + SH::B_LOADS + 1 + 1;
    static_assert((MM_RING - 2) * LOADS <= 63, "vmcnt counts at most 63 outstanding copies");

    // XCD-aware work mapping: work-group ids go round robin over the XCDs, so give
    // all row blocks of a tile the same id mod MM_XCD (they share the tile's
    // activation rows in that XCD's L2).  The wide shape takes GROUP = 4 consecutive
    // tiles (mostly one expert's) together on one XCD with their work groups
    // interleaved by row block, so one weight row block serves all four from L2 (two
    // against one: Zipf T=4096 Q4_0 ffn_up 2.578-2.617 -> 2.498-2.504 ms; four against
    // two, with the claimed tail below: the 4096-token Q8_0 stack -0.7 %, the Zipf
    // layer unchanged; eight: the Zipf layer 5 % slower.  On the tall shape's T=512
    // tiles, of two experts as often as of one, groups of two change nothing.  Before
    // the claimed tail, coarser groups ran slower: they unbalanced the XCDs.)
    //
    // The XCDs do not run equally fast (per-work-group stamps: the same full tile takes
    // 110-119 us on different XCDs of one launch), and with a fixed id -> item map the
    // launch waits for the slowest (4096-token Q8_0 gate/up launch: XCDs ending at
    // 2263-2457 us, the work groups' busy time 93 % of the launch's).  So only the
    // first part of each XCD's item list is fixed: its last RESERVE items (two rounds
    // of its work groups) are claimed through the XCD's work counter, and a work group
    // that finds its own XCD's list exhausted claims from the XCD with the most items
    // left.  Every item runs exactly once: a
    // fixed item by the one work group whose id maps to it, a reserved item by the
    // claim that drew it; the RESERVE work groups of an XCD whose ids follow its fixed
    // part each claim from their own counter first, so their claims alone cover that
    // XCD's reserve.  Work groups past an XCD's items (the tile bound's padding and
    // MM_XCD * SLACK extra ones) only steal, and exit as soon as nothing is left.
    constexpr int MM_G = SH::GROUP;
    constexpr int RESERVE = 2 * MM_CU_PER_XCD * SH::WG_PER_CU;
    const int id = (int)blockIdx.x;
    const int xcd = id % MM_XCD, local = id / MM_XCD;
    const int ntiles = a.R.meta[1];
    const int per_group = MM_G * a.nrb;                 // items of one tile group
    const int ngroups = (ntiles + MM_G - 1) / MM_G;     // group g belongs to XCD g % MM_XCD
    auto items_of = [&](int x) { return ngroups > x ? (ngroups - x + MM_XCD - 1) / MM_XCD * per_group : 0; };
    auto fixed_of = [&](int n_items) { return n_items > RESERVE ? n_items - RESERVE : 0; };
    const int own = items_of(xcd), fixed = fixed_of(own);
    int ix = xcd, ik = local;  // the item: XCD ix's ik-th
    if (local >= fixed) {
        __shared__ int claim_s[2];
        int* ctr = a.ctr + MODE * MM_XCD * MM_CTR_STRIDE;
        if (threadIdx.x < WAVE) {
            const int ln = threadIdx.x;
            int k = 0x3fffffff;
            if (ln == 0 && local < own) k = atomicAdd(ctr + xcd * MM_CTR_STRIDE, 1);
            k = __shfl(k, 0);
            int cx = -1, ck = 0;
            if (fixed + k < own) {
                cx = xcd;
                ck = fixed + k;
            } else {
                // steal: lanes 0..MM_XCD-1 read the counters, the XCD with the most reserved
                // items left (the lowest on ties) is drawn from; a lost race reads again
                for (int tries = 0; tries < 64 && cx < 0; tries++) {
                    int left = 0;
                    if (ln < MM_XCD) {
                        const int n_items = items_of(ln);
                        left = n_items - fixed_of(n_items) -
                               __hip_atomic_load(ctr + ln * MM_CTR_STRIDE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                    int best = left, bx = ln;
                    for (int m = 1; m < MM_XCD; m <<= 1) {
                        const int ob = __shfl_xor(best, m), ox = __shfl_xor(bx, m);
                        if (ob > best || (ob == best && ox < bx)) {
                            best = ob;
                            bx = ox;
                        }
                    }
                    best = __shfl(best, 0);
                    bx = __shfl(bx, 0);
                    if (best <= 0) break;
                    int k2 = 0;
                    if (ln == 0) k2 = atomicAdd(ctr + bx * MM_CTR_STRIDE, 1);
                    k2 = __shfl(k2, 0);
                    const int n_items = items_of(bx), f = fixed_of(n_items);
                    if (f + k2 < n_items) {
                        cx = bx;
                        ck = f + k2;
                    }
                }
            }
            if (ln == 0) {
                claim_s[0] = cx;
                claim_s[1] = ck;
            }
        }
        __syncthreads();
        ix = claim_s[0];
        ik = claim_s[1];
        if (ix < 0) return;
    }
    const int q = ik / per_group, within = ik % per_group;
    const int rb = within / MM_G;
    const int tile = (q * MM_XCD + ix) * MM_G + within % MM_G;
    if (tile >= ntiles) return;
    const int e = a.R.tile_e[tile];
    const int start = a.R.tile_start[tile], n = a.R.tile_n[tile];
    const bool shared = e == a.E;
    const int row0 = rb * MM_ROWS;
    const int Kd = a.Kdim;
    const int nb = Kd / QK;
    const int tid = threadIdx.x;
    const int wave = tid / WAVE, lane = tid % WAVE;

    if (tid < MM_TOK) {
        // the pair's slot: the row of the slot-ordered operands (gathered x, h) and of y
        int slot = 0;
        if (tid < n) slot = shared ? a.T * a.K + start + tid : a.R.off[e] + start + tid;
        slot_s[tid] = slot;
    }
    __syncthreads();

    // zero areas of the stage slots (never written by the copies)
    for (int i = tid; i < MM_RING * ZBYTES / 4; i += MM_THREADS)
        reinterpret_cast<uint32_t*>(ring[i / (ZBYTES / 4)] + OFF_Z)[i % (ZBYTES / 4)] = 0u;
    __syncthreads();

    constexpr int BPB = Q4 ? 16 : 32;
    const int G0 = row0 / 64;
    const int wv = __builtin_amdgcn_readfirstlane(wave);  // wave index as a scalar
    // copy sources: a wave-uniform base (advanced per stage) + a per-lane 32-bit offset
    // A: chunk c = wave / WPC (row group c / KB, block c % KB) of 64 rows x BPB bytes;
    // with WPC = 2 each of the chunk's two waves copies one half of it
    constexpr int CHB = 64 * BPB;  // bytes per chunk
    const int ch = wv / WPC, half = wv % WPC;
    const uint8_t* a_src = a.W.qs + (size_t)e * a.W.qs_stride +
                           ((size_t)(G0 + ch / MM_KB) * nb + ch % MM_KB) * CHB + half * (CHB / WPC);
    const uint16_t* as_src = a.W.sc + (size_t)e * a.W.sc_stride + ((size_t)(G0 + ch / MM_KB) * nb + ch % MM_KB) * 64 +
                             half * (64 / WPC);
    // B rows: wave w copies block w % KB of tokens (w / KB) * TPW .. + TPW, as 16-byte
    // pieces; lane position p (copy v, lane l: p = 64 v + l) lands at +16 p, i.e. token
    // row p / 2, position p % 2, which holds half (p % 2) ^ (bit 3 of the row).  The
    // operand is block-major in slot order ([Kdim/32][slots][32 B]): the tile's
    // consecutive slots are consecutive 32-byte pieces of one block plane, so each copy
    // reads one contiguous 1 KB; a stage advances KB planes
    constexpr int TPW = SH::TPW;
    const uint32_t n_slots = (uint32_t)(a.T * a.K + a.T);  // rows of the block planes
    uint32_t b_off[SH::B_LOADS];  // 32-bit: the host keeps slots x Kd below 2^32
#pragma unroll
    for (int v = 0; v < SH::B_LOADS; v++) {
        const int p = v * WAVE + lane;
        const int bt = (wave / MM_KB) * TPW + (p % SH::B_LANES) / 2;  // in range for masked lanes too
        b_off[v] = ((uint32_t)(wave % MM_KB) * n_slots + (uint32_t)slot_s[bt]) * 32u + swz_half(bt, p & 1);
    }
    const uint32_t b_step = n_slots * 32u;  // bytes per block plane of the B source
    // A rows (int8): copy lane l lands at +16 l (row l / 2 of a 32-row piece, position
    // l % 2) and fetches half (l % 2) ^ (bit 3 of the row); Q4_0 nibbles are copied as
    // they are and swizzled when unpacked
    const uint32_t a_sw = (uint32_t)((lane / 2) * 32 + swz_half(lane / 2, lane & 1));
    // B scales: wave w copies tokens w*TOK/8 .. +TOK/8, KB f32 each, as KB 4-byte pieces
    // (the token's KB scales sit in KB block planes)
    static_assert(MM_KB <= 2, "B scales: one 4-byte piece per (token, block), KB of them per token");
    constexpr int BS_LANES = MM_TOK / MM_WAVES * MM_KB;
    const int bst = wave * (MM_TOK / MM_WAVES) + (lane / MM_KB) % (MM_TOK / MM_WAVES);
    const uint32_t bs_off = ((uint32_t)(lane % MM_KB) * n_slots + (uint32_t)slot_s[bst]) * 4;
    const uint32_t bs_step = n_slots * 4u;  // bytes per block plane of the B-scale source

    // issue the asynchronous copies of stage s into ring slot s % MM_RING; lanes
    // outside a copy's range are masked (the wave still issues it once)
    // the copy sources as buffer descriptors: per copy a 32-bit lane offset (VGPR) and
    // the stage's offset (SGPR).  Offsets stay below 2^32: A and its scales within one
    // expert's chunk column, B rows x Kd (the host keeps that below 2^32), B scales
    // rows x nb x 4.
    const __amdgpu_buffer_rsrc_t r_a = buf_rsrc(a_src), r_as = buf_rsrc(as_src), r_b = buf_rsrc(a.aq),
                                 r_bs = buf_rsrc(a.ad);
    auto issue = [&](int s) {
        uint8_t* st = ring[s % MM_RING];
        const uint32_t kb0 = (uint32_t)(s * MM_KB);
        uint8_t* ad = st + OFF_A + ch * CHB + half * (CHB / WPC);
        if (Q4 && WPC == 2) {
            if (lane < 32) b2l(r_a, ad, 16u * lane, kb0 * CHB);  // 512 B
        } else {
#pragma unroll
            for (int c = 0; c < A_LOADS; c++) b2l(r_a, ad + c * 1024, (Q4 ? 16u * lane : a_sw) + c * 1024u, kb0 * CHB);
        }
        // B rows of this wave's tokens
        uint8_t* bdst = st + OFF_B + (wv % MM_KB) * (MM_TOK * 32) + (wv / MM_KB) * (TPW * 32);
#pragma unroll
        for (int v = 0; v < SH::B_LOADS; v++)
            if (v * WAVE + lane < SH::B_LANES) b2l(r_b, bdst + v * 1024, b_off[v], kb0 * b_step);
        // A scales of the chunk: 64 fp16 = 128 B (lanes 0..7), or its half (lanes 0..3)
        if (lane < 8 / WPC) b2l(r_as, st + OFF_AS + ch * 128 + half * (128 / WPC), 16u * lane, kb0 * 128u);
        // B scales of this wave's tokens
        uint8_t* sdst = st + OFF_BS + wv * (MM_TOK / MM_WAVES) * MM_KB * 4;
        if (lane < BS_LANES) b2l<4>(r_bs, sdst, bs_off, kb0 * bs_step);
    };

    const int sl = wave % MM_SLABS;    // 64-row slab within the row block
    const int nq = wave / MM_SLABS;    // 32-token column group of the tile
    constexpr int TT = SH::TT;
    const bool active = nq * 32 * TT < n;   // waves past the tile's last pair skip the math
    const int lr = lane % 32, lg = lane / 32;
    // acc0 / acc1: rows 0-31 / 32-63 of the slab x the first 32 tokens; acc2 / acc3 the
    // same rows x the second 32 tokens (TT = 2)
    float acc0[16], acc1[16], acc2[TT == 2 ? 16 : 1], acc3[TT == 2 ? 16 : 1];
#pragma unroll
    for (int v = 0; v < 16; v++) {
        acc0[v] = 0.0f;
        acc1[v] = 0.0f;
        if constexpr (TT == 2) {
            acc2[v] = 0.0f;
            acc3[v] = 0.0f;
        }
    }
    // per-lane LDS offsets inside a stage slot (the block kb adds a constant):
    //   A rows lr and 32+lr of this wave's slab, 16-byte half lg (swizzled)
    //   B row (token) nq*32+lr of the block, half lg (swizzled)
    //   rank-1 scale operands: lanes of the lower half read d_w of rows lr / 32+lr and
    //   d_x of token nq*32+lr; lanes of the upper half read zeros
    const uint32_t a_lane = (uint32_t)((Q4 ? 0 : OFF_A) + sl * MM_KB * 2048 + operand_lane_off(lr, lg));
    const uint32_t b_lane = (uint32_t)(OFF_B + nq * 32 * TT * 32 + operand_lane_off(lr, lg));
    const uint32_t sw_lane = (uint32_t)(lg == 0 ? OFF_AS + sl * MM_KB * 128 + lr * 2 : OFF_Z);
    const uint32_t sx_lane = (uint32_t)(lg == 0 ? OFF_BS + (nq * 32 * TT + lr) * MM_KB * 4 : OFF_Z);
    const uint32_t ring0 = lds_off(ring[0]);
    const uint32_t aun0 = lds_off(aun);
    // Q4_0 unpack: this thread's nibble row in a stage slot (chunk tid / 64, row tid % 64)
    // and the two swizzled halves of its int8 row in aun[0]
    const int un_c = tid >> 6;
    const uint32_t un_src = ring0 + (uint32_t)(OFF_A + un_c * 1024 + (lane >> 1) * 16);
    const uint32_t un_dst = aun0 + (uint32_t)(un_c * 2048 + lane * 16);
    const uint32_t un_sh = unpack_q4_shift(lane);
    // rank-1 operands {d, 0, 0, ...}: only element 0 changes, the zeros stay in place
    v4i_t xa0 = {0, 0, 0, 0}, xa1 = {0, 0, 0, 0}, xb = {0, 0, 0, 0};

    // one 32-wide block kb of a stage: this lane's B row, scale and A row addresses in
    // the stage's slot
    auto block = [&]<int KBI>(uint32_t bq, uint32_t swq, uint32_t sxq, uint32_t abase) {
        v4i_t A0 = lds_b128_at<KBI * 2048>(abase);
        v4i_t A1 = lds_b128_at<KBI * 2048 + 1024>(abase);
        v4i_t B = lds_b128_at<KBI * MM_TOK * 32>(bq);
        uint32_t dw0 = lds_u16_at<KBI * 128>(swq);
        uint32_t dw1 = lds_u16_at<KBI * 128 + 64>(swq);
        uint32_t dxb = lds_b32_at<KBI * 4>(sxq);
        v4i_t B1;
        uint32_t dxb1;
        if constexpr (TT == 2) {
            B1 = lds_b128_at<KBI * MM_TOK * 32 + 1024>(bq);
            dxb1 = lds_b32_at<KBI * 4 + 32 * MM_KB * 4>(sxq);
            lds_wait(A0, A1, B, B1, dw0, dw1, dxb, dxb1);
        } else {
            lds_wait(A0, A1, B, dw0, dw1, dxb);
        }
        // the block's MFMAs issue at raised wave priority, so a wave whose operands are
        // ready reaches the matrix unit ahead of the other waves' rescale (gate/up -2 %
        // at 4096 Q8_0 tokens, -3 % at 4096 Q4_0, -4 % at 512 Q8_0; down -2 % with the
        // 2 x 2 tiles, nothing with 2 x 1)
        __builtin_amdgcn_s_setprio(1);
        const v16i_t S0 = block_dot_tile(A0, B);
        const v16i_t S1 = block_dot_tile(A1, B);
        // the upper lanes read zeros; d_x is an fp16 value stored as f32, so the
        // truncating pack is exact
        xa0[0] = (int)dw0;
        xa1[0] = (int)dw1;
        xb[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_pkrtz(__builtin_bit_cast(float, dxb), 0.0f));
        const v16f_t zf = {};
        const v16f_t C0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_t, xa0),
                                                                 __builtin_bit_cast(v8h_t, xb), zf, 0, 0, 0);
        const v16f_t C1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_t, xa1),
                                                                 __builtin_bit_cast(v8h_t, xb), zf, 0, 0, 0);
        __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int v = 0; v < 16; v++) {
            acc0[v] = fmaf((float)S0[v], C0[v], acc0[v]);
            acc1[v] = fmaf((float)S1[v], C1[v], acc1[v]);
        }
        if constexpr (TT == 2) {
            // the second 32 tokens: same A operands and weight scales
            __builtin_amdgcn_s_setprio(1);
            const v16i_t S2 = block_dot_tile(A0, B1);
            const v16i_t S3 = block_dot_tile(A1, B1);
            xb[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_pkrtz(__builtin_bit_cast(float, dxb1), 0.0f));
            const v16f_t C2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_t, xa0),
                                                                     __builtin_bit_cast(v8h_t, xb), zf, 0, 0, 0);
            const v16f_t C3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_t, xa1),
                                                                     __builtin_bit_cast(v8h_t, xb), zf, 0, 0, 0);
            __builtin_amdgcn_s_setprio(0);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                acc2[v] = fmaf((float)S2[v], C2[v], acc2[v]);
                acc3[v] = fmaf((float)S3[v], C3[v], acc3[v]);
            }
        }
    };

    const int nstage = nb / MM_KB;
#pragma unroll
    for (int i = 0; i < MM_RING - 1; i++)
        if (i < nstage) issue(i);
    // per-lane LDS read bases at ring slot 0, plus the slot's offset (s % RING) * STAGE
    // kept in a scalar that wraps at the ring's end: one vector add per address and stage
    const uint32_t a_q0 = ring0 + a_lane, b_q0 = ring0 + b_lane, sw_q0 = ring0 + sw_lane, sx_q0 = ring0 + sx_lane;
    uint32_t soff = 0;
    for (int s = 0; s < nstage; s++) {
        soff = __builtin_amdgcn_readfirstlane(soff);
        // stage s landed (this wave's loads)
        wait_copies<LOADS, MM_RING - 2>(nstage - 1 - s);
        uint32_t abase;
        if constexpr (Q4) {
            // nibbles -> int8 (n - 8): wave w converts chunk w, the chunk it copied itself
            // (row = lane), so its own copies having landed is enough; the result goes to
            // aun[s & 1], last read by stage s - 2's math, which every wave finished before
            // the previous barrier
            const uint32_t ab = (uint32_t)((s & 1) * SH::ST_A);
            unpack_q4_chunk_at(un_src + soff, un_dst + ab, un_sh);
            lds_wait();
            abase = aun0 + ab + a_lane;
        } else {
            abase = a_q0 + soff;
        }
        // every wave's copies of stage s landed (and, for Q4_0, its unpack is written)
        __builtin_amdgcn_s_barrier();
        // refill: slot (s + RING - 1) % RING was last read in iteration s-1 (its B by the
        // math, its Q4_0 nibbles by the unpack), finished by every wave before this
        // barrier -- issue it now so that RING - 1 stages are in flight during the math
        if (s + MM_RING - 1 < nstage) issue(s + MM_RING - 1);
        if (active) {
            const uint32_t bq = b_q0 + soff, swq = sw_q0 + soff, sxq = sx_q0 + soff;
            [&]<int... KBI>(std::integer_sequence<int, KBI...>) {
                (block.template operator()<KBI>(bq, swq, sxq, abase), ...);
            }(std::make_integer_sequence<int, MM_KB>{});
        }
        soff = soff + STAGE == (uint32_t)(MM_RING * STAGE) ? 0u : soff + STAGE;
    }

    // ---- epilogues: one per 32-token column group of the wave (ag = the rows of the
    // slab's first half, au = the second half)
    auto epilogue = [&](const float (&ag)[16], const float (&au)[16], int j) {
        if (j >= n) return;
        if (MODE == 0) {
            // ag = gate rows, au = matching up rows of slab (MM_SLABS * rb + sl)
            const int slab = MM_SLABS * rb + sl;
            float h[16];
            float amax = 0.0f;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                h[v] = swiglu(ag[v], au[v]);
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
            // h block-major: block (slab) plane, slot row of 32 bytes
            const size_t hi = (size_t)slab * (size_t)(a.T * a.K + a.T) + (size_t)slot_s[j];
            int8_t* dst = a.hq + hi * QK;
#pragma unroll
            for (int g = 0; g < 4; g++) *reinterpret_cast<int*>(dst + 8 * g + 4 * lg) = packed[g];
            if (lg == 0) {
                a.hd[hi] = h2f(f2h(d));
                a.hs[hi] = qsum;
            }
        } else {
            const int rbase = row0 + sl * 64;
            float* yr = a.y + (size_t)slot_s[j] * a.H;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int r = 8 * g + 4 * lg;
                *reinterpret_cast<float4*>(yr + rbase + r) = make_float4(ag[4 * g], ag[4 * g + 1], ag[4 * g + 2], ag[4 * g + 3]);
                *reinterpret_cast<float4*>(yr + rbase + 32 + r) =
                    make_float4(au[4 * g], au[4 * g + 1], au[4 * g + 2], au[4 * g + 3]);
            }
        }
    };
    if (!active) return;
    const int j0 = nq * 32 * TT + lr;  // pair index within the tile
    epilogue(acc0, acc1, j0);
    if constexpr (TT == 2) epilogue(acc2, acc3, j0 + 32);
}

// The dispatched activations of the gate/up products (einsum_dispatch,
// src/hunyuan_moe_full.cpp:352-373, as a copy of the Q8_0 activations): slot r of the
// expert-sorted pair order (the shared expert's token t at slot T*K + t) receives its
// token's quantized row, block-major -- plane b holds every slot's block b (32 bytes)
// and its scale -- so that the grouped GEMM's copies of a tile's consecutive slots read
// contiguous memory.  A wave copies 16 slots x 4 blocks, one 32-byte block per thread
// (thread = 4 slot + block): each slot's 4 blocks are one 128-byte run of its token's
// row, each block's 16 slots one 512-byte run of its plane.
__global__ __launch_bounds__(256) void gather_act_kernel(const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                         const int* __restrict__ srt_tok, int T, int TK, int n_slots,
                                                         int nb, int8_t* __restrict__ gq, float* __restrict__ gd,
                                                         int* __restrict__ ctr) {
    const size_t wt = ((size_t)blockIdx.x * 256 + threadIdx.x) >> 6;  // the wave's (16 slots x 4 blocks) tile
    // the grouped GEMM's work counters start at zero for the two launches that follow
    if (blockIdx.x == 0 && threadIdx.x < 2 * MM_XCD) ctr[threadIdx.x * MM_CTR_STRIDE] = 0;
    const int lane = threadIdx.x & 63;
    const size_t n_sg = ((size_t)n_slots + 15) / 16;
    const int r = (int)(wt % n_sg) * 16 + (lane >> 2), b = (int)(wt / n_sg) * 4 + (lane & 3);
    if (r >= n_slots || b >= nb) return;
    int tok = r < TK ? srt_tok[r] : r - TK;
    tok = tok < 0 ? 0 : (tok >= T ? T - 1 : tok);
    const v4i_t* src = reinterpret_cast<const v4i_t*>(xq + ((size_t)tok * nb + b) * QK);
    v4i_t* dst = reinterpret_cast<v4i_t*>(gq + ((size_t)b * n_slots + r) * QK);
    const v4i_t lo = src[0], hi = src[1];
    dst[0] = lo;
    dst[1] = hi;
    gd[(size_t)b * n_slots + r] = xd[(size_t)tok * nb + b];
}

// Per-block int32 dots through the grouped GEMM's own operand path (hy_block_dots
// path 1), one wave per (64-row group, block).  The wave stages the block's 64 weight
// rows in the GEMM's LDS operand layout -- Q8_0 as swizzled 32-byte rows; Q4_0 as the
// raw 16-byte nibble rows, then the GEMM's stage unpack (unpack_q4_chunk_at) -- and the
// activation block into all 32 token rows of a B tile with the same swizzle, reads its
// A0 / A1 / B operands at the GEMM's lane offsets (operand_lane_off) and issues the
// GEMM's two block-dot MFMAs (block_dot_tile).  Every entry of the two 32x32 results
// is the dot of its weight row with the replicated activation block; the one written
// for (row r, block b) sits in column (r + b) % 32, so that over the rows and blocks
// every lane and every result register of both tiles is read out.  Rows past `rows`
// stage zeros and write nothing.
template <int WT>
__global__ __launch_bounds__(WAVE) void block_dots_mfma_kernel(const uint8_t* __restrict__ w,
                                                               const uint8_t* __restrict__ x, int rows, int nb,
                                                               int* __restrict__ out) {
    constexpr bool Q4 = WT == HY_TYPE_Q4_0;
    constexpr int BB = Q4 ? 18 : 34;  // GGUF block bytes (fp16 scale + quants)
    __shared__ __align__(16) int8_t a_s[64 * 32];
    __shared__ __align__(16) uint8_t nib_s[Q4 ? 64 * 16 : 16];
    __shared__ __align__(16) int8_t b_s[32 * 32];
    const int g = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const int r = g * 64 + lane;  // weight row this lane stages
    // GGUF blocks are only 2-byte aligned: assemble the dwords bytewise
    auto dw4 = [](const uint8_t* p) {
        int v[4];
        for (int i = 0; i < 4; i++)
            v[i] = (int)((uint32_t)p[4 * i] | ((uint32_t)p[4 * i + 1] << 8) | ((uint32_t)p[4 * i + 2] << 16) |
                         ((uint32_t)p[4 * i + 3] << 24));
        return v4i_t{v[0], v[1], v[2], v[3]};
    };
    const v4i_t zero4 = {0, 0, 0, 0};
    const uint8_t* wq = w + ((size_t)(r < rows ? r : 0) * nb + b) * BB + 2;
    if constexpr (Q4) {
        lds_st128(nib_s + lane * 16, r < rows ? dw4(wq) : zero4);
        lds_wait();
        __syncthreads();
        unpack_q4_chunk_at(lds_off(nib_s) + (uint32_t)((lane >> 1) * 16), lds_off(a_s) + (uint32_t)(lane * 16),
                           unpack_q4_shift(lane));
    } else {
        lds_st128(a_s + lane * 32 + swz_half(lane, 0), r < rows ? dw4(wq) : zero4);
        lds_st128(a_s + lane * 32 + swz_half(lane, 1), r < rows ? dw4(wq + 16) : zero4);
    }
    // B: every token row holds activation block b; lane l writes half l / 32 of row l % 32
    const int lr = lane % 32, lg = lane / 32;
    lds_st128(b_s + lr * 32 + swz_half(lr, lg), dw4(x + (size_t)b * 34 + 2 + 16 * lg));
    lds_wait();
    __syncthreads();
    const int off = operand_lane_off(lr, lg);
    v4i_t A0 = lds_b128(a_s + off), A1 = lds_b128(a_s + 1024 + off), B = lds_b128(b_s + off);
    lds_wait(A0, A1, B);
    const v16i_t S0 = block_dot_tile(A0, B), S1 = block_dot_tile(A1, B);
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int i = 8 * (v / 4) + 4 * lg + v % 4;  // tile row of result register v
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int rr = g * 64 + 32 * t + i;
            if (rr < rows && lr == (rr + b) % 32) out[(size_t)rr * nb + b] = t ? S1[v] : S0[v];
        }
    }
}

hipError_t launch_block_dots_mfma(int wtype, const uint8_t* w, const uint8_t* x, int rows, int nb, int* out,
                                  hipStream_t s) {
    const dim3 grid((unsigned)((rows + 63) / 64), (unsigned)nb);
    if (wtype == HY_TYPE_Q4_0)
        hipLaunchKernelGGL(block_dots_mfma_kernel<HY_TYPE_Q4_0>, grid, dim3(WAVE), 0, s, w, x, rows, nb, out);
    else
        hipLaunchKernelGGL(block_dots_mfma_kernel<HY_TYPE_Q8_0>, grid, dim3(WAVE), 0, s, w, x, rows, nb, out);
    return hipGetLastError();
}

template <int MODE, class SH>
static hipError_t launch_mode(int wtype, MmArgs a, int n_tiles_bound, int rows, hipStream_t s) {
    a.nrb = rows / SH::ROWS;
    a.tiles_pad = (n_tiles_bound + MM_XCD * SH::GROUP - 1) / (MM_XCD * SH::GROUP) * (MM_XCD * SH::GROUP);
    // every item of the tile bound has its work group, plus half a round per XCD that
    // only steals (a fast XCD's reserve claims beyond its own items)
    constexpr int SLACK = MM_CU_PER_XCD * SH::WG_PER_CU / 2;
    const dim3 grid(a.tiles_pad * a.nrb + MM_XCD * SLACK);
    if (wtype == HY_TYPE_Q4_0)
        hipLaunchKernelGGL((moe_mfma_kernel<HY_TYPE_Q4_0, MODE, SH>), grid, dim3(SH::THREADS), 0, s, a);
    else
        hipLaunchKernelGGL((moe_mfma_kernel<HY_TYPE_Q8_0, MODE, SH>), grid, dim3(SH::THREADS), 0, s, a);
    return hipGetLastError();
}

template <int MODE>
static hipError_t launch_shape(int wtype, int shape, MmArgs a, int n_tiles_bound, int rows, hipStream_t s) {
    if (shape == MM_SHAPE_TALL) return launch_mode<MODE, ShapeTall>(wtype, a, n_tiles_bound, rows, s);
    return launch_mode<MODE, ShapeWide>(wtype, a, n_tiles_bound, rows, s);
}

template <class SH>
static bool shape_fits(int H, int I) {
    return H % SH::ROWS == 0 && (2 * I) % SH::ROWS == 0 && (H / QK) % SH::KB == 0 && (I / QK) % SH::KB == 0;
}

bool mfma_path_ok(int wtype, int H, int I) {
    return (wtype == HY_TYPE_Q8_0 || wtype == HY_TYPE_Q4_0) && shape_fits<ShapeWide>(H, I);
}

// The tall shape (64-pair tiles, 256-row blocks) wins while experts see about 64
// pairs each (a 128-pair tile would leave half its waves idle); beyond ~96 the wide
// shape's reuse of every weight byte over 128 pairs wins.
int mfma_shape(int T, int K, int E, int H, int I) {
    const bool tall = shape_fits<ShapeTall>(H, I) && (int64_t)T * K < (int64_t)96 * E;
    return tall ? MM_SHAPE_TALL : MM_SHAPE_WIDE;
}

int mfma_shape_tokens(int shape) {
    return shape == MM_SHAPE_TALL ? ShapeTall::TOK : ShapeWide::TOK;
}

hipError_t launch_gather_act(const ActQ& X, const Routing& R, int T, int K, int H, int8_t* gq, float* gd,
                             int* mm_ctr, hipStream_t s) {
    const int n_slots = T * K + T, nb = H / QK;
    const size_t wave_tiles = (((size_t)n_slots + 15) / 16) * (((size_t)nb + 3) / 4);
    hipLaunchKernelGGL(gather_act_kernel, dim3((unsigned)((wave_tiles * 64 + 255) / 256)), dim3(256), 0, s, X.q, X.d,
                       R.srt_tok, T, T * K, n_slots, nb, gq, gd, mm_ctr);
    return hipGetLastError();
}

hipError_t launch_ffn_up_mfma(int wtype, int shape, int n_tiles_bound, const MatView& W, const Routing& R,
                              const ActQ& X, int T, int H, int I, int E, int K, int8_t* hq, float* hd, int* hs,
                              int* mm_ctr, hipStream_t s) {
    MmArgs a{W, R, X.q, X.d, T, H, I, E, K, H, 0, 0, hq, hd, hs, nullptr, mm_ctr};
    return launch_shape<0>(wtype, shape, a, n_tiles_bound, 2 * I, s);
}

hipError_t launch_ffn_down_mfma(int wtype, int shape, int n_tiles_bound, const MatView& W, const Routing& R,
                                const int8_t* hq, const float* hd, int T, int H, int I, int E, int K, float* y,
                                int* mm_ctr, hipStream_t s) {
    MmArgs a{W, R, hq, hd, T, H, I, E, K, I, 0, 0, nullptr, nullptr, nullptr, y, mm_ctr};
    return launch_shape<1>(wtype, shape, a, n_tiles_bound, H, s);
}

int mfma_counter_ints() { return MM_CTR_INTS; }

}  // namespace hy
