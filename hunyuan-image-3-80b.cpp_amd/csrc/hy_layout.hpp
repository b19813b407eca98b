// hy_layout.hpp -- resident weight layout and work-arena views shared by the
// kernels and the C ABI.
//
// Resident weights of one layer (per matrix kind, experts 0..E-1 then the shared
// expert at index E), "row-group interleaved": rows are taken in groups of 64 and,
// inside a group, block b of all 64 rows is contiguous:
//   quant plane: [E+1][rows/64][cols/32][64 rows][bpb]  (bpb = 32 B Q8_0 int8,
//                16 B Q4_0 nibbles in GGUF block order, 128 B F32)
//   scale plane: [E+1][rows/64][cols/32][64 rows] fp16 (none for F32)
// A wave whose lane l owns row l of a group reads one contiguous 64*bpb chunk per
// block (the decode GEMV), and an MFMA row block stages 64-row x block chunks.
// F32 blocks (8 KB) are stored quad-major inside: floats 4q..4q+3 of the 64 rows
// form 1 KB, [8 quads][64 rows][4 floats], so each 16-byte load of the wave (lane =
// row, one quad) reads 1 KB contiguous.
// gate_up rows are packed so each 64-row group holds 32 SiLU rows then the
// matching 32 linear rows: packed row 64g+r is gate row 32g+r for r < 32 and up
// row I+32g+(r-32) for r >= 32.  Down rows keep their natural order.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace hy {

struct MatView {
    const uint8_t* qs;   // quant (or f32) plane of expert 0
    const uint16_t* sc;  // fp16 scale plane of expert 0 (nullptr for F32)
    size_t qs_stride;    // bytes between experts
    size_t sc_stride;    // scale elements between experts
    int rows, cols;
    int n_mats;          // matrices in the table (routed experts + shared)
};

__host__ __device__ inline int gu_packed_row(int orig, int I) {
    if (orig < I) return (orig / 32) * 64 + (orig % 32);
    const int r = orig - I;
    return (r / 32) * 64 + 32 + (r % 32);
}

// byte offset of block b of row r in an interleaved quant plane (bpb bytes per block)
__host__ __device__ inline size_t il_q_offset(int r, int b, int nb, int bpb) {
    return (((size_t)(r / 64) * nb + b) * 64 + (r % 64)) * (size_t)bpb;
}
// float offset of element j (0..31) of block b of row r in an F32 plane
__host__ __device__ inline size_t il_f32_offset(int r, int b, int nb, int j) {
    return ((size_t)(r / 64) * nb + b) * 64 * 32 + (size_t)(j / 4) * 256 + (r % 64) * 4 + j % 4;
}
// element offset of the scale of block b of row r
__host__ __device__ inline size_t il_s_offset(int r, int b, int nb) {
    return ((size_t)(r / 64) * nb + b) * 64 + (r % 64);
}
__host__ __device__ inline int block_bytes(int wtype) { return wtype == 8 ? 32 : (wtype == 2 ? 16 : 128); }

// Routing / dispatch products in the work arena.
struct Routing {
    const int* topi;       // [T][K] expert ids, rank order
    const float* topw;     // [T][K]
    const int* cnt;        // [E]
    const int* off;        // [E+1] start of each expert's sorted pair list
    const int* srt_tok;    // [T*K] token of sorted pair
    const int* comb_pos;   // [T][K] sorted positions, ascending expert order
    const float* comb_w;   // [T][K] matching weights
    const int* tile_e;     // [max_tiles] expert (E = shared)
    const int* tile_start; // [max_tiles] first pair (routed) / token (shared)
    const int* tile_n;     // [max_tiles] tokens in tile
    const int* meta;       // [0] n_routed_tiles, [1] n_tiles, [2] distinct experts, [3] T,
                           // [META_TILE_OFF + e] first tile of expert e (e <= E + 1)
};

// Quantized activations: rows of `cols` int8 with one fp16-valued scale (kept as
// f32) and the int sum of the block's quants (Q4_0 offset correction).
struct ActQ {
    int8_t* q;
    float* d;
    int* s;
    int cols;
};

}  // namespace hy
