// hy_layout.hpp -- resident weight layout and work-arena views shared by the
// kernels and the C ABI.
//
// Resident weights of one layer (per matrix kind, experts 0..E-1 then the shared
// expert at index E):
//   Q8_0: qs  int8   [E+1][rows][cols]        scale fp16 [E+1][rows][cols/32]
//   Q4_0: qs  uint8  [E+1][rows][cols/2]      scale fp16 [E+1][rows][cols/32]
//         (each 16-byte group keeps the GGUF block order: byte j = elem j | elem j+16 << 4)
//   F32 : f32        [E+1][rows][cols]
// gate_up rows are stored interleaved in groups of 32: packed row 64g+r holds gate
// row 32g+r for r < 32 and up row I+32g+(r-32) for r >= 32, so one 64-row slab
// carries matching SiLU and linear halves.  Down rows keep their natural order.
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
};

__host__ __device__ inline int gu_packed_row(int orig, int I) {
    if (orig < I) return (orig / 32) * 64 + (orig % 32);
    const int r = orig - I;
    return (r / 32) * 64 + 32 + (r % 32);
}

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
    const int* meta;       // [0] n_routed_tiles, [1] n_tiles, [2] distinct experts
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
