/* hy_probe.h -- measurement probes of libhy_probe.so (bench.py only).
 *
 * Not part of the product library libhy_moe.so and not declared in include/: these
 * kernels measure the ceilings the product's kernels are reported against.  Each
 * returns 0, or -1 with the reason in hyp_last_error(). */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char* hyp_last_error(void);

/* The grouped int8 GEMM's per-block instruction mix with no memory traffic, at the
 * GEMM's occupancy: per iteration and wave, two v_mfma_i32_32x32x32_i8 (the exact block
 * dots of two 32x32 tiles), two rank-1 v_mfma_f32_32x32x16_f16 (the scale products),
 * 32 v_cvt_f32_i32 + 32 v_fmac_f32.  Variant 1 runs only the four MFMAs, variant 2 only
 * the 64 vector ops (plus 32 integer adds that vary their operands), variant 3 the f16
 * alternative (each block dot from two f16 32x32x16 MFMAs, exact in fp32, no
 * conversions; the operand unpack to f16 is not counted), variant 4 variant 3 plus the
 * unpack of the shared int8 A operand to f16.  Each wave does iters * 2 * 32*32*32
 * block-dot MACs; out_dev holds work_groups * 512 floats. */
int hyp_block_mix(int32_t variant, uint32_t work_groups, uint32_t iters, float* out_dev, void* stream);

/* Reads `bytes` of buf_dev as the decode GEMV streams its weights.  Variant 0: `waves`
 * single-wave work groups, each streaming its own contiguous bytes / waves with 16-byte
 * global->LDS copies through a private 3-step ring of 8 KB steps (bytes a multiple of
 * waves x 8192); variant 1: a grid-stride 16-byte vector read by waves x 64 threads
 * (waves a multiple of 4); variant 2: variant 0 with non-temporal copies.  out_dev holds
 * waves x 64 floats: lane l of wave w sums word l of every step it streamed. */
int hyp_stream(int32_t variant, const void* buf_dev, uint64_t bytes, uint32_t waves, float* out_dev, void* stream);

/* Copy rate from a window of `bytes` (a power-of-two number of KB; small enough to stay
 * in L2): work_groups 4-wave work groups, each wave issuing `iters` batches of eight
 * 1 KB global->LDS copies of the window's chunks into its own 8 KB of LDS, waiting for
 * each batch.  Each launch copies work_groups x 4 x iters x 8 KB.  out_dev holds
 * work_groups x 256 floats. */
int hyp_l2_window(const void* buf_dev, uint64_t bytes, uint32_t work_groups, uint32_t iters, float* out_dev,
                  void* stream);

#ifdef __cplusplus
}
#endif
