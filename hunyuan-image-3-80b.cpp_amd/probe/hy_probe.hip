// hy_probe.hip -- measurement probes (bench.py only; built into libhy_probe.so, not into
// the product library libhy_moe.so): the grouped GEMM's per-block instruction mix
// (compute only), the HBM read rate of the decode GEMV's access pattern, and the copy
// rate from an L2-resident window.
//
// Each wave repeats, `iters` times, exactly the math the grouped int8 GEMM issues for
// one 32-wide GGUF block of its two 32x32 output tiles (hy_mfma.hip):
//   * two v_mfma_i32_32x32x32_i8: the exact int32 block dots of the two tiles;
//   * two rank-1 v_mfma_f32_32x32x16_f16: the 32x32 scale products d_w * d_x;
//   * 32 v_cvt_f32_i32 + 32 v_fmac_f32: acc = fmaf((float)S, C, acc) per output.
// No memory traffic, no LDS, no barriers; launched at the GEMM's occupancy (8-wave
// work groups, two per CU, at most 128 VGPRs: four waves per SIMD).  Its rate is the
// ceiling the GEMM's instruction mix allows on this part; variants time the matrix
// and vector halves alone, and the alternative that takes the block dots from f16
// MFMAs (int8 values are exact in f16 and a 32-term dot of them stays below 2^24, so
// the fp32 result is the exact dot and needs no conversion).
#include "hy_device.hpp"
#include "hy_launch.hpp"
#include "hy_lds.hpp"
#include "hy_probe.h"

#include <cstdio>

namespace hy {

namespace {

typedef int v16i_p __attribute__((ext_vector_type(16)));
typedef float v16f_p __attribute__((ext_vector_type(16)));
typedef _Float16 v8h_p __attribute__((ext_vector_type(8)));
typedef int v4i_p __attribute__((ext_vector_type(4)));
typedef _Float16 v2h_p __attribute__((ext_vector_type(2)));

constexpr int PROBE_THREADS = 512;

// VARIANT 0: the full per-block mix; 1: the four MFMAs only; 2: the 64 vector ops only, plus
// 32 integer adds that vary their operands; 3: the block dots as two chained
// v_mfma_f32_32x32x16_f16 per tile (K = 32), the same two rank-1 scale MFMAs and 32 fmas,
// no conversions (operands already f16: the int8 -> f16 unpack it would also need is
// not counted); 4: variant 3 with the shared A operand unpacked from the 16 int8 a lane
// holds (byte ^ 0x80 placed under an 0x64 high byte is the f16 1152 + q, so a v_perm_b32
// and a packed f16 add of -1152 give two exact values), as a kernel reading int8
// weights from LDS would need; the B operand is taken as already f16
template <int VARIANT>
__global__ __launch_bounds__(PROBE_THREADS, 2) void block_mix_kernel(int iters, int seed, float* __restrict__ out) {
    const int lane = threadIdx.x % WAVE;
    float acc0[16], acc1[16];
    for (int v = 0; v < 16; v++) {
        acc0[v] = 0.0f;
        acc1[v] = 0.0f;
    }
    v4i_p A0 = {lane, seed, 3, 4}, A1 = {5, 6, seed, 7}, B = {1, 2, seed, 5};
    v8h_p xa = {}, xb = {};
    xb[0] = (_Float16)(float)(seed & 7);
    const v16i_p zi = {};
    const v16f_p zf = {};
    v16i_p S0 = zi, S1 = zi;
    v16f_p C0 = zf, C1 = zf;
    const v2h_p f16_bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    if (VARIANT == 2)
        for (int v = 0; v < 16; v++) {
            S0[v] = v * seed + lane;
            S1[v] = v + seed;
            C0[v] = 0.01f * (float)(v + seed);
            C1[v] = 0.02f * (float)v;
        }
    for (int it = 0; it < iters; it++) {
        xa[0] = (_Float16)(float)(it & 7);
        A0.x += 1;
        if (VARIANT == 0) {
            S0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A0, B, zi, 0, 0, 0);
            S1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A1, B, zi, 0, 0, 0);
            C0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa, xb, zf, 0, 0, 0);
            C1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(xb, xa, zf, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                acc0[v] = fmaf((float)S0[v], C0[v], acc0[v]);
                acc1[v] = fmaf((float)S1[v], C1[v], acc1[v]);
            }
        } else if (VARIANT == 3 || VARIANT == 4) {
            // four distinct products, each varying per iteration, so none is hoisted or merged
            v8h_p xc = xb;
            xc[1] = (_Float16)(float)(it & 3);
            v8h_p a_lo = xa, a_hi = xc;
            if (VARIANT == 4) {
                A0.y += 5;
                A0.z ^= it;
                A0.w += 3;
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    const uint32_t x = (uint32_t)A0[d] ^ 0x80808080u;
                    const v2h_p lo = __builtin_bit_cast(v2h_p, __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u)) + f16_bias;
                    const v2h_p hi = __builtin_bit_cast(v2h_p, __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u)) + f16_bias;
                    v8h_p& a = d < 2 ? a_lo : a_hi;
                    a[4 * (d & 1)] = lo[0];
                    a[4 * (d & 1) + 1] = lo[1];
                    a[4 * (d & 1) + 2] = hi[0];
                    a[4 * (d & 1) + 3] = hi[1];
                }
            }
            const v16f_p D0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                a_hi, xa, __builtin_amdgcn_mfma_f32_32x32x16_f16(a_lo, xc, zf, 0, 0, 0), 0, 0, 0);
            const v16f_p D1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                a_hi, xc, __builtin_amdgcn_mfma_f32_32x32x16_f16(a_lo, xa, zf, 0, 0, 0), 0, 0, 0);
            C0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa, xb, zf, 0, 0, 0);
            C1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(xb, xa, zf, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                acc0[v] = fmaf(D0[v], C0[v], acc0[v]);
                acc1[v] = fmaf(D1[v], C1[v], acc1[v]);
            }
        } else if (VARIANT == 1) {
            // chained through the accumulators so that nothing is hoisted
            S0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A0, B, S0, 0, 0, 0);
            S1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A1, B, S1, 0, 0, 0);
            C0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa, xb, C0, 0, 0, 0);
            C1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(xb, xa, C1, 0, 0, 0);
        } else {
            // the 64 vector ops; the integer sources change per iteration (32 more adds)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                S0[v] += 3;
                S1[v] += 5;
                acc0[v] = fmaf((float)S0[v], C0[v], acc0[v]);
                acc1[v] = fmaf((float)S1[v], C1[v], acc1[v]);
            }
        }
    }
    float r = 0.0f;
    for (int v = 0; v < 16; v++) r += acc0[v] + acc1[v] + (float)S0[v] + (float)S1[v] + C0[v] + C1[v];
    out[(size_t)blockIdx.x * PROBE_THREADS + threadIdx.x] = r;
}

// ---- read-rate probes (the decode GEMV's streams) ------------------------------
// Variant 0: one wave per work group streams its own contiguous range with 16-byte
// global->LDS copies into a private 3-step ring of 8 KB steps (8 copies of 1 KB per
// step, two steps in flight), as the decode GEMV streams one 64-row group of an
// expert; it reads back one word per step so every step is consumed.  Variant 1: a
// grid-stride 16-byte vector read of the same bytes into registers.  Variant 2:
// variant 0 with the copies' non-temporal cache policy (as the decode GEMV streams).
constexpr int STREAM_STEP = 8192, STREAM_RING = 3;

template <bool NT>
__global__ __launch_bounds__(WAVE) void stream_dma_kernel(const uint8_t* __restrict__ base, uint32_t steps,
                                                          float* __restrict__ out) {
    __shared__ __align__(16) uint8_t ring[STREAM_RING][STREAM_STEP];
    const int lane = threadIdx.x;
    const uint8_t* src = base + (size_t)blockIdx.x * steps * STREAM_STEP + 16u * lane;
    auto issue = [&](uint32_t st) {
        uint8_t* dst = ring[st % STREAM_RING];
#pragma unroll
        for (int c = 0; c < STREAM_STEP / 1024; c++) {
            if (NT)
                g2l16_nt(src + (size_t)st * STREAM_STEP + c * 1024, dst + c * 1024);
            else
                g2l16(src + (size_t)st * STREAM_STEP + c * 1024, dst + c * 1024);
        }
    };
    constexpr int LOADS = STREAM_STEP / 1024;
    for (uint32_t i = 0; i < STREAM_RING - 1 && i < steps; i++) issue(i);
    uint32_t acc = 0;
    for (uint32_t st = 0; st < steps; st++) {
        if (st + 1 < steps)
            MM_WAIT_VM_LGKM(LOADS);   // step st landed, step st + 1 may stay in flight
        else
            MM_WAIT_VM_LGKM(0);
        uint32_t w = lds_b32(ring[st % STREAM_RING] + 4 * lane);
        lds_wait();
        lds_pin(w);  // the read's register stays live until its wait
        acc += w;
        // every lane has read its word of slot st before the refill of that slot
        if (st + STREAM_RING - 1 < steps) issue(st + STREAM_RING - 1);
    }
    out[(size_t)blockIdx.x * WAVE + lane] = (float)acc;
}

__global__ __launch_bounds__(256) void stream_vec_kernel(const int4* __restrict__ p, size_t n16,
                                                         float* __restrict__ out) {
    const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x, nth = (size_t)gridDim.x * 256;
    int a = 0;
    for (size_t i = tid; i < n16; i += nth) {
        const int4 v = p[i];
        a ^= v.x + v.y + v.z + v.w;
    }
    out[tid] = (float)a;
}

// Variant 3: copy throughput from a window small enough to stay in L2 (the grouped
// GEMM's operand copies hit L2 for most of their bytes): every wave of a 4-wave work
// group issues batches of 8 one-KB global -> LDS copies of chunks (c + d) & mask of the
// window (mask + 1 KB, a power of two) into its own 8 KB of LDS and waits for them.
constexpr int L2W_BATCH = 8;

__global__ __launch_bounds__(256) void l2_window_kernel(const uint8_t* __restrict__ base, uint32_t mask, uint32_t iters,
                                                        float* __restrict__ out) {
    __shared__ __align__(16) uint8_t lds[4][L2W_BATCH * 1024];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const uint32_t wid = blockIdx.x * 4 + wave;
    uint32_t c = wid * 7919u;
    for (uint32_t it = 0; it < iters; it++) {
#pragma unroll
        for (int d = 0; d < L2W_BATCH; d++)
            g2l16(base + (size_t)((c + d) & mask) * 1024 + 16 * lane, lds[wave] + d * 1024);
        MM_WAIT_VM_LGKM(0);
        c += L2W_BATCH;
    }
    // a plain LDS load: the compiler waits for it before the value is used (the copies
    // landed at the last batch's vmcnt wait)
    out[(size_t)wid * WAVE + lane] = (float)reinterpret_cast<const uint32_t*>(lds[wave])[lane];
}

}  // namespace

static hipError_t launch_probe_l2(const void* buf, size_t bytes, int work_groups, uint32_t iters, float* out,
                                  hipStream_t s) {
    hipLaunchKernelGGL(l2_window_kernel, dim3((unsigned)work_groups), dim3(256), 0, s,
                       static_cast<const uint8_t*>(buf), (uint32_t)(bytes / 1024 - 1), iters, out);
    return hipGetLastError();
}

static hipError_t launch_probe_stream(int variant, const void* buf, size_t bytes, int waves, float* out, hipStream_t s) {
    if (variant == 0 || variant == 2) {
        const uint32_t steps = (uint32_t)(bytes / ((size_t)waves * STREAM_STEP));
        if (variant == 2)
            hipLaunchKernelGGL(stream_dma_kernel<true>, dim3((unsigned)waves), dim3(WAVE), 0, s,
                               static_cast<const uint8_t*>(buf), steps, out);
        else
            hipLaunchKernelGGL(stream_dma_kernel<false>, dim3((unsigned)waves), dim3(WAVE), 0, s,
                               static_cast<const uint8_t*>(buf), steps, out);
    } else {
        hipLaunchKernelGGL(stream_vec_kernel, dim3((unsigned)(waves * WAVE / 256)), dim3(256), 0, s,
                           static_cast<const int4*>(buf), bytes / 16, out);
    }
    return hipGetLastError();
}

static hipError_t launch_probe_block_mix(int variant, int work_groups, int iters, int seed, float* out, hipStream_t s) {
    const dim3 grid((unsigned)work_groups), blk(PROBE_THREADS);
    if (variant == 1)
        hipLaunchKernelGGL(block_mix_kernel<1>, grid, blk, 0, s, iters, seed, out);
    else if (variant == 2)
        hipLaunchKernelGGL(block_mix_kernel<2>, grid, blk, 0, s, iters, seed, out);
    else if (variant == 3)
        hipLaunchKernelGGL(block_mix_kernel<3>, grid, blk, 0, s, iters, seed, out);
    else if (variant == 4)
        hipLaunchKernelGGL(block_mix_kernel<4>, grid, blk, 0, s, iters, seed, out);
    else
        hipLaunchKernelGGL(block_mix_kernel<0>, grid, blk, 0, s, iters, seed, out);
    return hipGetLastError();
}

}  // namespace hy

// ---- C entry points (bench.py loads libhy_probe.so; nothing in libhy_moe.so calls these)

static thread_local char g_probe_err[256];

static int probe_fail(const char* msg) {
    snprintf(g_probe_err, sizeof g_probe_err, "%s", msg);
    return -1;
}

static int probe_hip(hipError_t e) {
    if (e == hipSuccess) return 0;
    snprintf(g_probe_err, sizeof g_probe_err, "HIP error: %s", hipGetErrorString(e));
    return -1;
}

extern "C" {

const char* hyp_last_error(void) { return g_probe_err; }

int hyp_block_mix(int32_t variant, uint32_t work_groups, uint32_t iters, float* out_dev, void* stream) {
    if (!out_dev || work_groups == 0 || iters == 0 || variant < 0 || variant > 4)
        return probe_fail("bad block-mix probe arguments (variant 0-4, work groups and iterations > 0)");
    return probe_hip(hy::launch_probe_block_mix(variant, (int)work_groups, (int)iters, 3, out_dev,
                                                static_cast<hipStream_t>(stream)));
}

int hyp_stream(int32_t variant, const void* buf_dev, uint64_t bytes, uint32_t waves, float* out_dev, void* stream) {
    const uint64_t per = (uint64_t)waves * hy::STREAM_STEP;
    if (!buf_dev || !out_dev || waves == 0 || variant < 0 || variant > 2 || bytes == 0 || bytes % per ||
        (variant == 1 && waves % 4))
        return probe_fail("bad stream probe arguments: bytes a multiple of waves x 8192, waves a multiple of 4 "
                          "for variant 1, variant 0-2");
    return probe_hip(hy::launch_probe_stream(variant, buf_dev, (size_t)bytes, (int)waves, out_dev,
                                             static_cast<hipStream_t>(stream)));
}

int hyp_l2_window(const void* buf_dev, uint64_t bytes, uint32_t work_groups, uint32_t iters, float* out_dev,
                  void* stream) {
    const uint64_t kb = bytes / 1024;
    if (!buf_dev || !out_dev || work_groups == 0 || iters == 0 || bytes % 1024 || kb == 0 || (kb & (kb - 1)) ||
        kb > (1u << 31))
        return probe_fail("bad L2 window probe arguments: bytes a power-of-two number of KB, work groups and "
                          "iterations > 0 (out holds work_groups x 256 floats)");
    return probe_hip(hy::launch_probe_l2(buf_dev, (size_t)bytes, (int)work_groups, iters, out_dev,
                                         static_cast<hipStream_t>(stream)));
}

}  // extern "C"
