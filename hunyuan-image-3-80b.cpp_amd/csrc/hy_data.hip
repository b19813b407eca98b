// hy_data.hip -- weight residency kernels: GGUF block repack into the resident
// layout, on-device synthetic weight generation + quantization, dequantization.
#include "hy_device.hpp"
#include "hy_launch.hpp"
#include "hy_layout.hpp"

namespace hy {

// ggml's scalar quantize_row_q4_0 for one block (the signed value of largest
// magnitude maps to -8; element j -> low nibble of byte j, j+16 -> high nibble).
__device__ void quant_block_q4_0(const float* v, uint8_t* qs16, uint16_t* dh) {
    float amax = 0.0f, mx = 0.0f;
    for (int j = 0; j < QK; j++) {
        if (amax < fabsf(v[j])) {
            amax = fabsf(v[j]);
            mx = v[j];
        }
    }
    const float d = mx / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    *dh = f2h(d);
    for (int j = 0; j < QK / 2; j++) {
        int q0 = (int)(int8_t)(v[j] * id + 8.5f);
        int q1 = (int)(int8_t)(v[QK / 2 + j] * id + 8.5f);
        q0 = q0 > 15 ? 15 : q0;
        q1 = q1 > 15 ? 15 : q1;
        qs16[j] = (uint8_t)(q0 | (q1 << 4));
    }
}

// ggml's scalar quantize_row_q8_0 for one block, sequentially (same float ops as
// the lane-parallel version: amax is exact, then d, 1/d, roundf).
__device__ void quant_block_q8_0(const float* v, int8_t* qs32, uint16_t* dh) {
    float amax = 0.0f;
    for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    *dh = f2h(d);
    for (int j = 0; j < QK; j++) qs32[j] = (int8_t)__builtin_roundf(v[j] * id);
}

// Synthetic matrix of one expert: rows x cols ~ N(0,std) from stream key, element
// index r*cols+c, quantized per 32-block and stored at packed row perm(r) of the
// row-group-interleaved layout.
// One thread per block.
__global__ void synth_matrix_kernel(int wtype, uint64_t key, float scale, int rows, int cols, int gu_I,
                                    uint8_t* __restrict__ qs, uint16_t* __restrict__ sc) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int nb = cols / QK;
    if (idx >= (size_t)rows * nb) return;
    const int r = (int)(idx / nb), b = (int)(idx % nb);
    const int pr = gu_I > 0 ? gu_packed_row(r, gu_I) : r;
    float v[QK];
    for (int j = 0; j < QK; j++) v[j] = synth_normal(key, (uint64_t)r * cols + (uint64_t)b * QK + j, scale);
    uint8_t* dq = qs + il_q_offset(pr, b, nb, block_bytes(wtype));
    if (wtype == HY_TYPE_F32) {
        float* dst = reinterpret_cast<float*>(qs);
        for (int j = 0; j < QK; j++) dst[il_f32_offset(pr, b, nb, j)] = v[j];
    } else if (wtype == HY_TYPE_Q8_0) {
        quant_block_q8_0(v, reinterpret_cast<int8_t*>(dq), sc + il_s_offset(pr, b, nb));
    } else {
        quant_block_q4_0(v, dq, sc + il_s_offset(pr, b, nb));
    }
}

hipError_t launch_synth_matrix(int wtype, uint64_t key, float scale, int rows, int cols, int gu_I, uint8_t* qs,
                               uint16_t* sc, hipStream_t s) {
    const size_t n = (size_t)rows * (cols / QK);
    hipLaunchKernelGGL(synth_matrix_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, wtype, key, scale,
                       rows, cols, gu_I, qs, sc);
    return hipGetLastError();
}

__global__ void synth_fill_kernel(float* __restrict__ out, size_t n, uint64_t key, float scale) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < n) out[idx] = synth_normal(key, idx, scale);
}

hipError_t launch_synth_fill(float* out, size_t n, uint64_t key, float scale, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(synth_fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, n, key, scale);
    return hipGetLastError();
}

// GGUF rows (ggml layout, blocks of 34 / 18 bytes, or raw f32) -> resident
// row-group-interleaved layout.
__global__ void repack_kernel(int wtype, const uint8_t* __restrict__ src, int rows, int cols, int gu_I,
                              uint8_t* __restrict__ qs, uint16_t* __restrict__ sc) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int nb = cols / QK;
    if (idx >= (size_t)rows * nb) return;
    const int r = (int)(idx / nb), b = (int)(idx % nb);
    const int pr = gu_I > 0 ? gu_packed_row(r, gu_I) : r;
    uint8_t* dq = qs + il_q_offset(pr, b, nb, block_bytes(wtype));
    if (wtype == HY_TYPE_F32) {
        const float* s = reinterpret_cast<const float*>(src) + (size_t)r * cols + (size_t)b * QK;
        float* d = reinterpret_cast<float*>(qs);
        for (int j = 0; j < QK; j++) d[il_f32_offset(pr, b, nb, j)] = s[j];
    } else if (wtype == HY_TYPE_Q8_0) {
        const uint8_t* blk = src + ((size_t)r * nb + b) * 34;
        sc[il_s_offset(pr, b, nb)] = (uint16_t)(blk[0] | (blk[1] << 8));
        for (int j = 0; j < QK; j++) dq[j] = blk[2 + j];
    } else {
        const uint8_t* blk = src + ((size_t)r * nb + b) * 18;
        sc[il_s_offset(pr, b, nb)] = (uint16_t)(blk[0] | (blk[1] << 8));
        for (int j = 0; j < 16; j++) dq[j] = blk[2 + j];
    }
}

hipError_t launch_repack(int wtype, const uint8_t* src, int rows, int cols, int gu_I, uint8_t* qs, uint16_t* sc,
                         hipStream_t s) {
    const size_t n = (size_t)rows * (cols / QK);
    hipLaunchKernelGGL(repack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, wtype, src, rows, cols,
                       gu_I, qs, sc);
    return hipGetLastError();
}

// GGUF dequantization, one element per thread.
__global__ void dequant_kernel(int wtype, const uint8_t* __restrict__ src, size_t n, float* __restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const size_t b = idx / QK;
    const int j = (int)(idx % QK);
    if (wtype == HY_TYPE_Q8_0) {
        const uint8_t* blk = src + b * 34;
        out[idx] = (float)(int8_t)blk[2 + j] * h2f((uint16_t)(blk[0] | (blk[1] << 8)));
    } else if (wtype == HY_TYPE_Q4_0) {
        const uint8_t* blk = src + b * 18;
        const uint8_t byte = blk[2 + (j % 16)];
        const int nib = j < 16 ? (byte & 0x0f) : (byte >> 4);
        out[idx] = (float)(nib - 8) * h2f((uint16_t)(blk[0] | (blk[1] << 8)));
    } else {
        out[idx] = reinterpret_cast<const float*>(src)[idx];
    }
}

hipError_t launch_dequant(int wtype, const uint8_t* src, size_t n, float* out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, wtype, src, n, out);
    return hipGetLastError();
}

// Plain streaming copy: 16-byte vectors, grid-stride, tail bytes one by one.
__global__ void copy_kernel(const int4* __restrict__ src, int4* __restrict__ dst, size_t n16,
                            const uint8_t* __restrict__ src_tail, uint8_t* __restrict__ dst_tail, size_t ntail) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
    if (blockIdx.x == 0 && threadIdx.x < ntail) dst_tail[threadIdx.x] = src_tail[threadIdx.x];
}

hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t s) {
    if (bytes == 0) return hipSuccess;
    const size_t n16 = bytes / 16, ntail = bytes % 16;
    const int threads = 256;
    const size_t want = (n16 + threads - 1) / threads;
    const int blocks = (int)(want < 1 ? 1 : (want > 8192 ? 8192 : want));
    hipLaunchKernelGGL(copy_kernel, dim3(blocks), dim3(threads), 0, s, (const int4*)src, (int4*)dst, n16,
                       (const uint8_t*)src + n16 * 16, (uint8_t*)dst + n16 * 16, ntail);
    return hipGetLastError();
}

}  // namespace hy
