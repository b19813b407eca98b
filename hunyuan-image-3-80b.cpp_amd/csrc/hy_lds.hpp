// hy_lds.hpp -- global->LDS DMA (flat addresses, or buffer descriptors with scalar
// offsets) and explicitly waited LDS reads, shared by the kernels that stream operands
// through LDS rings (grouped MFMA GEMM, decode GEMV).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace hy {

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

// 16-byte global -> LDS copy (global_load_lds_dwordx4): lane i of the wave writes
// lds_wave_base + 16*i.  The wave's loads are tracked by vmcnt, not by barriers.
__device__ __forceinline__ void g2l16(const void* g, void* lds_wave_base) {
    __builtin_amdgcn_global_load_lds(g, lds_wave_base, 16, 0, 0);
}
// The same copy with the non-temporal cache policy (gfx950 cpol bits: sc0 = 1, nt = 2,
// sc1 = 16), for streams read once per launch: decode weight streams read 9-10 %
// faster with it (a 127 MB read by 864 single-wave streams: 23.1 against 25.3 us).
constexpr int HY_CPOL_NT = 2;
__device__ __forceinline__ void g2l16_nt(const void* g, void* lds_wave_base) {
    __builtin_amdgcn_global_load_lds(g, lds_wave_base, 16, 0, HY_CPOL_NT);
}
// Buffer descriptor of a wave-uniform base with no range limit (raw buffer, stride 0,
// the gfx9 format word 0x00020000).  Copies through it (b2l) take a 32-bit per-lane
// byte offset in a VGPR and a wave-uniform byte offset in an SGPR, so a loop that
// advances the uniform part does its address arithmetic in scalar registers.  The two
// offsets must sum below 2^32.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* uniform_base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(uniform_base), (short)0, (int)0xffffffff, 0x00020000);
}
// global -> LDS copy of BYTES (4 or 16) per lane: lane l's bytes at base + lane_off +
// s_off land at lds_wave_base + BYTES * l
template <int BYTES = 16>
__device__ __forceinline__ void b2l(__amdgpu_buffer_rsrc_t r, void* lds_wave_base, uint32_t lane_off,
                                    uint32_t s_off) {
    static_assert(BYTES == 4 || BYTES == 16, "4- or 16-byte copies");
    auto* l = (__attribute__((address_space(3))) void*)(lds_wave_base);
    if constexpr (BYTES == 4)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 4, lane_off, s_off, 0, 0);
    else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 16, lane_off, s_off, 0, 0);
}
// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8])
#define MM_WAIT_VM_LGKM(N) __builtin_amdgcn_s_waitcnt(((N) & 0xF) | (0x7 << 4) | (((N) >> 4) << 14))

// vmcnt wait for the ring stage about to be consumed: the R stages issued after it
// may stay in flight (R = min(RING - 2, stages left after it), LOADS copies per stage
// and wave; copies complete in issue order)
template <int LOADS, int R>
__device__ __forceinline__ void wait_copies(int left) {
    if constexpr (R == 0) {
        MM_WAIT_VM_LGKM(0);
    } else {
        if (left >= R) {
            MM_WAIT_VM_LGKM(R * LOADS);
        } else {
            wait_copies<LOADS, R - 1>(left);
        }
    }
}

// LDS reads of the ring are issued as plain ds_read instructions: the compiler does
// not associate them with the in-flight global->LDS copies (it would otherwise wait
// for every outstanding copy, including the stages being prefetched).  Their
// completion is waited for explicitly (lds_wait) before any result is used; the
// vmcnt wait + barrier at the top of each stage orders them after the copies.
typedef __attribute__((address_space(3))) const uint8_t lds_u8_t;
__device__ __forceinline__ uint32_t lds_off(const void* p) { return (uint32_t)(uintptr_t)((lds_u8_t*)p); }
__device__ __forceinline__ v4i_t lds_b128(const void* p) {
    v4i_t r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(lds_off(p)));
    return r;
}
__device__ __forceinline__ uint32_t lds_u16(const void* p) {
    uint32_t r;
    asm volatile("ds_read_u16 %0, %1" : "=v"(r) : "v"(lds_off(p)));
    return r;
}
__device__ __forceinline__ uint32_t lds_b32(const void* p) {
    uint32_t r;
    asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(lds_off(p)));
    return r;
}
__device__ __forceinline__ void lds_st128(void* p, v4i_t v) {
    asm volatile("ds_write_b128 %0, %1" ::"v"(lds_off(p)), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_st128_at(uint32_t off, v4i_t v) {
    asm volatile("ds_write_b128 %0, %1" ::"v"(off), "v"(v) : "memory");
}
// ds_write_b128 at base + a compile-time byte offset
template <int OFF>
__device__ __forceinline__ void lds_st128_at(uint32_t base, v4i_t v) {
    asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(base), "v"(v), "i"(OFF) : "memory");
}
__device__ __forceinline__ void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// wait until at most N of this wave's LDS reads are outstanding (they complete in
// order); pin each consumed result afterwards (lds_pin)
template <int N>
__device__ __forceinline__ void lds_wait_upto() {
    static_assert(N >= 0 && N <= 15, "lgkmcnt is 4 bits");
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory");
}
// After a bare lds_wait(): pin a ds_read result so none of its uses is scheduled above
// the wait (volatile asm statements keep their program order).
__device__ __forceinline__ void lds_pin(v4i_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void lds_pin(uint32_t& v) { asm volatile("" : "+v"(v)); }
// Force a value to be computed here (before any later volatile asm, e.g. the next
// round of ds_reads), which bounds how many loaded operands are live at once.
__device__ __forceinline__ void pin_f32(float& v) { asm volatile("" : "+v"(v)); }
// wait for the ds_reads whose results are passed in: the values are threaded through
// the asm so no consumer can be scheduled ahead of the wait
__device__ __forceinline__ void lds_wait(v4i_t& a) { asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a)::"memory"); }
__device__ __forceinline__ void lds_wait(v4i_t& a, v4i_t& b) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b)::"memory");
}
__device__ __forceinline__ void lds_wait(v4i_t& a, v4i_t& b, v4i_t& c) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c)::"memory");
}
__device__ __forceinline__ void lds_wait(v4i_t& a, v4i_t& b, uint32_t& c) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c)::"memory");
}
__device__ __forceinline__ void lds_wait(v4i_t& a, v4i_t& b, uint32_t& c, uint32_t& d) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d)::"memory");
}
__device__ __forceinline__ void lds_wait(v4i_t& a, v4i_t& b, v4i_t& c, uint32_t& d, uint32_t& e, uint32_t& f) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f)::"memory");
}
__device__ __forceinline__ void lds_wait(v4i_t& a, v4i_t& b, v4i_t& c, v4i_t& c2, uint32_t& d, uint32_t& e,
                                         uint32_t& f, uint32_t& f2) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(a), "+v"(b), "+v"(c), "+v"(c2), "+v"(d), "+v"(e), "+v"(f), "+v"(f2)::"memory");
}

// ds_read_b128 / b32 at base + a compile-time byte offset (no address arithmetic)
template <int OFF>
__device__ __forceinline__ v4i_t lds_b128_at(uint32_t base) {
    v4i_t r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(base), "i"(OFF));
    return r;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_b32_at(uint32_t base) {
    uint32_t r;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(base), "i"(OFF));
    return r;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_u16_at(uint32_t base) {
    uint32_t r;
    asm volatile("ds_read_u16 %0, %1 offset:%2" : "=v"(r) : "v"(base), "i"(OFF));
    return r;
}

}  // namespace hy
