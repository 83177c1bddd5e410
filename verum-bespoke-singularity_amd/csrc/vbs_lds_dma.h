// vbs_lds_dma.h — loads that the compiler does not track, for kernels that
// keep many loads in flight and wait for them one by one: 16-byte LDS DMA
// (global_load_lds_dwordx4) and plain vector loads issued from inline
// assembly, explicit vmcnt waits, and a compile-time loop to count them.
//
// Vector memory loads of a wave complete in issue order, so "every load
// issued before the last N has landed" is s_waitcnt vmcnt(N), with N counted
// at compile time. The compiler sees none of these loads: it inserts no wait
// for them, so every consumer first waits explicitly and (for register loads)
// passes the destination through an empty asm that ties it to the wait.
#pragma once

#include <stdint.h>

#include <type_traits>

#include <hip/hip_runtime.h>

namespace vbs {

// 16 bytes per lane from g to LDS at lds + 16 lane (lds wave-uniform: it is
// passed in M0; nothing else in the kernels that use this touches M0).
__device__ __forceinline__ void dma16(const void *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g),
                 "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}
// The same from base + off: base wave-uniform (a scalar register pair), off a
// 32-bit byte offset per lane, so no 64-bit address is formed per lane.
__device__ __forceinline__ void dma16s(const void *base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base),
                 "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}
// 4 bytes per lane from g to LDS at lds + 4 lane (lds wave-uniform, in M0).
__device__ __forceinline__ void dma4(const void *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g),
                 "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}
template <uint32_t N>
__device__ __forceinline__ void vmcnt_le() {  // vmcnt <= N, other counters untouched
    static_assert(N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15u) | ((N >> 4) << 14) | (7u << 4) | (15u << 8));
}

// f(std::integral_constant<uint32_t, i>) for i = I .. N - 1, unrolled.
template <uint32_t I, uint32_t N, class F>
__device__ __forceinline__ void unroll_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<uint32_t, I>{});
        unroll_for<I + 1u, N>(f);
    }
}

// Compute units of the current device (host side; 256 if the query fails).
inline uint32_t device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
    }
    return (uint32_t)cus;
}

}  // namespace vbs
