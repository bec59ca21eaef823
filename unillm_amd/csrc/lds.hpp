// lds.hpp -- direct global -> LDS loads and compiler-opaque LDS reads (gfx950).
//
// The compiler inserts a wait for every direct (global -> LDS) load in flight
// before any LDS read it can see, which would drain a multi-stage ring.  Kernels
// that keep several stages in flight therefore read LDS through these inline-asm
// helpers and wait explicitly (lgkmcnt for the reads, vmcnt in issue order for
// the direct loads, then a bare s_barrier).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace unillm {

typedef uint32_t lds_u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t lds_u32x4 __attribute__((ext_vector_type(4)));

// Calls f(integral_constant<int, I>) for I = 0 .. N - 1 (compile-time indices).
template <int N, class F, int... I>
__device__ __forceinline__ void constexpr_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void constexpr_for(F&& f) {
    constexpr_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

typedef __attribute__((address_space(3))) void* lds_ptr;
typedef const __attribute__((address_space(1))) void* gbl_ptr;

// global_load_lds_dwordx4 / _dword: lane i's bytes land at lds + i * size.
__device__ __forceinline__ void dma16(const void* g, uint8_t* l) {
    __builtin_amdgcn_global_load_lds((gbl_ptr)g, (lds_ptr)l, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, uint8_t* l) {
    __builtin_amdgcn_global_load_lds((gbl_ptr)g, (lds_ptr)l, 4, 0, 0);
}

// LDS reads the compiler does not see (so it adds no wait for the direct loads
// before them).  The caller waits with s_waitcnt lgkmcnt before use.
template <int OFF>
__device__ __forceinline__ lds_u32x4 lds_read128(uint32_t addr) {
    lds_u32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
template <int OFF>
__device__ __forceinline__ lds_u32x2 lds_read64(uint32_t addr) {
    lds_u32x2 v;
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_read32(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_read_u16(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_u16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}

// s_waitcnt with only vmcnt = n (gfx950: vmcnt in bits 3:0 and 15:14; expcnt 6:4
// and lgkmcnt 11:8 at their maxima, i.e. no wait on them).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | (((N >> 4) & 3) << 14));
}

}  // namespace unillm
