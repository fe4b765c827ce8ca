// Device helpers of the kernels that stream KV pages through LDS with
// direct global->LDS loads (ring.hip, prefill.hip).
#pragma once
#include "common.hpp"

#include <cstdint>
#include <type_traits>

namespace rs {

// s_waitcnt vmcnt(N) leaving the other counters alone (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// A 16-byte global load that the compiler does not track: the kernel's own
// vmcnt waits cover it.  (Loads complete in order, so an untracked load never
// weakens a wait the compiler places for its own loads.)  Every use of the
// result must depend on an asm statement placed after that wait (pin() of
// the value, or an LDS wait whose result the use also takes), so that the
// compiler cannot move the use above the wait.
template <typename V>
__device__ __forceinline__ void global_load16(V &v, const void *p) {
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
}

// A 4-byte global load that the compiler does not track (like
// global_load16), and a 2- or 4-byte LDS write that it does not order
// against the rings' direct loads (like lds_read); both are awaited
// explicitly.
__device__ __forceinline__ void global_load4(float &v, const float *p) {
    asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(p) : "memory");
}
__device__ __forceinline__ void lds_write4(uint32_t addr, float v) {
    asm volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_write2(uint32_t addr, _Float16 v) {
    const unsigned u = __builtin_bit_cast(unsigned short, v);
    asm volatile("ds_write_b16 %0, %1" : : "v"(addr), "v"(u) : "memory");
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// LDS reads of page fragments at addr + OFF, issued as written.  They bypass
// the compiler's own wait insertion, which cannot tell the ring buffers'
// direct loads apart for every buffer and would drain the whole ring before
// some reads; their completion is awaited explicitly with lds_wait.
template <int OFF, typename V>
__device__ __forceinline__ void lds_read(V &v, uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds_read offset range");
    if constexpr (sizeof(V) == 16)
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    else
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
}
// LDS reads in flight are counted by lgkmcnt, a 4-bit counter: a wave never
// has more than 15 of them outstanding, so every wait count below is exact.
constexpr int kMaxLdsInFlight = 15;

// s_waitcnt lgkmcnt(N), after which v (read by lds_read) may be used.
template <int N, typename V>
__device__ __forceinline__ void lds_wait(V &v) {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "i"(N));
}
// The same for two reads, a and b, with one wait.
template <int N, typename V>
__device__ __forceinline__ void lds_wait(V &a, V &b) {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}

// Values v are computed (or loaded) before this point: an empty statement,
// ordered with the explicit LDS and memory waits around it, that takes them
// as operands, so their uses are not moved above it.
template <typename T>
__device__ __forceinline__ void pin1(T &v) {
    asm volatile("" : "+v"(v));
}
template <typename... T>
__device__ __forceinline__ void pin(T &...v) {
    (pin1(v), ...);
}

// Marks a rarely taken branch body as having side effects, so the compiler
// keeps the branch instead of executing the body on every page as selects.
__device__ __forceinline__ void keep_branch() { asm volatile(""); }

// Workgroup barrier for the page ring.  A workgroup-scope fence would also
// wait for every direct global->LDS load in flight (they count as LDS
// writes), draining the ring; instead each wave waits explicitly for the
// loads and LDS reads that the barrier hands over, and the empty asm
// statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void ring_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Maximum (sum) over the four 16-lane rows of the wave: lanes l, l^16, l^32
// and l^48, exchanged with the lane-swap instructions instead of LDS.
__device__ __forceinline__ float row_group_max(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float row_group_sum(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

}  // namespace rs
