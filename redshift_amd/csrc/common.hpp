// Shared definitions for libredshift_hip: vector types for the gfx950 MFMA
// operands, the KV page layout, and host-side error plumbing.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>

namespace rs {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;
// The reference's fixed model attention (src/runtime.h:38-41).
constexpr int kModelQHeads = 24, kModelKvHeads = 4, kModelHeadDim = 256;
constexpr int kModelCapacity = 139264;  // src/runtime.cu:174

// ---------------------------------------------------------------------------
// KV page layout.
//
// Each KV head owns a contiguous run of pages ("head-major"): head h starts at
// element h * capacity * D, capacity being a multiple of kPageTokens.  A page
// holds 32 consecutive tokens (32 * D 16-bit elements) arranged in the exact
// register order of the gfx950 16x16x32 MFMA operands, so the attention
// kernels fetch every operand with one fully coalesced 16-byte load per lane
// (1 KiB per wave instruction) and no LDS staging.
//
// K page: two tiles of 16 tokens.  Tile element (token r, dim d) sits at
//   tile * 16*D + (d / 8) * 128 + r * 8 + d % 8
// so that for k-step ks (dims 32*ks .. 32*ks+31) lane l of a wave reads the 8
// dims 32*ks + 8*(l/16) .. +7 of token l%16 at offset 512*ks + 8*l: the A
// operand of S^T = K * Q^T (rows = keys, k = head dims).
//
// V page: D/16 dim-tiles of [4 key groups][16 dims][8 slots].  Slot j of group
// g holds token tau(g, j) = (j < 4 ? 4g + j : 16 + 4g + j - 4), so the V^T
// operand of O^T = V^T * P^T (rows = dims, k = keys) for lane l pairs with the
// P values that lane l already holds in the C layout of the two S^T tiles
// (keys 4*(l/16)+r of tile 0 and of tile 1).  Element (token p, dim d):
//   (d / 16) * 512 + ((p / 4) % 4) * 128 + (d % 16) * 8 + (p / 16) * 4 + p % 4
// ---------------------------------------------------------------------------
constexpr int kPageTokens = 32;

__host__ __device__ inline size_t k_page_offset(int token, int d, int D) {
    const size_t page = (size_t)(token >> 5);
    const int p = token & 31, tile = p >> 4, r = p & 15;
    return page * 32 * D + (size_t)tile * 16 * D + (size_t)(d >> 3) * 128 + r * 8 + (d & 7);
}

__host__ __device__ inline size_t v_page_offset(int token, int d, int D) {
    const size_t page = (size_t)(token >> 5);
    const int p = token & 31, a = p >> 4, g = (p >> 2) & 3, i = p & 3;
    return page * 32 * D + (size_t)(d >> 4) * 512 + g * 128 + (d & 15) * 8 + a * 4 + i;
}

// ---------------------------------------------------------------------------
// Host-side errors: every C-ABI entry point catches these and returns -1.
// ---------------------------------------------------------------------------
inline void require(bool condition, const char *message) {
    if (!condition) throw std::invalid_argument(message);
}

inline void check(hipError_t result) {
    if (result != hipSuccess) throw std::runtime_error(hipGetErrorString(result));
}

// Device wave helpers ---------------------------------------------------------

// Workgroup barrier that orders LDS only.  __syncthreads() is a workgroup
// release/acquire fence over all address spaces, which makes every wave wait
// for its outstanding global loads (vmcnt 0) at each barrier and so drains any
// prefetch in flight; this one waits for LDS traffic (lgkmcnt 0) alone.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace rs
