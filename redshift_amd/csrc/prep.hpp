// The fused path's query/key preparation (the reference's attn_prepare,
// src/kernels.cu:416-434): RMSNorm over 256 dims with gamma, then RoPE on the
// pairs (i, i+32), i < 32, by the angle (position+t) * 1e7^(-i/32).  One
// wave prepares a row.
#pragma once
#include "kernels.hpp"

#include <cmath>

namespace rs {

// RoPE frequency of pair i: 1e7^(-i/32) (base 1e7 over 64 rotary dims,
// qvelox/model.py:13), in double precision.
__device__ __forceinline__ double rope_freq(int i) {
#pragma clang fp contract(off)
    constexpr double kLog2Base = 23.253496664211536;   // log2(1e7)
    return exp2(-(double)i * (kLog2Base / 32.0));
}

// cos and sin of the angle pos * freq (freq = rope_freq(i) of pair i).  The
// angle is evaluated and reduced to [-pi, pi] in double precision (the
// reference rounds it to fp32, which at position 139,263 is off by up to
// 2^-7 rad); the sine and cosine of the reduced angle are fp32.
__device__ __forceinline__ void rope_cos_sin(int pos, double freq, float &c, float &s) {
#pragma clang fp contract(off)
    constexpr double kTwoPi = 6.283185307179586476925286766559;
    const double theta = (double)pos * freq;
    const double r = theta - kTwoPi * rint(theta * (1.0 / kTwoPi));
    sincosf((float)r, &s, &c);
}

// The fp16 cache entry of an fp32 value, rounded as the reference rounds
// one (__float2half_rn of a float): the value is first held as fp32, so the
// compiler cannot fold the product that made it and the conversion into one
// mixed-precision FMA, which rounds once and differs in rare cases.
__device__ __forceinline__ _Float16 cache_half(float x) {
    asm volatile("" : "+v"(x));
    return (_Float16)x;
}

// Sum over the 64 lanes of a wave, the same in every lane: xor-1 and xor-2
// quad permutes, the half-row and row mirrors (within 16 lanes, all on
// DPP), then the 16-lane row groups exchanged with lane swaps.
template <int CTRL>
__device__ __forceinline__ float dpp_get(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum_dpp(float x) {
    x = (x + dpp_get<0xb1>(x));     // quad_perm [1,0,3,2]
    x = (x + dpp_get<0x4e>(x));     // quad_perm [2,3,0,1]
    x = (x + dpp_get<0x141>(x));    // row_half_mirror
    x = (x + dpp_get<0x140>(x));    // row_mirror
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = (__uint_as_float(a[0]) + __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return (__uint_as_float(b[0]) + __uint_as_float(b[1]));
}

// The value of x in lane l ^ 32 (a lane swap; {a0, a1} holds x and it).
__device__ __forceinline__ float lane_xor32(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(a[0] == __float_as_uint(x) ? a[1] : a[0]);
}

// RMSNorm (epsilon), gamma and RoPE of R 256-dim rows held by one wave, the
// rows' steps interleaved: lane l owns dims 64w + l in x[r][w] (gamma
// likewise); the rotated pairs (i, i+32) are lanes l and l ^ 32 of x[r][0].
// (c[r], s[r]) are rope_cos_sin(position of row r, rope_freq(l)) on lanes
// l < 32.  Every rounding step is explicit: contraction into fused
// multiply-adds is off here, since the compiler would otherwise pick which
// product to fuse per call site, and a K row appended to the cache must have
// the same bits whichever kernel instance prepared it.
template <int R>
__device__ __forceinline__ void norm_rope_rows(float (&x)[R][4], const float (&gamma)[4], const float (&c)[R],
                                               const float (&s)[R], float epsilon, int lane) {
#pragma clang fp contract(off)
    constexpr float kInvD = 1.f / (4 * kWave);
    float inv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float sq = (x[r][0] * x[r][0]);
#pragma unroll
        for (int w = 1; w < 4; ++w) sq = (sq + (x[r][w] * x[r][w]));
        inv[r] = sq;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) inv[r] = rsqrtf(wave_sum_dpp(inv[r]) * kInvD + epsilon);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int w = 0; w < 4; ++w) x[r][w] = ((x[r][w] * inv[r]) * gamma[w]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float other = lane_xor32(x[r][0]);
        const float cp = lane_xor32(c[r]), sp = lane_xor32(s[r]);
        x[r][0] = lane < 32 ? ((x[r][0] * c[r]) - (other * s[r]))    // a c - b s
                            : ((other * sp) + (x[r][0] * cp));    // a s + b c
    }
}

// The fused split kernels' new keys: the inputs of new token j's key for
// KV head h (its K row, the K gamma, its V row), lane l holding dims
// 64i + l like the prepare kernel; prepared (RMSNorm, gamma, RoPE with the
// angle's cosine and sine c, s on lanes < 32) and appended to the pages at
// position + j with the prepare kernel's functions and rounding, so the same
// bits.
struct NewKeyRow {
    float k[1][4], g[4], v[4];
};
__device__ __forceinline__ void load_new_key(NewKeyRow &r, const FusedToken &tok, int kv_heads, int h, int j,
                                             int lane) {
    const size_t row = ((size_t)j * kv_heads + h) * kModelHeadDim;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r.k[0][i] = tok.key[row + 64 * i + lane];
        r.g[i] = tok.k_norm[64 * i + lane];
        r.v[i] = tok.value[row + 64 * i + lane];
    }
}
__device__ __forceinline__ void append_new_key(NewKeyRow &r, const FusedToken &tok, int h, int j, float c,
                                               float s, int lane) {
    constexpr int D = kModelHeadDim;
    const float cr[1] = {c}, sr[1] = {s};
    norm_rope_rows<1>(r.k, r.g, cr, sr, tok.epsilon, lane);
    _Float16 *kp = static_cast<_Float16 *>(tok.k_pages) + (size_t)h * tok.head_stride;
    _Float16 *vp = static_cast<_Float16 *>(tok.v_pages) + (size_t)h * tok.head_stride;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        kp[k_page_offset(tok.position + j, 64 * i + lane, D)] = cache_half(r.k[0][i]);
        vp[v_page_offset(tok.position + j, 64 * i + lane, D)] = cache_half(r.v[i]);
    }
}

}  // namespace rs
