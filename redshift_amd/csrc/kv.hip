// KV page maintenance: token-major <-> page conversion, and the fused prepare
// step (RMSNorm + RoPE of q and k, fp16 append of k and v into the pages).
#include "kernels.hpp"

#include <cmath>

namespace rs {
namespace {

// Elementwise move of 16-bit values between token-major rows
// [count][kv_heads][D] (token first+t at row t) and the page layout.
template <bool IS_V, bool TO_PAGES>
__global__ __launch_bounds__(256)
void convert_pages(unsigned short *pages, unsigned short *rows, int kv_heads, int D,
                   size_t head_stride, int first, size_t total) {
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (size_t)gridDim.x * blockDim.x) {
        const int d = (int)(e % D);
        const size_t th = e / D;
        const int h = (int)(th % kv_heads);
        const int token = first + (int)(th / kv_heads);
        const size_t off = (size_t)h * head_stride +
                           (IS_V ? v_page_offset(token, d, D) : k_page_offset(token, d, D));
        if (TO_PAGES) pages[off] = rows[e];
        else rows[e] = pages[off];
    }
}

template <bool TO_PAGES>
void convert(void *k_pages, void *v_pages, const void *k_rows, const void *v_rows,
             int kv_heads, int head_dim, int capacity, int first, int count,
             hipStream_t stream) {
    const size_t total = (size_t)count * kv_heads * head_dim;
    if (!total) return;
    const size_t stride = (size_t)capacity * head_dim;
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 65536);
    if (k_pages && k_rows) {
        hipLaunchKernelGGL((convert_pages<false, TO_PAGES>), dim3(blocks), dim3(256), 0, stream,
                           static_cast<unsigned short *>(k_pages),
                           const_cast<unsigned short *>(static_cast<const unsigned short *>(k_rows)),
                           kv_heads, head_dim, stride, first, total);
        check(hipGetLastError());
    }
    if (v_pages && v_rows) {
        hipLaunchKernelGGL((convert_pages<true, TO_PAGES>), dim3(blocks), dim3(256), 0, stream,
                           static_cast<unsigned short *>(v_pages),
                           const_cast<unsigned short *>(static_cast<const unsigned short *>(v_rows)),
                           kv_heads, head_dim, stride, first, total);
        check(hipGetLastError());
    }
}

// RoPE frequencies 1e7^(-i/32), i = 0..31 (base 1e7 over 64 rotary dims,
// qvelox/model.py:13), as doubles.
__constant__ double kRopeFreq[32] = {
    0x1.0000000000000p+0, 0x1.3566562253c7ep-1, 0x1.75f034d79e965p-2, 0x1.c3f06b4e265cep-3,
    0x1.111aedafb9a9dp-3, 0x1.4a12ad8379eb8p-4, 0x1.8eec7def5d56cp-5, 0x1.e222ec75094e2p-6,
    0x1.235a71c5ee5ccp-6, 0x1.6020a364b1284p-7, 0x1.a99428b3d26b3p-8, 0x1.012cfaad0da13p-8,
    0x1.36d219065ac0cp-9, 0x1.77a7d87ee61b0p-10, 0x1.c603c39630446p-11, 0x1.125c04ab2d71fp-11,
    0x1.4b96be9c2da2cp-12, 0x1.90c181b38fe22p-13, 0x1.e459c57e28a47p-14, 0x1.24b0fd0e890d4p-14,
    0x1.61bea2721385fp-15, 0x1.ab88830de4ad5p-16, 0x1.025b57369650bp-16, 0x1.383f8796f72a9p-17,
    0x1.7961810874a9fp-18, 0x1.c8198c91f9fccp-19, 0x1.139e9527f964ep-19, 0x1.4d1c97f4e952fp-20,
    0x1.9298ace36f12ep-21, 0x1.e69338f8adcd3p-22, 0x1.26091b11c8665p-22, 0x1.635e883bbc816p-23,
};

// One workgroup per (head, token): heads 0..23 are query heads, 24..27 the KV
// heads (the reference's attn_prepare grid, src/kernels.cu:416-434).
// RMSNorm over 256 dims with gamma, then rotate pairs (i, i+32), i < 32, by
// (position+t) * 1e7^(-i/32).  The angle is evaluated and reduced to
// [-pi, pi] in double precision (the reference rounds the angle to fp32,
// which at position 139,263 is off by up to 2^-7 rad); its sine and cosine
// and the rotation are fp32.  Every global load is issued first and the
// angle computed while they are in flight; the pairs (i, i+32) sit in wave
// 0, which swaps them with a lane shuffle, so one barrier (the norm's
// cross-wave sum) remains.
__global__ __launch_bounds__(256)
void prepare_kernel(_Float16 *q_hilo, _Float16 *k_pages, _Float16 *v_pages, const float *q_gate,
                    const float *key, const float *value, const float *q_norm,
                    const float *k_norm, int position, size_t head_stride, float epsilon) {
    constexpr int D = kModelHeadDim, H = kModelQHeads, HKV = kModelKvHeads;
    static_assert(D == 4 * kWave, "four waves of one dim each");
    const int h = blockIdx.x, t = blockIdx.y, i = threadIdx.x;
    const bool is_q = h < H;
    const int kh = h - H;
    const float *src = is_q ? q_gate + ((size_t)t * H + h) * 2 * D : key + ((size_t)t * HKV + kh) * D;
    const float x = src[i];
    const float gamma = (is_q ? q_norm : k_norm)[i];
    const float v = is_q ? 0.f : value[((size_t)t * HKV + kh) * D + i];
    float c = 1.f, sn = 0.f;
    if (i < 32) {
        constexpr double kTwoPi = 6.283185307179586476925286766559;
        const double theta = (double)(position + t) * kRopeFreq[i];
        const double r = theta - kTwoPi * rint(theta * (1.0 / kTwoPi));
        sincosf((float)r, &sn, &c);
    }
    __shared__ float red[D / kWave];
    const float ss = wave_sum(x * x);
    if ((i & (kWave - 1)) == 0) red[i / kWave] = ss;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < D / kWave; ++w) total += red[w];
    const float inv = rsqrtf(total / D + epsilon);
    float y = x * inv * gamma;
    // Lane i < 32 of wave 0 holds a = y_i, lane i + 32 holds b = y_{i+32}.
    const float other = __shfl_xor(y, 32, kWave);
    if (i < 32) y = y * c - other * sn;                      // a c - b s
    const float cs = __shfl_xor(c, 32, kWave), ss2 = __shfl_xor(sn, 32, kWave);
    if (i >= 32 && i < 64) y = other * ss2 + y * cs;         // a s + b c
    if (is_q) {
        const size_t idx = ((size_t)t * H + h) * D + i;
        const _Float16 hi = (_Float16)y;
        q_hilo[idx] = hi;
        q_hilo[(size_t)gridDim.y * H * D + idx] = (_Float16)(y - (float)hi);
    } else {
        const int token = position + t;
        k_pages[(size_t)kh * head_stride + k_page_offset(token, i, D)] = (_Float16)y;
        v_pages[(size_t)kh * head_stride + v_page_offset(token, i, D)] = (_Float16)v;
    }
}

// Copy of whole pages: for every KV head, elements [0, n) of its run (the
// pages of tokens 0 .. n/D-1) from a cache of stride src_stride to one of
// stride dst_stride, 16 bytes per lane.
__global__ __launch_bounds__(256)
void copy_pages(uint4 *dst, const uint4 *src, size_t dst_stride, size_t src_stride, size_t n,
                int kv_heads) {
    const size_t per_head = n / 8;   // uint4 per head
    const size_t total = per_head * kv_heads;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (size_t)gridDim.x * blockDim.x) {
        const size_t h = e / per_head, i = e - h * per_head;
        dst[h * (dst_stride / 8) + i] = src[h * (src_stride / 8) + i];
    }
}

}  // namespace

void launch_copy(void *dst_k, void *dst_v, const void *src_k, const void *src_v, int kv_heads,
                 int head_dim, int dst_capacity, int src_capacity, int pages, hipStream_t stream) {
    const size_t n = (size_t)pages * kPageTokens * head_dim;   // 16-bit elements per head
    if (!n) return;
    const size_t total = n / 8 * kv_heads;
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 4096);
    const size_t ds = (size_t)dst_capacity * head_dim, ss = (size_t)src_capacity * head_dim;
    hipLaunchKernelGGL(copy_pages, dim3(blocks), dim3(256), 0, stream, static_cast<uint4 *>(dst_k),
                       static_cast<const uint4 *>(src_k), ds, ss, n, kv_heads);
    check(hipGetLastError());
    hipLaunchKernelGGL(copy_pages, dim3(blocks), dim3(256), 0, stream, static_cast<uint4 *>(dst_v),
                       static_cast<const uint4 *>(src_v), ds, ss, n, kv_heads);
    check(hipGetLastError());
}

void launch_pack(void *k_pages, void *v_pages, const void *k_rows, const void *v_rows,
                 int kv_heads, int head_dim, int capacity, int first, int count,
                 hipStream_t stream) {
    convert<true>(k_pages, v_pages, k_rows, v_rows, kv_heads, head_dim, capacity, first, count, stream);
}

void launch_unpack(void *k_rows, void *v_rows, const void *k_pages, const void *v_pages,
                   int kv_heads, int head_dim, int capacity, int first, int count,
                   hipStream_t stream) {
    convert<false>(const_cast<void *>(k_pages), const_cast<void *>(v_pages), k_rows, v_rows,
                   kv_heads, head_dim, capacity, first, count, stream);
}

void launch_prepare(void *q_hilo, void *k_pages, void *v_pages, const float *q_gate,
                    const float *key, const float *value, const float *q_norm,
                    const float *k_norm, int batch, int position, int capacity,
                    float epsilon, hipStream_t stream) {
    hipLaunchKernelGGL(prepare_kernel, dim3(kModelQHeads + kModelKvHeads, batch),
                       dim3(kModelHeadDim), 0, stream, static_cast<_Float16 *>(q_hilo),
                       static_cast<_Float16 *>(k_pages),
                       static_cast<_Float16 *>(v_pages), q_gate, key, value, q_norm, k_norm,
                       position, (size_t)capacity * kModelHeadDim, epsilon);
    check(hipGetLastError());
}

}  // namespace rs
