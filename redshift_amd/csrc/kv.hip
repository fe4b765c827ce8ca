// KV page maintenance: token-major <-> page conversion, and the fused prepare
// step (RMSNorm + RoPE of q and k, fp16 append of k and v into the pages).
#include "kernels.hpp"
#include "prep.hpp"

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

// One wave per (head, token): heads 0..23 are query heads, 24..27 the KV
// heads (the reference's attn_prepare grid, src/kernels.cu:416-434), lane l
// owning dims l, 64+l, 128+l, 192+l.  Every global load is issued first and
// the RoPE angle computed while they are in flight.
__global__ __launch_bounds__(kWave)
void prepare_kernel(_Float16 *q_hilo, _Float16 *k_pages, _Float16 *v_pages, const float *q_gate,
                    const float *key, const float *value, const float *q_norm,
                    const float *k_norm, int position, size_t head_stride, float epsilon, int head0) {
    constexpr int D = kModelHeadDim, H = kModelQHeads, HKV = kModelKvHeads;
    static_assert(D == 4 * kWave, "four dims per lane");
    const int h = head0 + blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const bool is_q = h < H;
    const int kh = h - H;
    const float *src = is_q ? q_gate + ((size_t)t * H + h) * 2 * D : key + ((size_t)t * HKV + kh) * D;
    const float *gamma_src = is_q ? q_norm : k_norm;
    float x[1][4], gamma[4], v[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        x[0][w] = src[64 * w + lane];
        gamma[w] = gamma_src[64 * w + lane];
        v[w] = is_q ? 0.f : value[((size_t)t * HKV + kh) * D + 64 * w + lane];
    }
    float c[1] = {1.f}, s[1] = {0.f};
    if (lane < 32) rope_cos_sin(position + t, rope_freq(lane), c[0], s[0]);
    norm_rope_rows(x, gamma, c, s, epsilon, lane);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const int d = 64 * w + lane;
        if (is_q) {
            const size_t idx = ((size_t)t * H + h) * D + d;
            const _Float16 hi = (_Float16)x[0][w];
            q_hilo[idx] = hi;
            q_hilo[(size_t)gridDim.y * H * D + idx] = (_Float16)(x[0][w] - (float)hi);
        } else {
            const int token = position + t;
            k_pages[(size_t)kh * head_stride + k_page_offset(token, d, D)] = cache_half(x[0][w]);
            v_pages[(size_t)kh * head_stride + v_page_offset(token, d, D)] = cache_half(v[w]);
        }
    }
}

// hi = fp16(q), lo = fp16(q - hi): q - hi is exact in fp32, so the two
// parts hold q to about 22 significant bits (|q| < 65504, error at most
// 2^-25 + 2^-22 |q| once lo falls into fp16's subnormal range).
__global__ __launch_bounds__(256)
void split_query(_Float16 *hi, _Float16 *lo, const float *q, size_t n) {
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (size_t)gridDim.x * blockDim.x) {
        const float x = q[e];
        const _Float16 h = (_Float16)x;
        hi[e] = h;
        lo[e] = (_Float16)(x - (float)h);
    }
}

// Copy of whole pages: for every KV head of K and of V, elements [0, n) of
// its run (the pages of tokens 0 .. n/D-1) from a cache of stride src_stride
// to one of stride dst_stride, both tensors in one launch (chunks of K's heads
// first, then V's).  Each thread moves kCopyUnroll 16-byte pieces of one
// head, all loads issued before the stores, non-temporal (every byte is
// touched once).  n is a whole number of pages, so per_head (16-byte pieces
// per head) is a multiple of 32 * D / 8 = 512 (D = 128) or 1024 (D = 256):
// the launch takes kCopyThreads threads when kCopyUnroll * kCopyThreads
// divides it, else half as many.  A sweep on the 139,264-token K and V
// prefix (4 KV heads, D = 256; per call, with a launch per tensor): 2 x 512
// 174.4 us, 4 x 256 177.7, 2 x 256 180.2, 4 x 128 184.8, 4 x 512 185.4,
// default-policy loads and stores 202.1.  One launch for both measured the
// same (176.47 against 176.81 us) and saves a launch per call.
constexpr int kCopyUnroll = 2, kCopyThreads = 512;
struct CopyArgs {
    uint4 *dst_k, *dst_v;
    const uint4 *src_k, *src_v;
    size_t dst_stride, src_stride, n;
    int kv_heads;
};
__global__ __launch_bounds__(kCopyThreads)
void copy_pages(CopyArgs a) {
    const size_t per_head = a.n / 8;   // uint4 per head
    const size_t chunk = (size_t)kCopyUnroll * blockDim.x;
    const size_t chunks = per_head / chunk * 2 * a.kv_heads;
    for (size_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        const size_t first = c * chunk;
        size_t h = first / per_head;
        const size_t i0 = first - h * per_head + threadIdx.x;
        const bool v_half = h >= (size_t)a.kv_heads;   // uniform per chunk
        if (v_half) h -= a.kv_heads;
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 *s = reinterpret_cast<const u32x4 *>((v_half ? a.src_v : a.src_k) + h * (a.src_stride / 8) + i0);
        u32x4 *d = reinterpret_cast<u32x4 *>((v_half ? a.dst_v : a.dst_k) + h * (a.dst_stride / 8) + i0);
        u32x4 v[kCopyUnroll];
#pragma unroll
        for (int u = 0; u < kCopyUnroll; ++u) v[u] = __builtin_nontemporal_load(s + u * blockDim.x);
#pragma unroll
        for (int u = 0; u < kCopyUnroll; ++u) __builtin_nontemporal_store(v[u], d + u * blockDim.x);
    }
}

}  // namespace

void launch_copy(void *dst_k, void *dst_v, const void *src_k, const void *src_v, int kv_heads,
                 int head_dim, int dst_capacity, int src_capacity, int pages, hipStream_t stream) {
    const size_t n = (size_t)pages * kPageTokens * head_dim;   // 16-bit elements per head
    if (!n) return;
    const int threads = (n / 8) % (kCopyUnroll * kCopyThreads) == 0 ? kCopyThreads : kCopyThreads / 2;
    require((n / 8) % (kCopyUnroll * threads) == 0, "page copy needs whole chunks of 16-byte pieces per head");
    const size_t chunks = n / 8 / (kCopyUnroll * threads) * 2 * kv_heads;
    const unsigned blocks = (unsigned)std::min<size_t>(chunks, 32768);
    CopyArgs a = {static_cast<uint4 *>(dst_k), static_cast<uint4 *>(dst_v), static_cast<const uint4 *>(src_k),
                  static_cast<const uint4 *>(src_v), (size_t)dst_capacity * head_dim,
                  (size_t)src_capacity * head_dim, n, kv_heads};
    hipLaunchKernelGGL(copy_pages, dim3(blocks), dim3(threads), 0, stream, a);
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

void launch_split_query(void *q_hilo, const float *q, size_t n, hipStream_t stream) {
    if (!n) return;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 65536);
    _Float16 *hi = static_cast<_Float16 *>(q_hilo);
    hipLaunchKernelGGL(split_query, dim3(blocks), dim3(256), 0, stream, hi, hi + n, q, n);
    check(hipGetLastError());
}

void launch_prepare(void *q_hilo, void *k_pages, void *v_pages, const float *q_gate,
                    const float *key, const float *value, const float *q_norm,
                    const float *k_norm, int batch, int position, int capacity,
                    float epsilon, hipStream_t stream, bool keys_only) {
    const int head0 = keys_only ? kModelQHeads : 0;
    hipLaunchKernelGGL(prepare_kernel, dim3(kModelQHeads + kModelKvHeads - head0, batch),
                       dim3(kWave), 0, stream, static_cast<_Float16 *>(q_hilo),
                       static_cast<_Float16 *>(k_pages),
                       static_cast<_Float16 *>(v_pages), q_gate, key, value, q_norm, k_norm,
                       position, (size_t)capacity * kModelHeadDim, epsilon, head0);
    check(hipGetLastError());
}

}  // namespace rs
