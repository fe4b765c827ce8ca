// GQA attention over the paged KV cache: split-K partial kernel (decode and
// speculative verification) and the log-sum-exp combine.
//
// Reference counterparts: attention / attention_tiled (src/kernels.cu:435-456,
// 466-503) compute, for every query head h and new token t, the causal softmax
// of q . K^T * scale over keys 0..base+t of kv head h/6, times V.  They run one
// 256-thread block per (head, token), so a 139,264-key decode uses 24 blocks
// and every KV head is read 6*T times.  Here one workgroup owns a (KV head,
// key range) pair and serves all group*tokens query rows of that KV head from
// one pass over the pages, on the matrix cores:
//   S^T[key][row] = K[key][:] . Q[row][:]    v_mfma_f32_16x16x32_{f16,bf16}
//   O^T[dim][row] += V^T[dim][key] P^T[key][row]
// Online softmax (base-2, fp32) runs on the S^T accumulators in registers: the
// C layout of S^T is already the B-operand layout of P^T for the next MFMA
// (see the V page layout in common.hpp), so P never leaves the lane.
#include "kernels.hpp"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

namespace rs {
namespace {

template <typename T> struct Vec8;
template <> struct Vec8<_Float16> { using type = f16x8; };
template <> struct Vec8<__bf16> { using type = bf16x8; };

__device__ __forceinline__ f32x4 mfma(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

constexpr int kWaves = 4;          // waves per workgroup of the split kernel
constexpr int kMaxSplits = 1024;   // bound on workgroups per KV head

struct SplitArgs {
    const void *q;
    const void *k_pages;
    const void *v_pages;
    float *part_o;    // [kv_heads][splits][rows][D]   unnormalised, base-2 max m
    float *part_ml;   // [kv_heads][splits][2][rows]   m (log2 domain), then l
    size_t head_stride;
    int q_heads, group, rows, position, n_keys, n_blocks, splits;
    float scale_log2;
};

// One workgroup = kWaves waves = one (split, KV head).  The split's 32-key
// blocks are shared out evenly over the waves; every wave keeps its own
// online-softmax state for all rows and the waves merge through LDS at the end.
// Keys past n_keys in the last page are masked (scores) and zeroed (values),
// so stale page contents never reach the result.
template <int D, int NQT, bool PRECISE, typename KV>
__global__ __launch_bounds__(kWaves * kWave)
void attention_split(SplitArgs a) {
    using V8 = typename Vec8<KV>::type;
    constexpr int KS = D / 32, DT = D / 16, NQ = PRECISE ? 2 : 1;
    constexpr int QBYTES = NQ * NQT * KS * kWave * 16;
    constexpr int OBYTES = NQT * DT * kWave * 16;
    constexpr int SBYTES = QBYTES > OBYTES ? QBYTES : OBYTES;
    __shared__ __attribute__((aligned(16))) unsigned char smem[SBYTES];
    __shared__ float sml[kWaves][2][16 * NQT];
    V8 *sq = reinterpret_cast<V8 *>(smem);          // [NQ][NQT][KS][64] query fragments
    f32x4 *so = reinterpret_cast<f32x4 *>(smem);    // [NQT][DT][64] merge buffer (after loop)

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int split = blockIdx.x, h = blockIdx.y;

    // Query fragments in B-operand order: lane l of (qt, ks) holds row
    // 16*qt + l%16, dims 32*ks + 8*(l/16) .. +7.  Rows past `rows` are zero.
    for (int e = threadIdx.x; e < NQT * KS * kWave; e += kWaves * kWave) {
        const int l = e & 63, ks = (e >> 6) % KS, qt = e / (KS * kWave);
        const int row = 16 * qt + (l & 15), d0 = 32 * ks + 8 * (l >> 4);
        V8 hi = {}, lo = {};
        if (row < a.rows) {
            const int t = row / a.group, g = row - t * a.group;
            const size_t base = ((size_t)t * a.q_heads + (size_t)h * a.group + g) * D + d0;
            if constexpr (PRECISE) {
                // fp32 query as hi + lo 16-bit parts: the two MFMAs carry ~22
                // significant bits, which keeps the fused path at fp32 accuracy.
                const float4 *src = reinterpret_cast<const float4 *>(static_cast<const float *>(a.q) + base);
                const float4 x0 = src[0], x1 = src[1];
                const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    hi[i] = (KV)x[i];
                    lo[i] = (KV)(x[i] - (float)hi[i]);
                }
            } else {
                hi = *reinterpret_cast<const V8 *>(static_cast<const KV *>(a.q) + base);
            }
        }
        sq[e] = hi;
        if constexpr (PRECISE) sq[NQT * KS * kWave + e] = lo;
    }
    __syncthreads();

    const long long waves_total = (long long)a.splits * kWaves;
    const long long wi = (long long)split * kWaves + w;
    const int b0 = (int)(wi * a.n_blocks / waves_total);
    const int b1 = (int)((wi + 1) * a.n_blocks / waves_total);
    const KV *kh = static_cast<const KV *>(a.k_pages) + (size_t)h * a.head_stride + lane * 8;
    const KV *vh = static_cast<const KV *>(a.v_pages) + (size_t)h * a.head_stride + lane * 8;

    // Last visible key of each row this lane holds (row 16*qt + lane%16).
    int limit[NQT];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        const int row = min(16 * qt + (lane & 15), a.rows - 1);
        limit[qt] = a.position + row / a.group;
    }

    f32x4 acc[NQT][DT];
    float m[NQT], l[NQT];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        m[qt] = -INFINITY;
        l[qt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    V8 kb[2][KS];
    if (b0 < b1) {
        const KV *kp = kh + (size_t)b0 * 32 * D;
#pragma unroll
        for (int tile = 0; tile < 2; ++tile)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                kb[tile][ks] = *reinterpret_cast<const V8 *>(kp + tile * 16 * D + ks * 512);
    }

    for (int b = b0; b < b1; ++b) {
        // V of this block is in flight while the scores are computed.
        V8 vb[DT];
        const KV *vp = vh + (size_t)b * 32 * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) vb[dt] = *reinterpret_cast<const V8 *>(vp + dt * 512);

        f32x4 s[NQT][2];
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt) s[qt][0] = s[qt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
            for (int qt = 0; qt < NQT; ++qt) {
                const V8 qf = sq[(qt * KS + ks) * kWave + lane];
                s[qt][0] = mfma(kb[0][ks], qf, s[qt][0]);
                s[qt][1] = mfma(kb[1][ks], qf, s[qt][1]);
                if constexpr (PRECISE) {
                    const V8 ql = sq[((NQT + qt) * KS + ks) * kWave + lane];
                    s[qt][0] = mfma(kb[0][ks], ql, s[qt][0]);
                    s[qt][1] = mfma(kb[1][ks], ql, s[qt][1]);
                }
            }
        }
        // K of the next block is in flight during the softmax and P.V.
        if (b + 1 < b1) {
            const KV *kp = kh + (size_t)(b + 1) * 32 * D;
#pragma unroll
            for (int tile = 0; tile < 2; ++tile)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    kb[tile][ks] = *reinterpret_cast<const V8 *>(kp + tile * 16 * D + ks * 512);
        }

        // Lane l holds keys b*32 + 16*tile + 4*(l/16) + r for r < 4.
        const int key0 = b * 32 + 4 * (lane >> 4);
        const bool edge = b * 32 + 31 > a.position;
        V8 ph[NQT], pl[NQT];
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt) {
            float x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = s[qt][j >> 2][j & 3] * a.scale_log2;
            if (edge) {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (key0 + 16 * (j >> 2) + (j & 3) > limit[qt]) x[j] = -INFINITY;
            }
            float bm = x[0];
#pragma unroll
            for (int j = 1; j < 8; ++j) bm = fmaxf(bm, x[j]);
            bm = fmaxf(bm, __shfl_xor(bm, 16, kWave));
            bm = fmaxf(bm, __shfl_xor(bm, 32, kWave));
            const float mn = fmaxf(m[qt], bm);
            const float mu = mn == -INFINITY ? 0.f : mn;   // fully masked so far
            const float alpha = exp2f(m[qt] - mu);
            m[qt] = mn;
            float ps = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float e = exp2f(x[j] - mu);
                const KV eh = (KV)e;
                ph[qt][j] = eh;
                if constexpr (PRECISE) {
                    pl[qt][j] = (KV)(e - (float)eh);
                    ps += e;
                } else {
                    ps += (float)eh;   // normalise by the weights actually applied
                }
            }
            l[qt] = l[qt] * alpha + ps;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) acc[qt][dt] *= alpha;
        }
        if (b * 32 + 32 > a.n_keys) {
            // Zero V slots past the last key: 0 * (stale NaN) would poison O.
            const int g = lane >> 4;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int token = b * 32 + (j < 4 ? 4 * g + j : 16 + 4 * g + j - 4);
                if (token >= a.n_keys) {
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) vb[dt][j] = (KV)0.f;
                }
            }
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
            for (int qt = 0; qt < NQT; ++qt) {
                acc[qt][dt] = mfma(vb[dt], ph[qt], acc[qt][dt]);
                if constexpr (PRECISE) acc[qt][dt] = mfma(vb[dt], pl[qt], acc[qt][dt]);
            }
        }
    }

    // ---- merge the waves of this workgroup -------------------------------
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        l[qt] += __shfl_xor(l[qt], 16, kWave);
        l[qt] += __shfl_xor(l[qt], 32, kWave);
    }
    if (lane < 16) {
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt) {
            sml[w][0][16 * qt + lane] = m[qt];
            sml[w][1][16 * qt + lane] = l[qt];
        }
    }
    __syncthreads();   // every wave is past the loop: smem may now hold `so`
    float *pml = a.part_ml + ((size_t)h * a.splits + split) * 2 * a.rows;
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        const int row = 16 * qt + (lane & 15);
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, sml[ww][0][row]);
        const float mu = M == -INFINITY ? 0.f : M;
        const float f = exp2f(m[qt] - mu);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[qt][dt] *= f;
        if (w == 0 && lane < 16 && row < a.rows) {
            float L = 0.f;
#pragma unroll
            for (int ww = 0; ww < kWaves; ++ww) L += sml[ww][1][row] * exp2f(sml[ww][0][row] - mu);
            pml[row] = M;
            pml[a.rows + row] = L;
        }
    }
    for (int step = 0; step < kWaves; ++step) {
        if (w == step) {
#pragma unroll
            for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    f32x4 &dst = so[(qt * DT + dt) * kWave + lane];
                    dst = step ? dst + acc[qt][dt] : acc[qt][dt];
                }
        }
        __syncthreads();
    }
    // Row-major store of the merged partial: element (row, 4*d4 .. +3) is the
    // f32x4 of lane (row%16) + 16*(d4%4) in fragment (row/16, d4/4).
    f32x4 *po = reinterpret_cast<f32x4 *>(a.part_o + ((size_t)h * a.splits + split) * a.rows * D);
    for (int e = threadIdx.x; e < a.rows * (D / 4); e += kWaves * kWave) {
        const int row = e / (D / 4), d4 = e - row * (D / 4);
        po[e] = so[((row >> 4) * DT + (d4 >> 2)) * kWave + (row & 15) + 16 * (d4 & 3)];
    }
}

struct CombineArgs {
    const float *part_o, *part_ml;
    void *out;
    const float *gate;   // fused mode: q_gate rows of 2*D floats, gate at +D
    int q_heads, group, rows, splits;
};

// One workgroup per (row, KV head), one thread per head dim.
template <int D, typename KV, bool FUSED>
__global__ __launch_bounds__(D)
void attention_combine(CombineArgs c) {
    constexpr int NW = D / kWave;
    __shared__ float wts[kMaxSplits];
    __shared__ float red[NW];
    const int row = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const float *ml = c.part_ml + (size_t)h * c.splits * 2 * c.rows;

    float M = -INFINITY;
    for (int s = tid; s < c.splits; s += D) M = fmaxf(M, ml[(size_t)s * 2 * c.rows + row]);
    M = wave_max(M);
    if (lane == 0) red[w] = M;
    __syncthreads();
    M = red[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) M = fmaxf(M, red[i]);
    __syncthreads();
    const float mu = M == -INFINITY ? 0.f : M;
    float L = 0.f;
    for (int s = tid; s < c.splits; s += D) {
        const float wgt = exp2f(ml[(size_t)s * 2 * c.rows + row] - mu);
        wts[s] = wgt;
        L += wgt * ml[(size_t)s * 2 * c.rows + c.rows + row];
    }
    L = wave_sum(L);
    if (lane == 0) red[w] = L;
    __syncthreads();
    L = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) L += red[i];

    const float *po = c.part_o + ((size_t)h * c.splits * c.rows + row) * D + tid;
    const size_t stride = (size_t)c.rows * D;
    float acc = 0.f;
    int s = 0;
    for (; s + 4 <= c.splits; s += 4) {
        const float v0 = po[(size_t)s * stride], v1 = po[(size_t)(s + 1) * stride];
        const float v2 = po[(size_t)(s + 2) * stride], v3 = po[(size_t)(s + 3) * stride];
        acc += wts[s] * v0 + wts[s + 1] * v1 + wts[s + 2] * v2 + wts[s + 3] * v3;
    }
    for (; s < c.splits; ++s) acc += wts[s] * po[(size_t)s * stride];
    const float o = acc / L;
    const int t = row / c.group, hq = h * c.group + (row - t * c.group);
    const size_t idx = ((size_t)t * c.q_heads + hq) * D + tid;
    if constexpr (FUSED) {
        const float g = c.gate[((size_t)t * c.q_heads + hq) * 2 * D + D + tid];
        static_cast<float *>(c.out)[idx] = o * (1.f / (1.f + expf(-g)));
    } else {
        static_cast<KV *>(c.out)[idx] = (KV)o;
    }
}

template <int D, int NQT, bool PRECISE, typename KV>
const void *split_symbol() {
    return reinterpret_cast<const void *>(&attention_split<D, NQT, PRECISE, KV>);
}

// Resolve the kernel instance for (D, nqt, precise, dtype).
const void *split_kernel(int D, int nqt, bool precise, Dtype dtype) {
#define RS_SPLIT_CASE(DD, Q)                                                        \
    if (D == DD && nqt == Q) {                                                      \
        if (precise) return split_symbol<DD, Q, true, _Float16>();                  \
        return dtype == Dtype::BF16 ? split_symbol<DD, Q, false, __bf16>()          \
                                    : split_symbol<DD, Q, false, _Float16>();       \
    }
    RS_SPLIT_CASE(128, 1)
    RS_SPLIT_CASE(256, 1)
#undef RS_SPLIT_CASE
    throw std::invalid_argument("unsupported head_dim / query rows for the split kernel");
}

}  // namespace

int device_cu_count() {
    static std::mutex mutex;
    static std::vector<int> cache;
    int device = 0;
    check(hipGetDevice(&device));
    std::lock_guard<std::mutex> lock(mutex);
    if ((int)cache.size() <= device) cache.resize(device + 1, 0);
    if (!cache[device]) {
        int cus = 0;
        check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
        cache[device] = cus > 0 ? cus : 1;
    }
    return cache[device];
}

int chunk_tokens(const Shape &s) { return std::max(1, kMaxRows / s.group()); }

SplitPlan plan_split(const Shape &s, int tokens, bool precise) {
    (void)precise;
    SplitPlan p;
    p.rows = s.group() * tokens;
    p.nqt = (p.rows + 15) / 16;
    const long long n_keys = (long long)s.position + tokens;
    p.n_blocks = (int)((n_keys + kPageTokens - 1) / kPageTokens);
    // One workgroup per CU keeps every CU streaming; never give a wave less
    // than one block on average.
    const int per_head = (device_cu_count() + s.kv_heads - 1) / s.kv_heads;
    const int by_blocks = (p.n_blocks + kWaves - 1) / kWaves;
    p.splits = std::max(1, std::min({per_head, by_blocks, kMaxSplits}));
    return p;
}

size_t plan_bytes(const Shape &s, const SplitPlan &p) {
    return (size_t)s.kv_heads * p.splits * p.rows * ((size_t)s.head_dim + 2) * sizeof(float);
}

size_t attention_workspace_bytes(const Shape &s, bool precise) {
    const int ct = chunk_tokens(s);
    size_t best = 0;
    for (int t0 = 0; t0 < s.tokens; t0 += ct) {
        Shape c = s;
        c.position = s.position + t0;
        best = std::max(best, plan_bytes(c, plan_split(c, std::min(ct, s.tokens - t0), precise)));
    }
    return best;
}

void launch_split(const Shape &s, const SplitPlan &plan, Dtype dtype, bool precise,
                  float scale, const void *q, const void *k_pages, const void *v_pages,
                  void *workspace, hipStream_t stream) {
    SplitArgs a;
    a.q = q;
    a.k_pages = k_pages;
    a.v_pages = v_pages;
    a.part_o = static_cast<float *>(workspace);
    a.part_ml = a.part_o + (size_t)s.kv_heads * plan.splits * plan.rows * s.head_dim;
    a.head_stride = (size_t)s.capacity * s.head_dim;
    a.q_heads = s.q_heads;
    a.group = s.group();
    a.rows = plan.rows;
    a.position = s.position;
    a.n_keys = s.position + plan.rows / s.group();
    a.n_blocks = plan.n_blocks;
    a.splits = plan.splits;
    a.scale_log2 = scale * 1.4426950408889634f;
    const void *kernel = split_kernel(s.head_dim, plan.nqt, precise, dtype);
    void *args[] = {&a};
    check(hipLaunchKernel(kernel, dim3(plan.splits, s.kv_heads), dim3(kWaves * kWave),
                          args, 0, stream));
}

void launch_combine(const Shape &s, const SplitPlan &plan, Dtype dtype,
                    const void *workspace, void *out, const float *gate,
                    hipStream_t stream) {
    CombineArgs c;
    c.part_o = static_cast<const float *>(workspace);
    c.part_ml = c.part_o + (size_t)s.kv_heads * plan.splits * plan.rows * s.head_dim;
    c.out = out;
    c.gate = gate;
    c.q_heads = s.q_heads;
    c.group = s.group();
    c.rows = plan.rows;
    c.splits = plan.splits;
    const dim3 grid(plan.rows, s.kv_heads);
    const void *kernel = nullptr;
    if (s.head_dim == 256) {
        kernel = gate ? (const void *)&attention_combine<256, _Float16, true>
               : dtype == Dtype::BF16 ? (const void *)&attention_combine<256, __bf16, false>
                                      : (const void *)&attention_combine<256, _Float16, false>;
    } else if (s.head_dim == 128) {
        kernel = gate ? (const void *)&attention_combine<128, _Float16, true>
               : dtype == Dtype::BF16 ? (const void *)&attention_combine<128, __bf16, false>
                                      : (const void *)&attention_combine<128, _Float16, false>;
    } else {
        throw std::invalid_argument("unsupported head_dim for the combine kernel");
    }
    void *args[] = {&c};
    check(hipLaunchKernel(kernel, grid, dim3(s.head_dim), args, 0, stream));
}

}  // namespace rs
