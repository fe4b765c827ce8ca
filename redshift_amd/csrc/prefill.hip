// Chunked prefill: many query tokens against the paged cache, on the matrix
// cores.  The reference has no prefill kernel (its server prefills 8 tokens
// at a time through attention/attention_tiled, src/kernels.cu:435-503 and
// qvelox/server.py:187-191); this is the same causal GQA formula for long
// token runs: row t sees keys 0..position+t.
//
// One workgroup owns 192 query rows of one KV head (row = token * group +
// query head within the group); each wave owns one 16-row tile (twelve
// waves: three per SIMD) whose query fragments stay in registers.  The workgroup walks
// the pages that its last row can see through a ring of four LDS buffers
// ([K page | V page], 32 KiB at D=256) filled by direct global->LDS loads,
// three pages ahead.  Since pages are stored in MFMA operand order, every
// wave reads its A operands as conflict-free 16-byte LDS fragments, each one
// feeding all of its tiles:
//   S^T[key][row] = K[key][:] . Q[row][:]     (A = K tile from LDS, B = Q)
//   O^T[dim][row] += V^T[dim][key] P^T[key][row]  (A = V^T from LDS, B = P^T,
//                                                  straight from S^T's C layout)
// A page's 16 K fragments are requested at once and consumed as they arrive
// (four independent accumulation chains), and its V fragments are requested
// while the softmax runs.  Online softmax in base 2 with a lazily moved row
// max (see ring.hip).  bf16 caches multiply by P split into hi + lo bf16
// parts, fp16 caches by a single fp16 P.
//
// Scheduling: workgroup i serves KV head i % kv_heads (with 4 KV heads the
// round-robin dispatch over the 8 XCDs keeps every head on the same two XCDs,
// whose L2s then hold that head's pages for all of its workgroups), and row
// tiles go heaviest (latest rows, most keys) first.
#include "kernels.hpp"
#include "lds.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>

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

// Waves per workgroup of ROWS query rows with RT 16-row tiles per wave.
template <int ROWS, int RT> constexpr int prefill_waves() { return ROWS / (16 * RT); }
constexpr float kLazy = 8.f;

struct PrefillArgs {
    const void *q;
    const void *k_pages;
    const void *v_pages;
    void *out;
    size_t head_stride;
    int q_heads, kv_heads, group, rows, position, n_tiles;
    float scale_log2;
};

__device__ __forceinline__ int v_slot_token(int g, int j) {
    return j < 4 ? 4 * g + j : 16 + 4 * g + j - 4;
}

template <int D, typename KV, bool PSPLIT, typename OUT, int RT, int ROWS>
__global__ __launch_bounds__((prefill_waves<ROWS, RT>() * kWave), 1)
void attention_prefill(PrefillArgs a) {
    using V8 = typename Vec8<KV>::type;
    constexpr int kPWaves = prefill_waves<ROWS, RT>(), kRowsPerWave = 16 * RT, kRowsPerGroup = ROWS;
    constexpr int KS = D / 32, DT = D / 16;
    constexpr int PAGE = 32 * D;                       // elements of one K (or V) page
    constexpr int CHUNKS = 2 * PAGE * 2 / 1024;        // 1 KiB chunks of K + V page
    // Waves 0..kLoaders-1 copy the pages (the largest power of two of waves
    // that divides the page's chunks).
    constexpr int kLoaders = kPWaves >= 8 ? 8 : kPWaves;
    constexpr int CPW = CHUNKS / kLoaders;             // chunks (loads) per loader wave per page
    static_assert(CHUNKS % kLoaders == 0, "chunks divide over the loader waves");
    __shared__ __attribute__((aligned(16))) KV ring0[2 * PAGE];
    __shared__ __attribute__((aligned(16))) KV ring1[2 * PAGE];
    __shared__ __attribute__((aligned(16))) KV ring2[2 * PAGE];
    __shared__ __attribute__((aligned(16))) KV ring3[2 * PAGE];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4;
    const int h = blockIdx.x % a.kv_heads;
    const int tile = a.n_tiles - 1 - blockIdx.x / a.kv_heads;        // heaviest first
    const int row0 = tile * kRowsPerGroup + w * kRowsPerWave;

    // Query fragments (B operand): tile rt, k-step ks of lane l holds row
    // row0 + 16*rt + l%16, dims 32*ks + 8*(l/16) .. +7.  Padded rows repeat
    // the last row; their results are not stored.  They are in registers
    // before the first page is requested (a workgroup runs for hundreds of
    // pages, so this one round trip is negligible, and the page loop never
    // waits on them).
    V8 qf[RT][KS];
    int limit[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int row = min(row0 + 16 * rt + (lane & 15), a.rows - 1);
        const int t = row / a.group, gg = row - t * a.group;
        limit[rt] = a.position + t;
        const KV *src = static_cast<const KV *>(a.q) +
                        ((size_t)t * a.q_heads + (size_t)h * a.group + gg) * D + 8 * g;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf[rt][ks] = *reinterpret_cast<const V8 *>(src + 32 * ks);
    }
    wait_vmcnt<0>();
    // Keys this workgroup can see: 0 .. position + (token of its last row).
    const int last_row = min(tile * kRowsPerGroup + kRowsPerGroup - 1, a.rows - 1);
    const int n_keys = a.position + last_row / a.group + 1;
    const int n = (n_keys + 31) / 32;
    // First page that any row of this wave masks (all rows see keys <= position).
    const int wave_first_limit = a.position + min(row0, a.rows - 1) / a.group;

    const KV *kh = static_cast<const KV *>(a.k_pages) + (size_t)h * a.head_stride;
    const KV *vh = static_cast<const KV *>(a.v_pages) + (size_t)h * a.head_stride;
    // Loader wave w copies 1 KiB chunks w*CPW .. of the [K | V] page p into
    // `dst` (the other waves have no loads in flight, so their page waits
    // below return at once).
    auto stage = [&](int p, KV *dst) __attribute__((always_inline)) {
        if (w >= kLoaders) return;
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            const int chunk = w * CPW + c;
            const int half = chunk / (CHUNKS / 2), off = (chunk % (CHUNKS / 2)) * 512;
            const KV *src = (half ? vh : kh) + (size_t)p * PAGE + off + lane * 8;
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(src),
                                             (__attribute__((address_space(3))) void *)(dst + half * PAGE + off),
                                             16, 0, 0);
        }
    };

    f32x4 acc[RT][DT];
    float m[RT], l[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        m[rt] = -INFINITY;
        l[rt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    auto compute = [&](int p, const KV *cur) __attribute__((always_inline)) {
        const uint32_t kbase = lds_addr(cur) + lane * 16;
        const uint32_t vbase = lds_addr(cur) + PAGE * 2 + lane * 16;
        // ---- S^T for both 16-key tiles of the page and all row tiles ----
        // K fragments stream through a window of KW k-steps (2*KW reads in
        // flight, at most 15): the pair of k-step ks+KW is requested as soon
        // as that of ks has landed, and each pair feeds 2*RT independent
        // accumulation chains (row tile x key tile).
        constexpr int KW = 2;
        V8 kf[KS][2];
        auto read_k = [&](auto ks) __attribute__((always_inline)) {
            static_for<0, 2>([&](auto kt) {
                lds_read<(decltype(kt)::value * 16 * D + decltype(ks)::value * 512) * 2>(
                    kf[decltype(ks)::value][decltype(kt)::value], kbase);
            });
        };
        static_for<0, KW>(read_k);
        f32x4 s[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) s[rt][0] = s[rt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
        static_for<0, KS>([&](auto ks_) {
            constexpr int ks = decltype(ks_)::value;
            // Reads issued after this pair: the rest of the window.
            constexpr int later = 2 * (ks + KW <= KS ? KW - 1 : KS - 1 - ks);
            lds_wait<later>(kf[ks][0]);
            lds_wait<later>(kf[ks][1]);
            if constexpr (ks + KW < KS) read_k(std::integral_constant<int, ks + KW>{});
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) s[rt][kt] = mfma(kf[ks][kt], qf[rt][ks], s[rt][kt]);
        });
        // The first VW V fragments are requested now and arrive during the
        // softmax; the rest stream through the same window during O^T.
        constexpr int VW = 4;
        V8 vf[DT];
        auto read_v = [&](auto dt) __attribute__((always_inline)) {
            lds_read<decltype(dt)::value * 1024>(vf[decltype(dt)::value], vbase);
        };
        static_for<0, VW>(read_v);
        // ---- online softmax; keys past a row's limit are masked ----
        V8 ph[RT], pl[RT];
        bool rescale = false;
        float alpha[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = s[rt][j >> 2][j & 3] * a.scale_log2;
            if (p * 32 + 31 > wave_first_limit) {
                keep_branch();
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (p * 32 + 16 * (j >> 2) + 4 * g + (j & 3) > limit[rt]) x[j] = -INFINITY;
            }
            const float bm = row_group_max(fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])),
                                                 fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7]))));
            alpha[rt] = 1.f;
            if (bm > m[rt] + kLazy) {
                alpha[rt] = __builtin_amdgcn_exp2f(m[rt] - bm);
                m[rt] = bm;
                rescale = true;
            }
            const float mu = m[rt] == -INFINITY ? 0.f : m[rt];
            float ps = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float e = __builtin_amdgcn_exp2f(x[j] - mu);
                const KV eh = (KV)e;
                ph[rt][j] = eh;
                if constexpr (PSPLIT) {
                    pl[rt][j] = (KV)(e - (float)eh);
                    ps += e;
                } else {
                    ps += (float)eh;
                }
            }
            l[rt] = l[rt] * alpha[rt] + ps;
        }
        if (__any(rescale)) {
            keep_branch();
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) acc[rt][dt] *= alpha[rt];
        }
        // Last page: V slots past the last key are zeroed (stale pages may
        // hold anything, and 0 * NaN is NaN).
        const bool tail = p * 32 + 32 > n_keys;
        // ---- O^T += V^T P^T ----
        static_for<0, DT>([&](auto dt_) {
            constexpr int dt = decltype(dt_)::value;
            constexpr int later = dt + VW <= DT ? VW - 1 : DT - 1 - dt;
            lds_wait<later>(vf[dt]);
            if constexpr (dt + VW < DT) read_v(std::integral_constant<int, dt + VW>{});
            if (tail) {
                keep_branch();
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (p * 32 + v_slot_token(g, j) >= n_keys) vf[dt][j] = (KV)0.f;
            }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                acc[rt][dt] = mfma(vf[dt], ph[rt], acc[rt][dt]);
                if constexpr (PSPLIT) acc[rt][dt] = mfma(vf[dt], pl[rt], acc[rt][dt]);
            }
        });
    };

    auto wait_page = [&](int i) __attribute__((always_inline)) {
        const int ahead = min(2, n - 1 - i);
        if (ahead >= 2) wait_vmcnt<2 * CPW>();
        else if (ahead == 1) wait_vmcnt<CPW>();
        else wait_vmcnt<0>();
    };
    // Step i: this wave's share of page i has landed (pages i+1 and i+2 may
    // stay in flight), the waves meet (page i complete, page i-1 consumed),
    // the consumed buffer is refilled with page i+3, and page i is consumed.
    auto step = [&](int i, const KV *cur, KV *fill) __attribute__((always_inline)) {
        wait_page(i);
        ring_barrier();
        if (i + 3 < n) stage(i + 3, fill);
        compute(i, cur);
    };

    stage(0, ring0);
    if (n > 1) stage(1, ring1);
    if (n > 2) stage(2, ring2);
    for (int i = 0; i < n; i += 4) {
        step(i, ring0, ring3);
        if (i + 1 < n) step(i + 1, ring1, ring0);
        if (i + 2 < n) step(i + 2, ring2, ring1);
        if (i + 3 < n) step(i + 3, ring3, ring2);
    }

    // ---- normalise and store rows ----
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        l[rt] = row_group_sum(l[rt]);
        const int row = row0 + 16 * rt + (lane & 15);
        if (row < a.rows) {
            const int t = row / a.group, gg = row - t * a.group;
            OUT *dst = static_cast<OUT *>(a.out) + ((size_t)t * a.q_heads + (size_t)h * a.group + gg) * D + 4 * g;
            const float inv = 1.f / l[rt];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                typedef OUT OUT4 __attribute__((ext_vector_type(4)));
                OUT4 o;
#pragma unroll
                for (int r = 0; r < 4; ++r) o[r] = (OUT)(acc[rt][dt][r] * inv);
                *reinterpret_cast<OUT4 *>(dst + dt * 16) = o;
            }
        }
    }
}

// Row tiles per wave: one.  Rows per workgroup: 192 (twelve waves, three
// per SIMD, whose softmax and matrix work overlap; and 2048 tokens of six
// query heads per KV head make 64 workgroups per KV head, one round on 256
// CUs) or 128 (RS_PREFILL_ROWS=128, for measurement).
constexpr int kPrefillRT = 1;

int prefill_rows() {
    static const int rows = [] {
        const char *v = std::getenv("RS_PREFILL_ROWS");
        return v && std::atoi(v) == 128 ? 128 : 192;
    }();
    return rows;
}

template <int D, int ROWS>
const void *prefill_kernel(Dtype dtype, bool out_f32) {
    constexpr int RT = kPrefillRT;
    if (dtype == Dtype::BF16)
        return out_f32 ? (const void *)&attention_prefill<D, __bf16, true, float, RT, ROWS>
                       : (const void *)&attention_prefill<D, __bf16, true, __bf16, RT, ROWS>;
    return out_f32 ? (const void *)&attention_prefill<D, _Float16, false, float, RT, ROWS>
                   : (const void *)&attention_prefill<D, _Float16, false, _Float16, RT, ROWS>;
}

template <int D>
const void *prefill_kernel(Dtype dtype, bool out_f32, int rows) {
    return rows == 128 ? prefill_kernel<D, 128>(dtype, out_f32) : prefill_kernel<D, 192>(dtype, out_f32);
}

}  // namespace

void launch_prefill(const Shape &s, Dtype dtype, float scale, const void *q, const void *k_pages,
                    const void *v_pages, void *out, bool out_f32, hipStream_t stream) {
    PrefillArgs a;
    a.q = q;
    a.k_pages = k_pages;
    a.v_pages = v_pages;
    a.out = out;
    a.head_stride = (size_t)s.capacity * s.head_dim;
    a.q_heads = s.q_heads;
    a.kv_heads = s.kv_heads;
    a.group = s.group();
    a.rows = s.group() * s.tokens;
    a.position = s.position;
    const int rows = prefill_rows();
    a.n_tiles = (a.rows + rows - 1) / rows;
    a.scale_log2 = scale * 1.4426950408889634f;
    const void *kernel = s.head_dim == 256 ? prefill_kernel<256>(dtype, out_f32, rows)
                       : s.head_dim == 128 ? prefill_kernel<128>(dtype, out_f32, rows) : nullptr;
    require(kernel != nullptr, "unsupported head_dim for the prefill kernel");
    void *args[] = {&a};
    const int threads = (rows / (16 * kPrefillRT)) * kWave;
    check(hipLaunchKernel(kernel, dim3(a.n_tiles * s.kv_heads), dim3(threads), args, 0, stream));
}

}  // namespace rs
