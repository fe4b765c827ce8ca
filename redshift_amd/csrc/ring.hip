// Split-K partial kernel for 17..64 query rows per KV head: speculative
// verification of up to 8 candidate tokens (6 query heads per KV head), the
// reference's attention_tiled (src/kernels.cu:466-503) over a T-token block
// with causal masking inside the block.
//
// One workgroup (8 waves) owns a contiguous run of pages of one KV head and
// every query row of that head.  The pages stream through a ring of four LDS
// buffers, each holding one [K page | V page] (32 keys, 32 KiB at D=256),
// filled by direct global->LDS loads: three pages are in flight while the
// fourth is consumed, and the loads cost no registers.  All waves share the
// copying.  Query tile t (16 rows) belongs to waves t and t+4, which take the
// first and the second 16 keys of every page with separate online-softmax
// states, merged once at the end; so two waves per SIMD overlap their
// latency chains, and no wave ever waits for another's scores.
//   S^T[key][row] = K[key][:] . Q[row][:]     16x16x32 MFMA (A = K from LDS)
//   O^T[dim][row] += V^T[dim][key] P^T[key][row]
//                                             16x16x16 MFMA (A = V^T from LDS,
//                                             B = P^T straight from S^T's C
//                                             layout)
// The partials (m, l, unnormalised O) use the layout of the other split
// kernels, so attention_combine merges them.
#include "kernels.hpp"

#include <cmath>
#include <cstdint>
#include <type_traits>

namespace rs {
namespace {

template <typename T> struct Vec8;
template <> struct Vec8<_Float16> { using type = f16x8; };
template <> struct Vec8<__bf16> { using type = bf16x8; };
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
template <typename T> struct Vec4;
template <> struct Vec4<_Float16> { using type = f16x4; };
template <> struct Vec4<__bf16> { using type = bf16x4; };

__device__ __forceinline__ f32x4 mfma(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma(f16x4 a, f16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma(bf16x4 a, bf16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                     __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
}

constexpr int kRingWaves = 8;
constexpr float kLazy = 8.f;   // lazy row-max threshold, log2 units

// s_waitcnt vmcnt(N) leaving the other counters alone (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
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
// s_waitcnt lgkmcnt(N), after which v (read by lds_read) may be used.
template <int N, typename V>
__device__ __forceinline__ void lds_wait(V &v) {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "i"(N));
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

template <int D, int NQT, bool PSPLIT, typename KV>
__global__ __launch_bounds__(kRingWaves * kWave, 1)
void attention_ring(SplitArgs a) {
    using V8 = typename Vec8<KV>::type;
    using V4 = typename Vec4<KV>::type;
    constexpr int KS = D / 32, DT = D / 16;
    constexpr int PAGE = 32 * D;                   // elements of one K (or V) page
    constexpr int CHUNKS = 2 * PAGE * 2 / 1024;    // 1 KiB chunks of [K | V]
    constexpr int CPW = CHUNKS / kRingWaves;       // chunks (loads) per wave per page
    static_assert(CHUNKS % kRingWaves == 0, "chunks divide over the waves");
    static_assert(NQT >= 1 && NQT <= 4, "four query tiles at most");
    // The ring: four buffers of one [K page | V page] each.
    __shared__ __attribute__((aligned(16))) KV ring0[2 * PAGE];
    __shared__ __attribute__((aligned(16))) KV ring1[2 * PAGE];
    __shared__ __attribute__((aligned(16))) KV ring2[2 * PAGE];
    __shared__ __attribute__((aligned(16))) KV ring3[2 * PAGE];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4;
    const int qt = w & 3, kt = w >> 2;             // query tile, key half of every page
    const bool computes = qt < NQT;                // wave-uniform
    const int split = blockIdx.x % a.splits, h = blockIdx.x / a.splits;
    const int p0 = (int)((long long)split * a.n_pages / a.splits);
    const int p1 = (int)((long long)(split + 1) * a.n_pages / a.splits);
    const int n = p1 - p0;

    const KV *kh = static_cast<const KV *>(a.k_pages) + (size_t)h * a.head_stride;
    const KV *vh = static_cast<const KV *>(a.v_pages) + (size_t)h * a.head_stride;
    // Wave w copies 1 KiB chunks w*CPW .. w*CPW+CPW-1 of page p's [K | V].
    auto stage = [&](int p, KV *dst) __attribute__((always_inline)) {
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

    // Query fragments of tile qt (B operand of S^T): k-step ks of lane l holds
    // row 16qt + l%16, dims 32ks + 8(l/16) .. +7.  Padded rows repeat the last
    // row and are never stored.  They travel through LDS (ring buffer 3, before
    // its first page), copied by the first wave of each tile: loaded into
    // registers from global memory they would make the compiler wait for every
    // load in flight before the page loop.
    const int row = min(16 * qt + (lane & 15), a.rows - 1);
    const int t = row / a.group;
    const int limit = a.position + t;                            // last key of this row
    const int tile_limit = a.position + min(16 * qt, a.rows - 1) / a.group;
    static_assert(4 * KS * kWave * 8 <= 2 * PAGE, "query fragments fit one ring buffer");
    if (computes && kt == 0) {
        const KV *src = static_cast<const KV *>(a.q) +
                        ((size_t)t * a.q_heads + (size_t)h * a.group + (row - t * a.group)) * D + 8 * g;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(src + 32 * ks),
                                             (__attribute__((address_space(3))) void *)(ring3 + (qt * KS + ks) * kWave * 8),
                                             16, 0, 0);
    }
    V8 qf[KS];

    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;

    auto compute = [&](int p, const KV *cur) __attribute__((always_inline)) {
        const uint32_t kbase = lds_addr(cur) + lane * 16 + kt * (16 * D * 2);
        const uint32_t vbase = lds_addr(cur) + PAGE * 2 + lane * 16 + kt * 8;
        // The wave's 16-key tile of K: KS fragments, requested at once.
        V8 kf[KS];
        static_for<0, KS>([&](auto ks) {
            lds_read<decltype(ks)::value * 1024>(kf[decltype(ks)::value], kbase);
        });
        // Two accumulation chains (even and odd k-steps) halve the latency.
        f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
        static_for<0, KS>([&](auto ks_) {
            constexpr int ks = decltype(ks_)::value;
            lds_wait<KS - 1 - ks>(kf[ks]);
            if constexpr (ks % 2 == 0) s0 = mfma(kf[ks], qf[ks], s0);
            else s1 = mfma(kf[ks], qf[ks], s1);
        });
        // V^T fragments of the same 16 keys (half of each 32-key fragment).
        V4 vf[DT];
        static_for<0, DT>([&](auto dt) {
            lds_read<decltype(dt)::value * 1024>(vf[decltype(dt)::value], vbase);
        });
        // Online softmax over the wave's 16 keys of the page (lane: keys
        // 16kt + 4g + r for row l%16); keys past the row's limit (later
        // candidates, or past the last key) are masked.
        const int key0 = p * 32 + 16 * kt + 4 * g;
        float x[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = (s0[r] + s1[r]) * a.scale_log2;
        if (p * 32 + 31 > tile_limit) {
            keep_branch();
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (key0 + r > limit) x[r] = -INFINITY;
        }
        const float bm = row_group_max(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
        float alpha = 1.f;
        if (bm > m + kLazy) {   // also the first finite block max of a row
            alpha = __builtin_amdgcn_exp2f(m - bm);
            m = bm;
        }
        const float mu = m == -INFINITY ? 0.f : m;
        V4 ph, pl;
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float e = __builtin_amdgcn_exp2f(x[r] - mu);
            const KV eh = (KV)e;
            ph[r] = eh;
            if constexpr (PSPLIT) {
                pl[r] = (KV)(e - (float)eh);
                ps += e;
            } else {
                ps += (float)eh;
            }
        }
        l = l * alpha + ps;
        if (__any(alpha != 1.f)) {
            keep_branch();
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
        }
        if (p * 32 + 32 > a.n_keys) {
            // Last page: V slots past the last key are zeroed (stale pages
            // may hold anything, and 0 * NaN is NaN).
            keep_branch();
            static_for<0, DT>([&](auto dt_) {
                constexpr int dt = decltype(dt_)::value;
                lds_wait<0>(vf[dt]);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (key0 + r >= a.n_keys) vf[dt][r] = (KV)0.f;
            });
        }
        // O^T += V^T P^T over the 16 keys.
        static_for<0, DT>([&](auto dt_) {
            constexpr int dt = decltype(dt_)::value;
            constexpr int later = DT - 1 - dt;
            lds_wait<(later < 15 ? later : 15)>(vf[dt]);
            acc[dt] = mfma(vf[dt], ph, acc[dt]);
            if constexpr (PSPLIT) acc[dt] = mfma(vf[dt], pl, acc[dt]);
        });
    };

    auto wait_page = [&](int i) __attribute__((always_inline)) {
        const int ahead = min(2, n - 1 - i);
        if (ahead >= 2) wait_vmcnt<2 * CPW>();
        else if (ahead == 1) wait_vmcnt<CPW>();
        else wait_vmcnt<0>();
    };
    // Step i: wait for this wave's share of page i (pages i+1 and i+2 may
    // stay in flight; vector-memory counters retire in issue order), meet
    // the other waves (page i complete, page i-1 consumed), refill the
    // consumed buffer with page i+3, then consume page i.
    auto step = [&](int i, const KV *cur, KV *fill) __attribute__((always_inline)) {
        wait_page(i);
        ring_barrier();
        if (i + 3 < n) stage(p0 + i + 3, fill);
        if (computes) compute(p0 + i, cur);
    };

    if (n > 0) {
        stage(p0, ring0);
        if (n > 1) stage(p0 + 1, ring1);
        if (n > 2) stage(p0 + 2, ring2);
        // Step 0: page 0 and the query fragments (loaded first) have landed;
        // the fragments move to registers before page 3 overwrites them.
        wait_page(0);
        ring_barrier();
        if (computes) {
            const uint32_t qbase = lds_addr(ring3) + qt * KS * 1024 + lane * 16;
            static_for<0, KS>([&](auto ks) {
                lds_read<decltype(ks)::value * 1024>(qf[decltype(ks)::value], qbase);
            });
            static_for<0, KS>([&](auto ks) { lds_wait<0>(qf[decltype(ks)::value]); });
        }
        ring_barrier();
        if (3 < n) stage(p0 + 3, ring3);
        if (computes) compute(p0, ring0);
        for (int i = 1; i < n; i += 4) {
            step(i, ring1, ring0);
            if (i + 1 < n) step(i + 1, ring2, ring1);
            if (i + 2 < n) step(i + 2, ring3, ring2);
            if (i + 3 < n) step(i + 3, ring0, ring3);
        }
    }

    // ---- merge the two key halves of every tile, then store the partials ----
    // The last step waited for every load; once all waves are past this
    // barrier no page is read any more, and ring0..ring2 hold the exchange:
    // tile qt's second-half accumulators in ring(qt/2), its m and l in ring2.
    ring_barrier();
    float *xacc = reinterpret_cast<float *>(qt < 2 ? ring0 : ring1) + (qt & 1) * DT * kWave * 4;
    float *xml = reinterpret_cast<float *>(ring2) + qt * 2 * kWave;
    l = row_group_sum(l);
    if (computes && kt == 1) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4 *>(xacc + (dt * kWave + lane) * 4) = acc[dt];
        xml[lane] = m;
        xml[kWave + lane] = l;
    }
    lds_barrier();
    if (computes && kt == 0) {
        const float m1 = xml[lane], l1 = xml[kWave + lane];
        const float M = fmaxf(m, m1);
        const float mu = M == -INFINITY ? 0.f : M;
        const float f0 = __builtin_amdgcn_exp2f(m - mu), f1 = __builtin_amdgcn_exp2f(m1 - mu);
        const int r = 16 * qt + (lane & 15);
        if (r < a.rows) {
            float *pml = a.part_ml + ((size_t)h * a.splits + split) * 2 * a.rows;
            float *po = a.part_o + (((size_t)h * a.splits + split) * a.rows + r) * D + 4 * g;
            if (lane < 16) {
                pml[r] = M;
                pml[a.rows + r] = l * f0 + l1 * f1;
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const f32x4 o1 = *reinterpret_cast<const f32x4 *>(xacc + (dt * kWave + lane) * 4);
                *reinterpret_cast<f32x4 *>(po + dt * 16) = acc[dt] * f0 + o1 * f1;
            }
        }
    }
}

// Raw fp16: 16-bit P; raw bf16: hi + lo P (bf16's 8-bit significand alone
// would dominate the error).
template <int D, int NQT>
const void *pick(Dtype dtype) {
    if (dtype == Dtype::BF16) return (const void *)&attention_ring<D, NQT, true, __bf16>;
    return (const void *)&attention_ring<D, NQT, false, _Float16>;
}

template <int D>
const void *pick_tiles(int nqt, Dtype dtype) {
    switch (nqt) {
        case 1: return pick<D, 1>(dtype);
        case 2: return pick<D, 2>(dtype);
        case 3: return pick<D, 3>(dtype);
        case 4: return pick<D, 4>(dtype);
    }
    return nullptr;
}

}  // namespace

const void *ring_kernel(int D, int nqt, Dtype dtype, bool precise) {
    if (precise) return nullptr;   // fp32 queries (hi + lo parts) use attention_coop
    if (D == 256) return pick_tiles<256>(nqt, dtype);
    if (D == 128) return pick_tiles<128>(nqt, dtype);
    return nullptr;
}

}  // namespace rs
