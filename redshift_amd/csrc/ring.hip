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
// kernels, so attention_combine merges them.  A precise instance (QSPLIT)
// takes an fp32 query as fp16 hi + lo parts (the fused path): S^T gets one
// more MFMA per fragment and P is split into hi + lo parts as well.
//
// PREP (the fused verification of 3..8 new tokens): the precise query is
// not read from q / q_lo but prepared here from a.tok while the first pages
// are in flight.  Wave w prepares the six query rows of new token w with
// the prepare kernel's functions and layout (so the same bits): untracked
// loads requested before the pages, RMSNorm, gamma and RoPE, the fp32 rows
// then written to a query area in LDS, from which every computing wave
// reads its tile's fragments and splits them into hi + lo fp16 parts.  The
// ring has three buffers here (the query area takes the fourth's LDS).
// Every row sees the cached keys 0 .. a.position; the first split's wave w
// also prepares new key w in the prologue and writes it into a block of 16
// keys in the free ring buffer, which the first key half of every tile
// attends to (row t seeing new keys 0..t) before page 0.  So the partials
// hold every key, and the plain gated combine merges them.  The first
// split appends key and value w to the pages once its page loop is done,
// before the merge of the key halves: stores issued among the page loads
// would share the vector-memory counter that the ring's waits count page
// loads on.  (Appending in the combine instead,
// by one workgroup per KV head, measured slower: the combine's critical
// path grew by more than the split kernel's.)
#include "kernels.hpp"
#include "lds.hpp"
#include "prep.hpp"

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
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
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
constexpr int kRingBuffers = 4;   // NBUF-1 pages in flight while one is consumed
// Cache policy of the page loads: non-temporal (each page is read once).
// The partials are stored and read back non-temporally as well: split +
// combine at verify-8 on a 16K prefix take 21.0-21.3 us that way, against
// 22.8-23.0 us with default loads and stores, and 24.2 us with non-temporal
// page loads alone.
constexpr int kStreamLoad = 2;
constexpr float kLazy = 8.f;   // lazy row-max threshold, log2 units

// OUT: kOutPartials stores the split's partial rows; a direct output
// (kOutSame or kOutF32: one split per KV head) stores the final rows
// instead, and no combine runs.
template <int D, int NQT, bool PSPLIT, typename KV, bool QSPLIT = false, int OUT = kOutPartials, bool PREP = false>
__global__ __launch_bounds__(kRingWaves * kWave, 1)
void attention_ring(SplitArgs a) {
    using V8 = typename Vec8<KV>::type;
    using V4 = typename Vec4<KV>::type;
    constexpr int KS = D / 32, DT = D / 16;
    constexpr int PAGE = 32 * D;                   // elements of one K (or V) page
    // Raw fp16: partial rows stored as fp16 O / l (SplitPlan::half_parts).
    constexpr bool HALF = OUT == kOutPartials && !QSPLIT && std::is_same<KV, _Float16>::value;
    constexpr int CHUNKS = 2 * PAGE * 2 / 1024;    // 1 KiB chunks of [K | V]
    constexpr int CPW = CHUNKS / kRingWaves;       // chunks (loads) per wave per page
    static_assert(CHUNKS % kRingWaves == 0, "chunks divide over the waves");
    static_assert(NQT >= 1 && NQT <= 4, "four query tiles at most");
    static_assert(!PREP || (D == kModelHeadDim && QSPLIT && PSPLIT && OUT == kOutPartials &&
                            std::is_same<KV, _Float16>::value),
                  "the prepared query is the fp32 query of the 256-dim fp16 model, as hi + lo parts");
    // The ring: NBUF buffers of one [K page | V page] each (128 KiB of LDS
    // at D=256; PREP: three buffers and the query area, 145 KiB).
    constexpr int NBUF = PREP ? 3 : kRingBuffers;
    __shared__ __attribute__((aligned(16))) KV ring[NBUF][2 * PAGE];
    // PREP: the prepared fp32 query rows, row r at r * QSTRIDE floats (the
    // padding keeps the row-wise writes and the fragment reads free of bank
    // conflicts).
    constexpr int QSTRIDE = D + 4;
    __shared__ __attribute__((aligned(16))) float qarea[PREP ? kMaxRows * QSTRIDE : 4];
    KV *const ring0 = ring[0], *const ring1 = ring[1], *const ring2 = ring[2];

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
                                             16, 0, kStreamLoad);
        }
    };

    // Query fragments of tile qt (B operand of S^T): k-step ks of lane l holds
    // row 16qt + l%16, dims 32ks + 8(l/16) .. +7.  Padded rows repeat the last
    // row and are never stored.  They travel through LDS (ring buffer 3, before
    // its first page), copied by the first wave of each tile: loaded into
    // registers from global memory they would make the compiler wait for every
    // load in flight before the page loop.  The lo parts of a precise query
    // travel through ring buffer 2, copied by the tile's second wave; page 2
    // is then requested after the fragments have moved to registers.
    const int row = min(16 * qt + (lane & 15), a.rows - 1);
    const int t = row / a.group;
    // Last key of this row (PREP: the last cached key, for every row).
    const int limit = a.position + (PREP ? 0 : t);
    const int tile_limit = a.position + (PREP ? 0 : min(16 * qt, a.rows - 1) / a.group);
    static_assert(4 * KS * kWave * 8 <= 2 * PAGE, "query fragments fit one ring buffer");
    if (!PREP && computes && (kt == 0 || QSPLIT)) {
        const KV *src = static_cast<const KV *>(kt == 0 ? a.q : a.q_lo) +
                        ((size_t)t * a.q_heads + (size_t)h * a.group + (row - t * a.group)) * D + 8 * g;
        KV *dst = kt == 0 ? ring[NBUF - 1] : ring[NBUF - 2];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(src + 32 * ks),
                                             (__attribute__((address_space(3))) void *)(dst + (qt * KS + ks) * kWave * 8),
                                             16, 0, 0);
    }
    V8 qf[KS], qlo[QSPLIT ? KS : 1];

    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;

    // attend: the wave's 16 keys of the page in `cur` whose first key is
    // k_first; keys past lim (a row's last key; tlim: the tile's smallest
    // lim) are masked, and with `tail` the V slots past the last key zeroed.
    auto attend = [&](int k_first, const KV *cur, int lim, int tlim, bool tail) __attribute__((always_inline)) {
        const uint32_t kbase = lds_addr(cur) + lane * 16 + kt * (16 * D * 2);
        const uint32_t vbase = lds_addr(cur) + PAGE * 2 + lane * 16 + kt * 8;
        // S^T and the softmax run at raised wave priority, P.V at the
        // default one: the two waves of a query tile share a SIMD and leave
        // each barrier together, and the priorities let one run ahead
        // (verify-8 at 16K: 20.38-20.81 -> 20.29-20.44 us per layer).
        __builtin_amdgcn_s_setprio(1);
        // The wave's 16-key tile of K: KS fragments, requested at once.
        V8 kf[KS];
        static_for<0, KS>([&](auto ks) {
            lds_read<decltype(ks)::value * 1024>(kf[decltype(ks)::value], kbase);
        });
        // Two accumulation chains (even and odd k-steps, or hi and lo query
        // parts) halve the latency.
        f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
        static_for<0, KS>([&](auto ks_) {
            constexpr int ks = decltype(ks_)::value;
            lds_wait<KS - 1 - ks>(kf[ks]);
            if constexpr (QSPLIT) {
                s0 = mfma(kf[ks], qf[ks], s0);
                s1 = mfma(kf[ks], qlo[ks], s1);
            } else if constexpr (ks % 2 == 0) {
                s0 = mfma(kf[ks], qf[ks], s0);
            } else {
                s1 = mfma(kf[ks], qf[ks], s1);
            }
        });
        // V^T fragments of the same 16 keys (half of each 32-key fragment):
        // the first half requested now, the second once it has landed (at
        // most 15 LDS reads in flight).
        constexpr int VB = DT / 2;
        V4 vf[DT];
        auto read_v = [&](auto dt) __attribute__((always_inline)) {
            lds_read<decltype(dt)::value * 1024>(vf[decltype(dt)::value], vbase);
        };
        static_for<0, VB>(read_v);
        // Online softmax over the wave's 16 keys of the page (lane: keys
        // 16kt + 4g + r for row l%16); keys past the row's limit (later
        // candidates, or past the last key) are masked.
        const int key0 = k_first + 16 * kt + 4 * g;
        float x[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = (s0[r] + s1[r]) * a.scale_log2;
        if (k_first + 31 > tlim) {
            keep_branch();
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (key0 + r > lim) x[r] = -INFINITY;
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
        __builtin_amdgcn_s_setprio(0);
        lds_wait<VB - 1>(vf[0]);
        static_for<VB, DT>(read_v);
        if (tail) {
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
        // O^T += V^T P^T over the 16 keys.  With hi + lo P, both parts go
        // through one 16x16x32 product: its k = 8g + r takes P_hi of key
        // 4g + r and k = 8g + 4 + r P_lo of the same key (lane group g's own
        // registers), and V^T holds those four keys in both halves, so the
        // product sums V (P_hi + P_lo) over the 16 keys in one instruction
        // instead of two 16x16x16 ones.
        static_for<0, DT>([&](auto dt_) {
            constexpr int dt = decltype(dt_)::value;
            lds_wait<DT - 1 - dt>(vf[dt]);
            if constexpr (PSPLIT)
                acc[dt] = mfma(__builtin_shufflevector(vf[dt], vf[dt], 0, 1, 2, 3, 0, 1, 2, 3),
                               __builtin_shufflevector(ph, pl, 0, 1, 2, 3, 4, 5, 6, 7), acc[dt]);
            else
                acc[dt] = mfma(vf[dt], ph, acc[dt]);
        });
    };

    auto compute = [&](int p, const KV *cur) __attribute__((always_inline)) {
        attend(p * 32, cur, limit, tile_limit, p * 32 + 32 > a.n_keys);
    };

    // Before step i's barrier, pages i+1 .. i+NBUF-2 may stay in flight
    // (vector-memory counters retire in issue order).
    auto wait_page = [&](int i) __attribute__((always_inline)) {
        const int ahead = min(NBUF - 2, n - 1 - i);
        static_for<0, NBUF - 1>([&](auto k) {
            if (ahead == decltype(k)::value) wait_vmcnt<decltype(k)::value * CPW>();
        });
    };
    // Step i: wait for this wave's share of page i, meet the other waves
    // (page i complete, page i-1 consumed), refill the consumed buffer with
    // page i+NBUF-1, then consume page i.
    auto step = [&](int i, auto b) __attribute__((always_inline)) {
        constexpr int B = decltype(b)::value;   // i % NBUF
        wait_page(i);
        ring_barrier();
        if (i + NBUF - 1 < n) stage(p0 + i + NBUF - 1, ring[(B + NBUF - 1) % NBUF]);
        if (computes) compute(p0 + i, ring[B]);
    };

    // PREP, first split: new key w prepared in the prologue (fp16, as the
    // cache holds it), attended to as a block of its own and appended after
    // the partials.
    [[maybe_unused]] _Float16 new_k[4] = {}, new_v[4] = {};
    if constexpr (PREP) {
      if (n > 0) {
        constexpr int G = kModelQHeads / kModelKvHeads;
        const bool preps = w < a.tok.tokens;                  // wave-uniform
        float xq[G][4] = {}, gq[4] = {};
        NewKeyRow nk = {};
        if (preps) {
            const float *src = a.tok.q_gate + ((size_t)w * a.q_heads + (size_t)h * G) * 2 * D + lane;
#pragma unroll
            for (int r = 0; r < G; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i) global_load4(xq[r][i], src + r * 2 * D + 64 * i);
#pragma unroll
            for (int i = 0; i < 4; ++i) global_load4(gq[i], a.tok.q_norm + 64 * i + lane);
            if (split == 0) {
                const size_t krow = ((size_t)w * a.kv_heads + h) * D + lane;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    global_load4(nk.k[0][i], a.tok.key + krow + 64 * i);
                    global_load4(nk.g[i], a.tok.k_norm + 64 * i + lane);
                    global_load4(nk.v[i], a.tok.value + krow + 64 * i);
                }
            }
        }
        static_for<0, NBUF - 1>([&](auto k) {
            if (decltype(k)::value < n) stage(p0 + decltype(k)::value, ring[decltype(k)::value]);
        });
        if (preps) {
            float c = 1.f, sn = 0.f;
            if (lane < 32) rope_cos_sin(a.tok.position + w, rope_freq(lane), c, sn);
            // The inputs were requested before this wave's pages.
            const int pages = min(n, NBUF - 1);
            static_for<1, NBUF>([&](auto k) {
                if (pages == decltype(k)::value) wait_vmcnt<decltype(k)::value * CPW>();
            });
#pragma unroll
            for (int r = 0; r < G; ++r) pin(xq[r][0], xq[r][1], xq[r][2], xq[r][3]);
            pin(gq[0], gq[1], gq[2], gq[3]);
            const float cr[G] = {c, c, c, c, c, c}, sr[G] = {sn, sn, sn, sn, sn, sn};
            norm_rope_rows<G>(xq, gq, cr, sr, a.tok.epsilon, lane);
            const uint32_t qw = lds_addr(qarea) + ((G * w) * QSTRIDE + lane) * 4;
#pragma unroll
            for (int r = 0; r < G; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i) lds_write4(qw + (r * QSTRIDE + 64 * i) * 4, xq[r][i]);
            if (split == 0) {
                pin(nk.k[0][0], nk.k[0][1], nk.k[0][2], nk.k[0][3], nk.g[0], nk.g[1], nk.g[2], nk.g[3],
                    nk.v[0], nk.v[1], nk.v[2], nk.v[3]);
                const float kc[1] = {c}, ksn[1] = {sn};
                norm_rope_rows<1>(nk.k, nk.g, kc, ksn, a.tok.epsilon, lane);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    new_k[i] = cache_half(nk.k[0][i]);
                    new_v[i] = cache_half(nk.v[i]);
                }
                // Key w of the new-key block in ring buffer NBUF-1 (free
                // until page NBUF-1 is requested after step 0's barrier).
                const uint32_t nb = lds_addr(ring[NBUF - 1]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    lds_write2(nb + k_page_offset(w, 64 * i + lane, D) * 2, new_k[i]);
                    lds_write2(nb + (PAGE + v_page_offset(w, 64 * i + lane, D)) * 2, new_v[i]);
                }
            }
        }
        if (split == 0) {
            // The block's other V slots of keys 0..15 (the first key half,
            // the only one that attends to it) are zero: its masked keys'
            // P of 0 must not meet stale LDS bits.  Their K slots may hold
            // anything: those scores are masked.
            const uint32_t nv = lds_addr(ring[NBUF - 1]) + PAGE * 2;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lds_write2(nv + v_page_offset(w + 8, 64 * i + lane, D) * 2, (_Float16)0.f);
                if (!preps) lds_write2(nv + v_page_offset(w, 64 * i + lane, D) * 2, (_Float16)0.f);
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
        ring_barrier();
        if (computes) {
            // The tile's fp32 fragments (k-step ks: dims 32ks + 8g .. +7 of
            // row `row`, two float4), split into hi + lo parts, in two rounds
            // of eight LDS reads.
            const uint32_t qb = lds_addr(qarea) + (row * QSTRIDE + 8 * g) * 4;
            static_for<0, 2>([&](auto half_) {
                constexpr int K0 = decltype(half_)::value * KS / 2;
                f32x4 fa[KS / 2][2];
                static_for<0, KS / 2>([&](auto k_) {
                    constexpr int k = decltype(k_)::value;
                    lds_read<(K0 + k) * 128>(fa[k][0], qb);
                    lds_read<(K0 + k) * 128 + 16>(fa[k][1], qb);
                });
                static_for<0, KS / 2>([&](auto k_) {
                    constexpr int k = decltype(k_)::value;
                    lds_wait<2 * (KS / 2 - 1 - k)>(fa[k][0], fa[k][1]);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float x = fa[k][e / 4][e % 4];
                        const _Float16 hi = (_Float16)x;
                        qf[K0 + k][e] = hi;
                        qlo[K0 + k][e] = (_Float16)(x - (float)hi);
                    }
                });
            });
            // First split: the new keys n_keys + j, row t seeing j <= t.
            if (split == 0 && kt == 0)
                attend(a.n_keys, ring[NBUF - 1], a.n_keys + t, a.n_keys + min(16 * qt, a.rows - 1) / a.group, false);
        }
        // Page 0 has landed (pages 1 .. NBUF-2 may stay in flight).
        {
            const int ahead = min(NBUF - 2, n - 1);
            static_for<0, NBUF - 1>([&](auto k) {
                if (ahead == decltype(k)::value) wait_vmcnt<decltype(k)::value * CPW>();
            });
        }
        ring_barrier();
        if (NBUF - 1 < n) stage(p0 + NBUF - 1, ring[NBUF - 1]);
        if (computes) compute(p0, ring[0]);
        for (int i = 1; i < n; i += NBUF) {
            static_for<0, NBUF>([&](auto k) {
                constexpr int B = (decltype(k)::value + 1) % NBUF;
                if (i + decltype(k)::value < n) step(i + decltype(k)::value, std::integral_constant<int, B>{});
            });
        }
      }
    } else if (n > 0) {
        // Pages 0 .. NBUF-2 (NBUF-3 with a precise query, whose lo parts
        // occupy buffer NBUF-2) are requested after the query fragments.
        constexpr int FIRST = QSPLIT ? NBUF - 2 : NBUF - 1;
        static_for<0, FIRST>([&](auto k) {
            if (decltype(k)::value < n) stage(p0 + decltype(k)::value, ring[decltype(k)::value]);
        });
        // Step 0: page 0 and the query fragments (loaded first) have landed;
        // the fragments move to registers before the last buffers are
        // refilled with pages.
        {
            const int ahead = min(FIRST - 1, n - 1);
            static_for<0, FIRST>([&](auto k) {
                if (ahead == decltype(k)::value) wait_vmcnt<decltype(k)::value * CPW>();
            });
        }
        ring_barrier();
        if (computes) {
            const uint32_t qbase = lds_addr(ring[NBUF - 1]) + qt * KS * 1024 + lane * 16;
            static_for<0, KS>([&](auto ks) {
                lds_read<decltype(ks)::value * 1024>(qf[decltype(ks)::value], qbase);
            });
            if constexpr (QSPLIT) {
                const uint32_t lbase = lds_addr(ring[NBUF - 2]) + qt * KS * 1024 + lane * 16;
                static_for<0, KS>([&](auto ks) {
                    lds_read<decltype(ks)::value * 1024>(qlo[decltype(ks)::value], lbase);
                });
                static_for<0, KS>([&](auto ks) { lds_wait<0>(qlo[decltype(ks)::value]); });
            }
            static_for<0, KS>([&](auto ks) { lds_wait<0>(qf[decltype(ks)::value]); });
        }
        ring_barrier();
        static_for<FIRST, NBUF>([&](auto k) {
            if (decltype(k)::value < n) stage(p0 + decltype(k)::value, ring[decltype(k)::value]);
        });
        if (computes) compute(p0, ring[0]);
        for (int i = 1; i < n; i += NBUF) {
            static_for<0, NBUF>([&](auto k) {
                constexpr int B = (decltype(k)::value + 1) % NBUF;
                if (i + decltype(k)::value < n) step(i + decltype(k)::value, std::integral_constant<int, B>{});
            });
        }
    }

    if constexpr (PREP) {
        // First split: new key and value w appended to the pages, issued as
        // soon as the page loop is done (no load is in flight any more), so
        // the stores overlap the merge below.  Keys past n_keys-1 are masked
        // in every split (scores) and their V slots zeroed, so a split that
        // streams the page receiving them reads either bits harmlessly.
        if (split == 0 && n > 0 && w < a.tok.tokens) {
            _Float16 *kp = static_cast<_Float16 *>(a.tok.k_pages) + (size_t)h * a.tok.head_stride;
            _Float16 *vp = static_cast<_Float16 *>(a.tok.v_pages) + (size_t)h * a.tok.head_stride;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kp[k_page_offset(a.tok.position + w, 64 * i + lane, D)] = new_k[i];
                vp[v_page_offset(a.tok.position + w, 64 * i + lane, D)] = new_v[i];
            }
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
        if (OUT != kOutPartials && r < a.rows) {
            // The only split of this KV head: the final rows.  Every row sees
            // key 0, so L > 0.  Lane group g holds dims 4g..4g+3 of every
            // 16-dim tile.
            const int t = r / a.group, head = h * a.group + (r - t * a.group);
            const size_t hrow = (size_t)t * a.q_heads + head;       // [token][head] row
            const size_t orow = hrow * D + 4 * g;                   // out: rows of D
            const float inv = 1.f / (l * f0 + l1 * f1);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const f32x4 o1 = *reinterpret_cast<const f32x4 *>(xacc + (dt * kWave + lane) * 4);
                const f32x4 o = (acc[dt] * f0 + o1 * f1) * inv;
                if constexpr (OUT == kOutSame) {
                    const V4 v = {(KV)o[0], (KV)o[1], (KV)o[2], (KV)o[3]};
                    *reinterpret_cast<V4 *>(static_cast<KV *>(a.out) + orow + dt * 16) = v;
                } else {
                    *reinterpret_cast<f32x4 *>(static_cast<float *>(a.out) + orow + dt * 16) = o;
                }
            }
        } else if (OUT == kOutPartials && r < a.rows) {
            float *pml = a.part_ml + ((size_t)h * a.splits + split) * 2 * a.rows;
            const size_t prow = (((size_t)h * a.splits + split) * a.rows + r) * D + 4 * g;
            const float L = l * f0 + l1 * f1;
            if (lane < 16) {
                pml[r] = M;
                pml[a.rows + r] = L;
            }
            if constexpr (HALF) {
                // O / L is a convex combination of the split's V rows, so it
                // lies within their range and fp16 holds it to 2^-11
                // relative.  A row that sees none of the split's keys (a
                // split of candidate keys only) has L = 0 and stores zeros.
                const float inv = L > 0.f ? 1.f / L : 0.f;
                // Lane group g holds dims 4g..4g+3 of every 16-dim tile.
                // For each pair of tiles (dt0, dt0+1) the groups g and g^1
                // swap halves (permlane16_swap exchanges lane groups 0<->1
                // and 2<->3), so that every lane holds 8 consecutive dims:
                // group 0 dims 0-7 of dt0, group 2 dims 8-15 of dt0, groups
                // 1 and 3 the same of dt0+1.  Each store then writes 16 B
                // per lane and 64 contiguous bytes per row.
                _Float16 *po = static_cast<_Float16 *>(static_cast<void *>(a.part_o)) +
                               (prow - 4 * g) + 16 * (g & 1) + 4 * (g & 2);
                auto half4 = [&](int dt) __attribute__((always_inline)) {
                    const f32x4 o1 = *reinterpret_cast<const f32x4 *>(xacc + (dt * kWave + lane) * 4);
                    const f32x4 o = (acc[dt] * f0 + o1 * f1) * inv;
                    const f16x4 v = {(_Float16)o[0], (_Float16)o[1], (_Float16)o[2], (_Float16)o[3]};
                    return __builtin_bit_cast(u32x2, v);
                };
#pragma unroll
                for (int dt = 0; dt < DT; dt += 2) {
                    const u32x2 x = half4(dt), y = half4(dt + 1);
                    const auto s0 = __builtin_amdgcn_permlane16_swap(x[0], y[0], false, false);
                    const auto s1 = __builtin_amdgcn_permlane16_swap(x[1], y[1], false, false);
                    const u32x4 v = {s0[0], s1[0], s0[1], s1[1]};
                    __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(po + dt * 16));
                }
            } else {
                float *po = a.part_o + prow;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    const f32x4 o1 = *reinterpret_cast<const f32x4 *>(xacc + (dt * kWave + lane) * 4);
                    __builtin_nontemporal_store(acc[dt] * f0 + o1 * f1, reinterpret_cast<f32x4 *>(po + dt * 16));
                }
            }
        }
    }
}

// Instances: raw fp16 multiplies V by a 16-bit P, raw bf16 by hi + lo P
// (bf16's 8-bit significand alone would dominate the error), and fp32
// queries (hi + lo fp16 parts) by hi + lo P as well.
template <int D, int NQT, int OUT>
const void *pick(Dtype dtype, bool precise) {
    if (precise) {
        if constexpr (OUT == kOutSame) return nullptr;
        else return dtype == Dtype::F16 ? (const void *)&attention_ring<D, NQT, true, _Float16, true, OUT> : nullptr;
    }
    if (dtype == Dtype::BF16) return (const void *)&attention_ring<D, NQT, true, __bf16, false, OUT>;
    return (const void *)&attention_ring<D, NQT, false, _Float16, false, OUT>;
}

template <int D, int NQT>
const void *pick_out(Dtype dtype, bool precise, int out_mode) {
    switch (out_mode) {
        case kOutPartials: return pick<D, NQT, kOutPartials>(dtype, precise);
        case kOutSame: return pick<D, NQT, kOutSame>(dtype, precise);
        case kOutF32: return pick<D, NQT, kOutF32>(dtype, precise);
    }
    return nullptr;
}

template <int D>
const void *pick_tiles(int nqt, Dtype dtype, bool precise, int out_mode) {
    switch (nqt) {
        case 1: return pick_out<D, 1>(dtype, precise, out_mode);
        case 2: return pick_out<D, 2>(dtype, precise, out_mode);
        case 3: return pick_out<D, 3>(dtype, precise, out_mode);
    }
    return nullptr;
}

}  // namespace

const void *ring_kernel(int D, int nqt, Dtype dtype, bool precise, int out_mode) {
    if (D == 256) return pick_tiles<256>(nqt, dtype, precise, out_mode);
    if (D == 128) return pick_tiles<128>(nqt, dtype, precise, out_mode);
    return nullptr;
}

const void *ring_prep_kernel(int nqt) {
    constexpr int D = kModelHeadDim;
    switch (nqt) {
        case 2: return (const void *)&attention_ring<D, 2, true, _Float16, true, kOutPartials, true>;
        case 3: return (const void *)&attention_ring<D, 3, true, _Float16, true, kOutPartials, true>;
    }
    return nullptr;
}

}  // namespace rs
