// GQA attention over the paged KV cache: split-K partial kernels (decode and
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
// (see the V page layout in common.hpp).
//
// Two partial kernels share that arithmetic:
//   attention_stream  one query tile (<= 16 rows, decode).  Every wave streams
//                     its own run of pages with a private softmax state; the
//                     four waves merge through LDS once at the end (one
//                     barrier: each wave's state in its own slot).
//   attention_ring    (ring.hip) 17..48 rows (verification): eight waves
//                     share a ring of LDS page buffers filled by direct
//                     global->LDS loads.
#include "combine.hpp"
#include "kernels.hpp"
#include "prep.hpp"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>
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

constexpr int kWaves = 4;          // waves per workgroup of the partial kernels
constexpr int kMaxSplits = 1024;   // bound on workgroups per KV head

// Query fragments (B operand of S^T): fragment (i, qt, ks) of lane l holds
// row 16*qt + l%16, dims 32*ks + 8*(l/16) .. +7 of the hi (i = 0) or lo (i = 1,
// QSPLIT) part.  A fp32 query arrives split into hi + lo 16-bit parts; the two
// MFMAs carry ~22 significant bits, which keeps the fused path at fp32
// accuracy.  Rows past `rows` repeat the last row; their results are never
// stored.
//
// Every workgroup needs every fragment, and all of them start at once, so the
// loads are shared: wave w fetches fragments w, w+4, ... (issue), the kernel
// then issues its first KV loads, and only afterwards waits for the query
// (publish: vector-memory counters retire in issue order, so that wait does
// not drain the KV loads) and hands the fragments over through LDS.
//
// F32: a.q holds the fp32 query itself, and publish splits each loaded
// fragment into its hi and lo parts (hi = fp16(q), lo = fp16(q - hi): the
// rounding of the query split kernel, so the same bits), which saves the
// split kernel's launch.
template <int D, int NQT, bool QSPLIT, typename KV, bool F32 = false>
struct QueryStage {
    using V8 = typename Vec8<KV>::type;
    static constexpr int KS = D / 32, NQ = QSPLIT ? 2 : 1, N = NQ * NQT * KS;
    static constexpr int NL = F32 ? NQT * KS : N;    // fragments loaded
    static constexpr int PER = NL / kWaves;
    static_assert(NL % kWaves == 0, "fragments divide evenly over the waves");
    static_assert(!F32 || (QSPLIT && std::is_same<KV, _Float16>::value), "an fp32 query splits into fp16 parts");
    V8 part[F32 ? 1 : PER];
    f32x4 part32[F32 ? PER : 1][2];

    __device__ __forceinline__ void issue(const SplitArgs &a, int h, int lane, int w) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = w + kWaves * i;
            const int ks = e % KS, qt = (e / KS) % NQT, lo = e / (KS * NQT);
            const int row = min(16 * qt + (lane & 15), a.rows - 1);
            const int t = row / a.group, gg = row - t * a.group;
            const size_t at = ((size_t)t * a.q_heads + (size_t)h * a.group + gg) * D + 32 * ks + 8 * (lane >> 4);
            if constexpr (F32) {
                const f32x4 *src = reinterpret_cast<const f32x4 *>(static_cast<const float *>(a.q) + at);
                part32[i][0] = src[0];
                part32[i][1] = src[1];
            } else {
                part[i] = *reinterpret_cast<const V8 *>(static_cast<const KV *>(lo ? a.q_lo : a.q) + at);
            }
        }
    }
    __device__ __forceinline__ void publish(V8 *sq, int lane, int w) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if constexpr (F32) {
                // Fragment e's hi part is fragment e, its lo part e + NQT*KS.
                V8 hi, lo;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float x = part32[i][j >> 2][j & 3];
                    hi[j] = (KV)x;
                    lo[j] = (KV)(x - (float)hi[j]);
                }
                sq[(w + kWaves * i) * kWave + lane] = hi;
                sq[(NQT * KS + w + kWaves * i) * kWave + lane] = lo;
            } else {
                sq[(w + kWaves * i) * kWave + lane] = part[i];
            }
        }
    }
    // After an LDS barrier: all fragments into registers.
    static __device__ __forceinline__ void gather(const V8 *sq, int lane, V8 (&qf)[NQ][NQT][KS]) {
#pragma unroll
        for (int i = 0; i < NQ; ++i)
#pragma unroll
            for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) qf[i][qt][ks] = sq[((i * NQT + qt) * KS + ks) * kWave + lane];
    }
};

// Token held in slot j of a V^T operand by lane group g (see common.hpp).
__device__ __forceinline__ int v_slot_token(int g, int j) {
    return j < 4 ? 4 * g + j : 16 + 4 * g + j - 4;
}

// ---------------------------------------------------------------------------
// attention_stream: one query tile; wave-private online softmax over a run of
// pages, merged across the four waves through LDS at the end.  Keys past
// n_keys in the last page are masked (scores) and zeroed (values), so stale
// page contents never reach the result.  Page loads are non-temporal (each
// byte is touched once): at 139,264 keys the kernel takes 86 us that way
// against 95.5 us with default loads.  The partial stores (a few KiB per
// workgroup) keep the default policy, and the combine loads them the same
// way: that pair takes 0.5 us less per decode layer than non-temporal
// stores and loads.
// ---------------------------------------------------------------------------
//
// PREP (the fused path's new tokens, 1 or 2 of them, group 6): the query is
// not read from q but prepared here from a.tok (RMSNorm, gamma, RoPE, hi +
// lo fp16 parts; the same functions as the prepare kernel, so the same bits)
// while the first K page is in flight: wave w prepares rows 3w .. 3w+2, three
// query heads of token w/2.  Every row sees the cached keys 0 .. a.position
// only.  The first split's workgroups also store the prepared rows in
// a.tok.q_prep and prepare and append the new keys (wave j: token j), which
// the combine adds.
//
// OUT: kOutPartials stores the split's partial rows; a direct output
// (kOutSame or kOutF32: one split per KV head) stores the final rows
// instead, and no combine runs.
template <int D, bool QSPLIT, bool PSPLIT, typename KV, bool PREP, int OUT = kOutPartials>
__global__ __launch_bounds__(kWaves * kWave)
void attention_stream(SplitArgs a) {
    using V8 = typename Vec8<KV>::type;
    // A precise raw call passes its fp32 query as it is (the split kernels'
    // other precise callers prepare theirs: PREP).
    using QS = QueryStage<D, 1, QSPLIT, KV, QSPLIT && !PREP>;
    constexpr int KS = D / 32, DT = D / 16, NQ = QSPLIT ? 2 : 1;
    static_assert(!PREP || (D == kModelHeadDim && D == 4 * kWave && QSPLIT && std::is_same<KV, _Float16>::value),
                  "the prepared query is the fp32 query of the 256-dim fp16 model, as hi + lo parts");
    __shared__ f32x4 so[kWaves][DT * kWave];   // merge slots, one per wave
    __shared__ V8 sq[QS::N * kWave];       // query fragments
    __shared__ float sml[kWaves][2][16];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int split = blockIdx.x % a.splits, h = blockIdx.x / a.splits;
    QS qs;
    // PREP: rows 3w + r of token w/2 (lane l holding dims 64i + l), and the
    // new key of token w in the first split.
    constexpr int PR = 3;
    float xq[PR][4], gq[4];
    NewKeyRow nk;
    const int ptok = w >> 1;
    const bool prows = PREP && ptok < a.tok.tokens;               // wave-uniform
    const bool pkey = PREP && split == 0 && w < a.tok.tokens;     // wave-uniform
    if constexpr (PREP) {
        if (prows) {
#pragma unroll
            for (int r = 0; r < PR; ++r) {
                const float *src = a.tok.q_gate + ((size_t)ptok * a.q_heads + h * a.group + 3 * (w & 1) + r) * 2 * D;
#pragma unroll
                for (int i = 0; i < 4; ++i) xq[r][i] = src[64 * i + lane];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) gq[i] = a.tok.q_norm[64 * i + lane];
        }
        if (pkey) load_new_key(nk, a.tok, a.kv_heads, h, w, lane);
    } else {
        qs.issue(a, h, lane, w);
    }

    // Pages are dealt out round-robin over the waves of all splits of this
    // head: step j of wave wi is page j*waves_total + wi, so waves running in
    // step stream one contiguous stretch of the head.
    const int waves_total = a.splits * kWaves;
    const int wi = split * kWaves + w;
    const int n_steps = wi < a.n_pages ? (a.n_pages - 1 - wi) / waves_total + 1 : 0;
    const KV *kh = static_cast<const KV *>(a.k_pages) + (size_t)h * a.head_stride + lane * 8;
    const KV *vh = static_cast<const KV *>(a.v_pages) + (size_t)h * a.head_stride + lane * 8;
    const int limit = a.position + (PREP ? 0 : min(lane & 15, a.rows - 1) / a.group);   // last visible key

    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;

    V8 qf1[NQ][1][KS];
    V8 kb[2][KS];
    auto load_k = [&](int b) {
        const KV *kp = kh + (size_t)b * 32 * D;
#pragma unroll
        for (int tile = 0; tile < 2; ++tile)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                kb[tile][ks] = __builtin_nontemporal_load(reinterpret_cast<const V8 *>(kp + tile * 16 * D + ks * 512));
    };
    // One page; with PREFETCH the next page's K is loaded into kb once the
    // scores no longer need it.  The last page runs without it, so every
    // path issues the same loads.
    auto page = [&](int b, auto prefetch) {
        // V of this page is in flight while the scores are computed.
        V8 vb[DT];
        const KV *vp = vh + (size_t)b * 32 * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) vb[dt] = __builtin_nontemporal_load(reinterpret_cast<const V8 *>(vp + dt * 512));

        f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            s0 = mfma(kb[0][ks], qf1[0][0][ks], s0);
            s1 = mfma(kb[1][ks], qf1[0][0][ks], s1);
            if constexpr (QSPLIT) {
                s0 = mfma(kb[0][ks], qf1[NQ - 1][0][ks], s0);
                s1 = mfma(kb[1][ks], qf1[NQ - 1][0][ks], s1);
            }
        }
        if constexpr (decltype(prefetch)::value) load_k(b + waves_total);

        // Lane l holds keys b*32 + 16*tile + 4*(l/16) + r, r < 4.
        const int key0 = b * 32 + 4 * (lane >> 4);
        float x[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            x[r] = s0[r] * a.scale_log2;
            x[4 + r] = s1[r] * a.scale_log2;
        }
        // Keys past a row's last visible key score -inf.  The fused decode
        // (PREP) relies on this mask and on the value zeroing below: the
        // first split appends the new key and value at key `position + 1`
        // of the page it streams while other workgroups read that page,
        // and every PREP row's limit is `position` (the last cached key,
        // n_keys = position + 1), so whatever such a read returns for that
        // slot is masked here and its value zeroed.  A change to either
        // mask (or to which keys the split covers) must keep that slot
        // invisible.
        if (b * 32 + 31 > a.position) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (key0 + 16 * (j >> 2) + (j & 3) > limit) x[j] = -INFINITY;
        }
        float bm = x[0];
#pragma unroll
        for (int j = 1; j < 8; ++j) bm = fmaxf(bm, x[j]);
        bm = fmaxf(bm, __shfl_xor(bm, 16, kWave));
        bm = fmaxf(bm, __shfl_xor(bm, 32, kWave));
        const float mn = fmaxf(m, bm);
        const float mu = mn == -INFINITY ? 0.f : mn;   // fully masked so far
        const float alpha = exp2f(m - mu);
        m = mn;
        V8 ph, pl;
        float ps = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float e = exp2f(x[j] - mu);
            const KV eh = (KV)e;
            ph[j] = eh;
            if constexpr (PSPLIT) {
                pl[j] = (KV)(e - (float)eh);
                ps += e;
            } else {
                ps += (float)eh;   // normalise by the weights actually applied
            }
        }
        l = l * alpha + ps;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
        if (b * 32 + 32 > a.n_keys) {
            // Zero V slots past the last key: 0 * (stale NaN) would poison O.
            // (The fused decode's appended value sits in such a slot.)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (b * 32 + v_slot_token(lane >> 4, j) >= a.n_keys) {
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) vb[dt][j] = (KV)0.f;
                }
            }
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            acc[dt] = mfma(vb[dt], ph, acc[dt]);
            if constexpr (PSPLIT) acc[dt] = mfma(vb[dt], pl, acc[dt]);
        }
    };

    // The first K load is unconditional (a wave without pages re-reads the
    // head's last page), so every wave issues it before waiting on the query.
    load_k(min(wi, a.n_pages - 1));
    // PREP: the prepared rows are staged in LDS as fp32, row-major with a
    // stride of D + 4 floats, in the query-fragment buffer (which PREP does
    // not otherwise use, and which nothing writes after the gather), so the
    // writes (lane l: dims 64i + l) and the fragment reads (16 rows, 32
    // bytes each) are both free of bank conflicts; hi and lo parts are split
    // while gathering.
    constexpr int kStage = D + 4;
    static_assert(!PREP || kWaves * PR * kStage * sizeof(float) <= sizeof(sq), "the staged rows fit the query buffer");
    float *stage = reinterpret_cast<float *>(sq);
    if constexpr (PREP) {
        const double freq = rope_freq(lane);
        if (prows) {
            float c = 1.f, sn = 0.f;
            if (lane < 32) rope_cos_sin(a.tok.position + ptok, freq, c, sn);
            const float cr[PR] = {c, c, c}, sr[PR] = {sn, sn, sn};
            norm_rope_rows<PR>(xq, gq, cr, sr, a.tok.epsilon, lane);
#pragma unroll
            for (int r = 0; r < PR; ++r) {
                const int row = 3 * w + r;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    stage[row * kStage + 64 * i + lane] = xq[r][i];
                    if (split == 0) a.tok.q_prep[((size_t)h * a.rows + row) * D + 64 * i + lane] = xq[r][i];
                }
            }
        }
        if (pkey) {
            float c = 1.f, sn = 0.f;
            if (lane < 32) rope_cos_sin(a.tok.position + w, freq, c, sn);
            append_new_key(nk, a.tok, h, w, c, sn, lane);
        }
    } else {
        qs.publish(sq, lane, w);
    }
    lds_barrier();
    if constexpr (PREP) {
        // Fragment ks of lane l: row l%16, dims 32ks + 8(l/16) .. +7, as
        // hi = fp16(q) and lo = fp16(q - hi).  Rows past the group are zero
        // (their results are never stored).
        const int row = lane & 15;
        const bool live = row < a.rows;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const float *src = stage + row * kStage + 32 * ks + 8 * (lane >> 4);
            const f32x4 lo4 = live ? *reinterpret_cast<const f32x4 *>(src) : f32x4{0.f, 0.f, 0.f, 0.f};
            const f32x4 hi4 = live ? *reinterpret_cast<const f32x4 *>(src + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = j < 4 ? lo4[j] : hi4[j - 4];
                const _Float16 hi = (_Float16)x;
                qf1[0][0][ks][j] = hi;
                qf1[NQ - 1][0][ks][j] = (_Float16)(x - (float)hi);
            }
        }
    } else {
        QS::gather(sq, lane, qf1);
    }
    if (n_steps > 0) {
        for (int j = 0; j + 1 < n_steps; ++j) page(j * waves_total + wi, std::true_type{});
        page((n_steps - 1) * waves_total + wi, std::false_type{});
    }

    // ---- merge the waves of this workgroup -------------------------------
    // One barrier: every wave leaves its (m, l) and its unscaled
    // accumulators in its own LDS slot; then every thread merges the four
    // slots of its output elements (row-major, D contiguous floats per row,
    // so each store instruction writes whole rows).  Element (row, 4*d4 ..
    // +3) is the f32x4 of lane (row%16) + 16*(d4%4) in fragment d4/4.
    l += __shfl_xor(l, 16, kWave);
    l += __shfl_xor(l, 32, kWave);
    if (lane < 16) {
        sml[w][0][lane] = m;
        sml[w][1][lane] = l;
    }
    // Only the rows that exist are merged (decode: 6 of the tile's 16).
    if ((lane & 15) < a.rows) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) so[w][dt * kWave + lane] = acc[dt];
    }
    lds_barrier();
    if (OUT == kOutPartials && w == 0 && lane < a.rows && lane < 16) {
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, sml[ww][0][lane]);
        const float mu = M == -INFINITY ? 0.f : M;
        float L = 0.f;
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) L += sml[ww][1][lane] * exp2f(sml[ww][0][lane] - mu);
        float *pml = a.part_ml + ((size_t)h * a.splits + split) * 2 * a.rows;
        pml[lane] = M;
        pml[a.rows + lane] = L;
    }
    f32x4 *po = reinterpret_cast<f32x4 *>(a.part_o + ((size_t)h * a.splits + split) * a.rows * D);
    for (int e = threadIdx.x; e < a.rows * (D / 4); e += kWaves * kWave) {
        const int r = e / (D / 4), d4 = e - r * (D / 4);
        const int idx = (d4 >> 2) * kWave + r + 16 * (d4 & 3);
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, sml[ww][0][r]);
        const float mu = M == -INFINITY ? 0.f : M;
        f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) o += so[ww][idx] * exp2f(sml[ww][0][r] - mu);
        if constexpr (OUT == kOutPartials) {
            po[e] = o;
        } else {
            // The only split of this KV head: the final row (every row sees
            // key 0, so L > 0).
            float L = 0.f;
#pragma unroll
            for (int ww = 0; ww < kWaves; ++ww) L += sml[ww][1][r] * exp2f(sml[ww][0][r] - mu);
            o *= 1.f / L;
            const int t = r / a.group;
            const size_t hrow = (size_t)t * a.q_heads + h * a.group + (r - t * a.group);
            if constexpr (OUT == kOutSame) {
                typedef KV KV4 __attribute__((ext_vector_type(4)));
                const KV4 v = {(KV)o[0], (KV)o[1], (KV)o[2], (KV)o[3]};
                *reinterpret_cast<KV4 *>(static_cast<KV *>(a.out) + hrow * D + 4 * d4) = v;
            } else {
                *reinterpret_cast<f32x4 *>(static_cast<float *>(a.out) + hrow * D + 4 * d4) = o;
            }
        }
    }
}

struct CombineArgs {
    const void *part_o;   // float or _Float16 rows (SplitPlan::half_parts)
    const float *part_ml;
    void *out;
    const float *gate;   // gated output: q_gate rows of 2*D floats, gate at +D
    int q_heads, group, rows, splits;
    float scale_log2;     // NEWKEY: the new keys' score scale
    FusedToken tok;       // NEWKEY: the new tokens
};

// Standalone combine: one workgroup (4 waves) per (row, KV head), or with
// QD > 1 one per (row, KV head, QD-th of the head dims): blockIdx.z.
// Plans of at most kCombineSplitRows rows per KV head (decode) take QD =
// D / 64, so that each workgroup loads a quarter of the row's partials
// (decode at 139,264 keys 86.07 -> 85.88 us per layer, at 4,096 10.47 ->
// 10.28; medians of 3 in-process rounds).  Verification keeps whole rows:
// four times its 192 workgroups measured slower (19.80 -> 20.12 us).
template <int D, typename KV, int OUT, typename PT, bool NT, bool NEWKEY, int QD = 1>
__global__ __launch_bounds__(kWaves * kWave)
void attention_combine(CombineArgs c) {
    __shared__ float scratch[4 * (D / QD + 1) + 4];
    combine_row<D, KV, PT, NT, NEWKEY, QD>(static_cast<const PT *>(c.part_o), c.part_ml, c.splits, c.rows, c.group,
                                           c.q_heads, blockIdx.x, blockIdx.y, true, threadIdx.x >> 6, threadIdx.x & 63,
                                           scratch, c.out, c.gate, OUT, &c.tok, c.scale_log2, blockIdx.z);
}
constexpr int kCombineSplitRows = 16;

// attention_stream instance: raw fp16 multiplies V by a 16-bit P; raw bf16
// by hi + lo P (bf16's 8-bit significand alone would dominate the error); a
// precise query (fp32 as fp16 hi + lo parts) takes hi + lo P as well.
template <int D, int OUT>
const void *stream_kernel(Dtype dtype, bool precise) {
    if (precise) {
        if constexpr (OUT == kOutSame) return nullptr;
        else return dtype == Dtype::F16 ? (const void *)&attention_stream<D, true, true, _Float16, false, OUT> : nullptr;
    }
    if (dtype == Dtype::BF16) return (const void *)&attention_stream<D, false, true, __bf16, false, OUT>;
    return (const void *)&attention_stream<D, false, false, _Float16, false, OUT>;
}

template <int D>
const void *stream_kernel(Dtype dtype, bool precise, int out_mode) {
    switch (out_mode) {
        case kOutPartials: return stream_kernel<D, kOutPartials>(dtype, precise);
        case kOutSame: return stream_kernel<D, kOutSame>(dtype, precise);
        case kOutF32: return stream_kernel<D, kOutF32>(dtype, precise);
    }
    return nullptr;
}

template <int D, typename PT, bool NT, int QD>
const void *combine_kernel(Dtype dtype, bool out_f32, bool gated) {
    if (gated) return (const void *)&attention_combine<D, _Float16, kOutGated, PT, NT, false, QD>;
    if (out_f32) return (const void *)&attention_combine<D, _Float16, kOutF32, PT, NT, false, QD>;
    return dtype == Dtype::BF16 ? (const void *)&attention_combine<D, __bf16, kOutSame, PT, NT, false, QD>
                                : (const void *)&attention_combine<D, _Float16, kOutSame, PT, NT, false, QD>;
}

// fp16 partial rows come only from the ring kernel, which stores them
// non-temporally; fp32 ones are non-temporal from the ring kernel and
// default-policy from attention_stream.
template <int D, int QD>
const void *combine_kernel(Dtype dtype, bool out_f32, bool gated, bool half_parts, bool nt_parts) {
    if (half_parts) return combine_kernel<D, _Float16, true, QD>(dtype, out_f32, gated);
    return nt_parts ? combine_kernel<D, float, true, QD>(dtype, out_f32, gated)
                    : combine_kernel<D, float, false, QD>(dtype, out_f32, gated);
}
template <int D>
const void *combine_kernel(Dtype dtype, bool out_f32, bool gated, bool half_parts, bool nt_parts, bool split_dims) {
    return split_dims ? combine_kernel<D, D / kWave>(dtype, out_f32, gated, half_parts, nt_parts)
                      : combine_kernel<D, 1>(dtype, out_f32, gated, half_parts, nt_parts);
}

const void *split_kernel(const SplitPlan &p, int D, Dtype dtype, bool precise, int out_mode = kOutPartials) {
    const void *k = p.kind == SplitKind::Ring ? ring_kernel(D, p.nqt, dtype, precise, out_mode)
                  : D == 256                  ? stream_kernel<256>(dtype, precise, out_mode)
                  : D == 128                  ? stream_kernel<128>(dtype, precise, out_mode)
                                              : nullptr;
    require(k != nullptr, "unsupported head_dim / query rows / output for the split kernel");
    return k;
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

int block_threads(const SplitPlan &p) {
    return p.kind == SplitKind::Stream ? kWaves * kWave : kRingThreads;
}

// Resident workgroups per CU of a kernel instance (cached per device).
int blocks_per_cu(const void *kernel, int threads) {
    static std::mutex mutex;
    static std::vector<std::pair<std::pair<int, const void *>, int>> cache;
    int device = 0;
    check(hipGetDevice(&device));
    std::lock_guard<std::mutex> lock(mutex);
    for (const auto &e : cache)
        if (e.first.first == device && e.first.second == kernel) return e.second;
    int n = 0;
    check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0));
    n = std::max(1, n);
    cache.push_back({{device, kernel}, n});
    return n;
}

SplitPlan plan_split_for(const Shape &s, int tokens, Dtype dtype, bool precise, bool allow_direct,
                         int cus, int (*resident_per_cu)(const SplitPlan &, int D, Dtype, bool)) {
    SplitPlan p;
    p.rows = s.group() * tokens;
    p.nqt = (p.rows + 15) / 16;
    // One query tile (decode) streams; several (verification) use the ring.
    p.kind = p.nqt == 1 ? SplitKind::Stream : SplitKind::Ring;
    const long long n_keys = (long long)s.position + tokens;
    p.n_pages = (int)((n_keys + kPageTokens - 1) / kPageTokens);
    p.splits = 1;
    p.half_parts = false;
    p.direct = allow_direct && p.n_pages <= (p.kind == SplitKind::Stream ? kDirectStreamPages : kDirectRingPages);
    if (p.direct) return p;
    // Fill every CU with as many workgroups as stay resident.
    const int resident = cus * resident_per_cu(p, s.head_dim, dtype, precise);
    int per_head = std::max(1, std::min(resident / s.kv_heads, kMaxSplits));
    if (p.kind == SplitKind::Stream) {
        // Decode streams fastest from three quarters of the CUs: on the
        // 139,264-key decode (4 KV heads) 48 splits per head (192
        // workgroups) take 95.5 us against 97.6 us for 64, and the combine
        // has fewer partials to merge.
        per_head = std::max(1, std::min(per_head, cus * 3 / (4 * s.kv_heads)));
        // Every wave gets at least one page on average.
        p.splits = std::max(1, std::min(per_head, (p.n_pages + kWaves - 1) / kWaves));
    } else {
        // Contiguous page runs: the longest run sets the time, so use as few
        // splits as give that same longest run (fewer partials to combine).
        const int longest = (p.n_pages + per_head - 1) / per_head;
        p.splits = (p.n_pages + longest - 1) / longest;
    }
    // The raw fp16 ring kernel stores its partial rows as fp16 O / l: half
    // the partial traffic, which every workgroup writes at once at the end.
    p.half_parts = p.kind == SplitKind::Ring && dtype == Dtype::F16 && !precise;
    return p;
}

namespace {
int resident_on_device(const SplitPlan &p, int D, Dtype dtype, bool precise) {
    return blocks_per_cu(split_kernel(p, D, dtype, precise), block_threads(p));
}
}  // namespace

SplitPlan plan_split(const Shape &s, int tokens, Dtype dtype, bool precise, bool allow_direct) {
    return plan_split_for(s, tokens, dtype, precise, allow_direct, device_cu_count(), resident_on_device);
}

size_t plan_bytes(const Shape &s, const SplitPlan &p) {
    if (p.direct) return 0;
    return (size_t)s.kv_heads * p.splits * p.rows * ((size_t)s.head_dim + 2) * sizeof(float);
}

size_t attention_workspace_bytes(const Shape &s, Dtype dtype, bool precise) {
    if (s.group() * s.tokens > kMaxRows) return prefill_workspace_bytes(s, dtype, precise);   // prefill kernel
    const int ct = chunk_tokens(s);
    size_t best = 0;
    for (int t0 = 0; t0 < s.tokens; t0 += ct) {
        Shape c = s;
        c.position = s.position + t0;
        best = std::max(best, plan_bytes(c, plan_split(c, std::min(ct, s.tokens - t0), dtype, precise)));
    }
    return best;
}

void launch_split(const Shape &s, const SplitPlan &plan, Dtype dtype, bool precise,
                  float scale, const void *q, const void *q_lo, const void *k_pages,
                  const void *v_pages, void *workspace, hipStream_t stream,
                  void *out, bool out_f32) {
    SplitArgs a = {};
    a.q = q;
    a.q_lo = q_lo;
    a.k_pages = k_pages;
    a.v_pages = v_pages;
    a.part_o = static_cast<float *>(workspace);
    a.part_ml = a.part_o ? a.part_o + (size_t)s.kv_heads * plan.splits * plan.rows * s.head_dim : nullptr;
    a.head_stride = (size_t)s.capacity * s.head_dim;
    a.q_heads = s.q_heads;
    a.kv_heads = s.kv_heads;
    a.group = s.group();
    a.rows = plan.rows;
    a.position = s.position;
    a.n_keys = s.position + plan.rows / s.group();
    a.n_pages = plan.n_pages;
    a.splits = plan.splits;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.out = out;
    // The precise stream kernel reads q as the fp32 query and splits it
    // itself; hi + lo parts (q_lo set) are for the ring and prefill kernels.
    require(!(precise && plan.kind == SplitKind::Stream && q_lo != nullptr),
            "the precise stream kernel takes the fp32 query, not its hi + lo parts");
    require(!(precise && plan.kind == SplitKind::Ring && q_lo == nullptr),
            "the precise ring kernel takes the query's hi + lo parts");
    int out_mode = kOutPartials;
    if (plan.direct) {
        require(out != nullptr && plan.splits == 1, "a direct split plan writes the output");
        out_mode = out_f32 ? kOutF32 : kOutSame;
    }
    const void *kernel = split_kernel(plan, s.head_dim, dtype, precise, out_mode);
    void *args[] = {&a};
    // One-dimensional grid: workgroup id = KV head * splits + split.
    check(hipLaunchKernel(kernel, dim3(plan.splits * s.kv_heads), dim3(block_threads(plan)),
                          args, 0, stream));
}

void launch_combine(const Shape &s, const SplitPlan &plan, Dtype dtype,
                    const void *workspace, void *out, bool out_f32, const float *gate,
                    hipStream_t stream) {
    CombineArgs c;
    c.part_o = workspace;
    c.part_ml = static_cast<const float *>(workspace) + (size_t)s.kv_heads * plan.splits * plan.rows * s.head_dim;
    c.out = out;
    c.gate = gate;
    c.q_heads = s.q_heads;
    c.group = s.group();
    c.rows = plan.rows;
    c.splits = plan.splits;
    const bool nt_parts = plan.kind != SplitKind::Stream;
    const bool split_dims = plan.rows <= kCombineSplitRows;
    const dim3 grid(plan.rows, s.kv_heads, split_dims ? s.head_dim / kWave : 1);
    const void *kernel = s.head_dim == 256 ? combine_kernel<256>(dtype, out_f32, gate != nullptr, plan.half_parts, nt_parts, split_dims)
                       : s.head_dim == 128 ? combine_kernel<128>(dtype, out_f32, gate != nullptr, plan.half_parts, nt_parts, split_dims)
                                           : nullptr;
    require(kernel != nullptr, "unsupported head_dim for the combine kernel");
    void *args[] = {&c};
    check(hipLaunchKernel(kernel, grid, dim3(kWaves * kWave), args, 0, stream));
}

namespace {
// The split plan of a fused call: rows = 6 * tokens query rows per KV head
// over the cached keys 0 .. position-1 (the shape's position is chosen so
// that position + tokens is the cached key count).
SplitPlan fused_plan(int tokens, int position) {
    const Shape s{kModelQHeads, kModelKvHeads, kModelHeadDim, tokens, position - tokens, 0};
    return plan_split(s, tokens, Dtype::F16, true);
}
}  // namespace

// The partials, then the prepared queries (fp32 [kv_heads][rows][D]).
size_t fused_prep_offset(int tokens, int position) {
    const Shape s{kModelQHeads, kModelKvHeads, kModelHeadDim, tokens, position - tokens, 0};
    return (plan_bytes(s, fused_plan(tokens, position)) + 255) & ~size_t(255);
}

size_t fused_tokens_workspace_bytes(int tokens, int position) {
    return fused_prep_offset(tokens, position) + (size_t)kModelQHeads * tokens * kModelHeadDim * sizeof(float);
}

void launch_fused_tokens(const FusedToken &tok, int capacity, void *workspace, float *out, hipStream_t stream) {
    constexpr int D = kModelHeadDim;
    const int T = tok.tokens;
    require(tok.position >= 1, "the fused split needs at least one cached key");
    require(T >= 1 && T <= kMaxFusedSplitTokens, "too many tokens for the fused split");
    const SplitPlan plan = fused_plan(T, tok.position);
    require(!plan.half_parts && plan.splits >= 1, "the fused split stores fp32 partials");
    constexpr float kScaleLog2 = (1.0f / 16.0f) * 1.4426950408889634f;
    const int kv_heads = kModelKvHeads, group = kModelQHeads / kModelKvHeads;
    require(plan.rows == group * T, "the fused split serves every query head of every token");
    FusedToken ft = tok;
    ft.q_prep = reinterpret_cast<float *>(static_cast<char *>(workspace) + fused_prep_offset(T, tok.position));

    // One or two tokens (one query tile): the stream kernel, whose first
    // split appends the new keys and publishes the prepared query rows, from
    // which the combine adds the new keys.  More: the ring kernel, whose
    // first split attends to the new keys itself and appends them.
    const bool ring = plan.kind == SplitKind::Ring;
    require(ring || plan.rows <= 12, "the prepared-query stream kernel takes one or two tokens");
    const void *split = ring ? ring_prep_kernel(plan.nqt) : (const void *)&attention_stream<D, true, true, _Float16, true>;
    require(split != nullptr, "no prepared-query ring kernel for this many tokens");

    SplitArgs a = {};
    a.k_pages = tok.k_pages;
    a.v_pages = tok.v_pages;
    a.part_o = static_cast<float *>(workspace);
    a.part_ml = a.part_o + (size_t)kv_heads * plan.splits * plan.rows * D;
    a.head_stride = tok.head_stride;
    a.q_heads = kModelQHeads;
    a.kv_heads = kv_heads;
    a.group = group;
    a.rows = plan.rows;
    a.position = tok.position - 1;   // every row sees keys 0 .. position-1
    a.n_keys = tok.position;
    a.n_pages = plan.n_pages;
    a.splits = plan.splits;
    a.scale_log2 = kScaleLog2;
    a.tok = ft;
    void *split_args[] = {&a};
    check(hipLaunchKernel(split, dim3(plan.splits * kv_heads), dim3(block_threads(plan)), split_args, 0, stream));

    CombineArgs c = {};
    c.part_o = workspace;
    c.part_ml = a.part_ml;
    c.out = out;
    c.gate = tok.q_gate;
    c.q_heads = kModelQHeads;
    c.group = group;
    c.rows = plan.rows;
    c.splits = plan.splits;
    c.scale_log2 = kScaleLog2;
    c.tok = ft;
    // The stream kernel stores its partials with the default policy, the
    // ring kernel non-temporally; the combine loads them the same way.
    // The stream kernel's rows (one or two tokens) take a workgroup per
    // quarter of the head dims, as the raw decode's combine does.
    const void *combine = ring ? (const void *)&attention_combine<D, _Float16, kOutGated, float, true, false>
                               : (const void *)&attention_combine<D, _Float16, kOutGated, float, false, true, D / kWave>;
    void *combine_args[] = {&c};
    check(hipLaunchKernel(combine, dim3(plan.rows, kv_heads, ring ? 1 : D / kWave), dim3(kWaves * kWave), combine_args,
                          0, stream));
}

}  // namespace rs
