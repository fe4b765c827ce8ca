// The fused attention of a short context in one launch: the reference's
// k_attention (src/kernels.cu:575-580: attn_prepare, then attention) for the
// 24/4/256 model when the whole context is a few pages.  There the cost is
// latency, not bandwidth: the prepare, split-K and combine launches of the
// long-context path each cost a few microseconds however little they do,
// and within this kernel every phase is a chain of dependent steps, so the
// work is spread so that each wave's chain is as short as it can be.
//
// One workgroup per (new token t, KV head h), eight waves:
//   * every load is issued first: wave w's query row (w < 6) and new key
//     and value j = w (tokens 0..t, so rows past t are not used), the norm
//     weights, the gate of this thread's output element, and cached page w;
//   * wave w prepares its query row (RMSNorm, gamma, RoPE: the prepare
//     kernel's functions) into fp16 hi + lo matrix-core fragments in LDS,
//     and its new key, rounded to fp16 as the cache holds it, into slot j of
//     a page of new keys in LDS (the page layout); the workgroup of token t
//     also appends that key and value to the cache (only it writes the slot,
//     and no workgroup reads the new slots from the cache);
//   * cached page w (w < ceil(position/32)) and the page of new keys go
//     through the matrix cores as in the split kernels (S^T = K.Q^T in four
//     independent accumulations, O^T += V^T.P^T, P as fp16 hi + lo, online
//     softmax in base 2); position + tokens <= 256 leaves at most one wave
//     with a second page;
//   * every wave rescales its partial O to the workgroup's row maxima, waves
//     4..7 hand theirs to waves 0..3 through LDS, and each thread sums the
//     four remaining partials of one output element and writes it gated:
//     out = O / L * sigmoid(gate).
// Cached-page slots from `position` on are masked and their values zeroed:
// other workgroups append the new tokens there while this one reads.
#include "kernels.hpp"
#include "prep.hpp"

#include <cmath>

namespace rs {
namespace {

__device__ __forceinline__ f32x4 mfma(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Token held in slot j of a V^T operand by lane group g (see common.hpp).
__device__ __forceinline__ int v_slot_token(int g, int j) {
    return j < 4 ? 4 * g + j : 16 + 4 * g + j - 4;
}

constexpr int kShortWaves = 8;

struct ShortArgs {
    FusedToken tok;   // q_gate, key, value, norms, pages, epsilon, position, tokens
    float *out;       // [tokens][24][256]
    float scale_log2;
};

__global__ __launch_bounds__(kShortWaves * kWave)
void attention_fused_short(ShortArgs a) {
    constexpr int D = kModelHeadDim, H = kModelQHeads, HKV = kModelKvHeads, G = H / HKV;
    constexpr int KS = D / 32, DT = D / 16, PAGE = 32 * D;
    constexpr int NE = G * D / 4;               // output elements (f32x4) of the workgroup
    constexpr int kHalf = kShortWaves / 2;
    static_assert(D == 4 * kWave, "256-dim rows, four values per lane");
    static_assert(kShortWaves == kShortMaxTokens && G <= kShortWaves, "one query row and one new key per wave");
    static_assert(NE <= kShortWaves * kWave, "one output element per thread");
    // Query fragments: qf[part][ks][lane] is the B operand of k-step ks for
    // lane l (row l % 16, dims 32ks + 8(l/16) .. +7), part 0 = fp16(q),
    // part 1 = fp16(q - part 0); rows past the group are zero.
    __shared__ f16x8 qf[2][KS][kWave];
    __shared__ __attribute__((aligned(16))) _Float16 knew[PAGE], vnew[PAGE];   // the new keys' page
    __shared__ f32x4 so[kHalf][DT * kWave];     // partial O of waves 4..7, then of the pairs
    __shared__ float sml[kShortWaves][2][16];

    const FusedToken &tok = a.tok;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int t = blockIdx.x, h = blockIdx.y;
    const int position = tok.position;          // cached keys 0 .. position-1
    const int n_cached = (position + 31) / 32;  // cached pages; page n_cached is the new keys'
    const bool has_q = w < G, has_key = w <= t;   // wave-uniform

    // ---- every load first (lane l holds dims 64i + l of a row); rows a wave
    // does not use are read at a clamped index so every address is valid ----
    float xq[1][4], xk[1][4], xv[4], gq[4], gk[4];
    {
        const float *qs = tok.q_gate + ((size_t)t * H + h * G + min(w, G - 1)) * 2 * D;
        const size_t kr = ((size_t)min(w, t) * HKV + h) * D;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xq[0][i] = qs[64 * i + lane];
            xk[0][i] = tok.key[kr + 64 * i + lane];
            xv[i] = tok.value[kr + 64 * i + lane];
            gq[i] = tok.q_norm[64 * i + lane];
            gk[i] = tok.k_norm[64 * i + lane];
        }
    }
    // The gate of this thread's output element e: row e / 64, dims
    // 4 (e % 64) .. +3.
    const int e = min((int)threadIdx.x, NE - 1);
    const f32x4 gate = *reinterpret_cast<const f32x4 *>(tok.q_gate + ((size_t)t * H + h * G + e / 64) * 2 * D + D +
                                                        4 * (e % 64));
    const _Float16 *kh = static_cast<const _Float16 *>(tok.k_pages) + (size_t)h * tok.head_stride + lane * 8;
    const _Float16 *vh = static_cast<const _Float16 *>(tok.v_pages) + (size_t)h * tok.head_stride + lane * 8;
    f16x8 kb[2][KS], vb[DT];
    if (w < n_cached) {
        const _Float16 *kp = kh + (size_t)w * PAGE;
#pragma unroll
        for (int tile = 0; tile < 2; ++tile)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                kb[tile][ks] = __builtin_nontemporal_load(reinterpret_cast<const f16x8 *>(kp + tile * 16 * D + ks * 512));
        const _Float16 *vp = vh + (size_t)w * PAGE;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) vb[dt] = __builtin_nontemporal_load(reinterpret_cast<const f16x8 *>(vp + dt * 512));
    }
    // Zero the fragments of rows G..15 (lanes 16g + r, r >= G), which no
    // wave prepares: KS*4*(16-G) entries per part.
    for (int i = threadIdx.x; i < 2 * KS * 4 * (16 - G); i += kShortWaves * kWave) {
        const int part = i / (KS * 4 * (16 - G)), rest = i % (KS * 4 * (16 - G));
        const int ks = rest / (4 * (16 - G)), g = (rest / (16 - G)) % 4, r = G + rest % (16 - G);
        qf[part][ks][16 * g + r] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }

    // ---- prepare this wave's query row and new key ----
    const double freq = rope_freq(lane);
    if (has_q) {
        float c[1] = {1.f}, s[1] = {0.f};
        if (lane < 32) rope_cos_sin(position + t, freq, c[0], s[0]);
        norm_rope_rows<1>(xq, gq, c, s, tok.epsilon, lane);
        // Dim d = 64i + l of row w: k-step d / 32, lane 16 ((d % 32) / 8) + w,
        // element d % 8.
        _Float16 *qh = reinterpret_cast<_Float16 *>(&qf[0][0][0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = 64 * i + lane;
            const int at = ((d >> 5) * kWave + 16 * ((d >> 3) & 3) + w) * 8 + (d & 7);
            const _Float16 hi = (_Float16)xq[0][i];
            qh[at] = hi;
            qh[KS * kWave * 8 + at] = (_Float16)(xq[0][i] - (float)hi);
        }
    }
    if (has_key) {
        float c[1] = {1.f}, s[1] = {0.f};
        if (lane < 32) rope_cos_sin(position + w, freq, c[0], s[0]);
        norm_rope_rows<1>(xk, gk, c, s, tok.epsilon, lane);
        _Float16 *kp = static_cast<_Float16 *>(tok.k_pages) + (size_t)h * tok.head_stride;
        _Float16 *vp = static_cast<_Float16 *>(tok.v_pages) + (size_t)h * tok.head_stride;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const _Float16 kq = cache_half(xk[0][i]), vq = cache_half(xv[i]);
            knew[k_page_offset(w, 64 * i + lane, D)] = kq;
            vnew[v_page_offset(w, 64 * i + lane, D)] = vq;
            if (w == t) {
                kp[k_page_offset(position + t, 64 * i + lane, D)] = kq;
                vp[v_page_offset(position + t, 64 * i + lane, D)] = vq;
            }
        }
    }
    lds_barrier();

    // ---- the pages on the matrix cores ----
    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;
    // One page: the first `valid` keys of kb / vb are live (keys from there
    // on are masked and their values zeroed).
    auto page = [&](int valid) __attribute__((always_inline)) {
        // S^T of the two key tiles, the query's hi and lo parts accumulated
        // apart: four chains of KS dependent products instead of two of 2 KS.
        f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0, s2 = s0, s3 = s0;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const f16x8 qhi = qf[0][ks][lane], qlo = qf[1][ks][lane];
            s0 = mfma(kb[0][ks], qhi, s0);
            s1 = mfma(kb[1][ks], qhi, s1);
            s2 = mfma(kb[0][ks], qlo, s2);
            s3 = mfma(kb[1][ks], qlo, s3);
        }
        // Lane l holds local keys 16*tile + 4*(l/16) + r.
        const int key0 = 4 * (lane >> 4);
        float x[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            x[r] = (s0[r] + s2[r]) * a.scale_log2;
            x[4 + r] = (s1[r] + s3[r]) * a.scale_log2;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (key0 + 16 * (j >> 2) + (j & 3) >= valid) x[j] = -INFINITY;
        float bm = x[0];
#pragma unroll
        for (int j = 1; j < 8; ++j) bm = fmaxf(bm, x[j]);
        bm = fmaxf(bm, __shfl_xor(bm, 16, kWave));
        bm = fmaxf(bm, __shfl_xor(bm, 32, kWave));
        const float mn = fmaxf(m, bm);   // finite: every page has a valid key
        const float alpha = __builtin_amdgcn_exp2f(m - mn);
        m = mn;
        f16x8 ph, pl;
        float ps = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float p = __builtin_amdgcn_exp2f(x[j] - mn);
            const _Float16 p16 = (_Float16)p;
            ph[j] = p16;
            pl[j] = (_Float16)(p - (float)p16);
            ps += p;
        }
        l = l * alpha + ps;
        if (valid < 32) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (v_slot_token(lane >> 4, j) >= valid) {
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) vb[dt][j] = (_Float16)0.f;
                }
            }
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            acc[dt] *= alpha;
            acc[dt] = mfma(vb[dt], ph, acc[dt]);
            acc[dt] = mfma(vb[dt], pl, acc[dt]);
        }
    };
    // Cached page w holds position - 32w valid keys (at least one).
    if (w < n_cached) page(min(32, position - 32 * w));
    // The new keys' page (t + 1 valid keys; its slots past t were never
    // written) goes to wave n_cached % 8: a wave without a cached page, or
    // wave 0 after page 0 when n_cached = 8.
    if (w == n_cached % kShortWaves) {
#pragma unroll
        for (int tile = 0; tile < 2; ++tile)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                kb[tile][ks] = *reinterpret_cast<const f16x8 *>(knew + tile * 16 * D + ks * 512 + lane * 8);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) vb[dt] = *reinterpret_cast<const f16x8 *>(vnew + dt * 512 + lane * 8);
        page(t + 1);
    }

    // ---- merge the waves and write the gated rows ----
    l += __shfl_xor(l, 16, kWave);
    l += __shfl_xor(l, 32, kWave);
    if (lane < 16) {
        sml[w][0][lane] = m;
        sml[w][1][lane] = l;
    }
    lds_barrier();
    // Row r = l % 16 of lane l: the workgroup's maximum, finite for every
    // row (key t is always seen; rows past the group have zero scores).  A
    // wave without pages has m = -inf and acc = 0 and adds nothing.
    {
        const int r = lane & 15;
        float M = sml[0][0][r];
#pragma unroll
        for (int ww = 1; ww < kShortWaves; ++ww) M = fmaxf(M, sml[ww][0][r]);
        const float f = __builtin_amdgcn_exp2f(m - M);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] *= f;
    }
    if (w >= kHalf) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) so[w - kHalf][dt * kWave + lane] = acc[dt];
    }
    lds_barrier();
    if (w < kHalf) {
        // Each slot is read and rewritten by the same lanes of one wave.
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) so[w][dt * kWave + lane] += acc[dt];
    }
    lds_barrier();
    // Element e: row e / 64, dims 4 (e % 64) .. +3, which is the f32x4 of
    // lane r + 16 (d4 % 4) in fragment d4 / 4 of every slot.
    if ((int)threadIdx.x < NE) {
        const int r = e / 64, d4 = e % 64;
        float M = sml[0][0][r];
#pragma unroll
        for (int ww = 1; ww < kShortWaves; ++ww) M = fmaxf(M, sml[ww][0][r]);
        float L = 0.f;
#pragma unroll
        for (int ww = 0; ww < kShortWaves; ++ww) L += sml[ww][1][r] * __builtin_amdgcn_exp2f(sml[ww][0][r] - M);
        f32x4 o = so[0][(d4 >> 2) * kWave + r + 16 * (d4 & 3)];
#pragma unroll
        for (int s = 1; s < kHalf; ++s) o += so[s][(d4 >> 2) * kWave + r + 16 * (d4 & 3)];
        const float inv = 1.f / L;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] *= inv * (1.f / (1.f + expf(-gate[j])));
        *reinterpret_cast<f32x4 *>(a.out + ((size_t)t * H + h * G + r) * D + 4 * d4) = o;
    }
}

}  // namespace

void launch_fused_short(const FusedToken &tok, float *out, hipStream_t stream) {
    require(tok.tokens >= 1 && tok.tokens <= kShortMaxTokens, "the short fused kernel takes 1..8 tokens");
    require(tok.position + tok.tokens <= kShortFusedKeys, "the short fused kernel takes up to 256 keys");
    ShortArgs a;
    a.tok = tok;
    a.out = out;
    a.scale_log2 = (1.0f / 16.0f) * 1.4426950408889634f;
    void *args[] = {&a};
    check(hipLaunchKernel((const void *)&attention_fused_short, dim3(tok.tokens, kModelKvHeads),
                          dim3(kShortWaves * kWave), args, 0, stream));
}

}  // namespace rs
