// Log-sum-exp combine of split-K partials (the per-row work of the combine
// kernel).
#pragma once
#include "kernels.hpp"
#include "prep.hpp"

#include <cmath>
#include <type_traits>

namespace rs {


// One row of one KV head, combined by the four waves w4 = 0..3 of a
// workgroup (every wave must call it, `valid` or not: it holds a workgroup
// barrier); with QD > 1, head dims dq*D/QD .. of that row only (a workgroup
// per (row, dq)).  Lane l owns head dims DV*l .. DV*l+DV-1 of them (DV =
// D/QD/64);
// wave w4 takes splits w4, w4+4, ... and issues the loads of up to kBatch of
// them at once, so a combine over up to 4*kBatch splits costs one memory
// round trip: their partial rows, and their m and l held one split per lane
// (lane i: split w4 + 4i), two loads for the wave.  The round's max and sum
// come from lane reductions over the 16 lanes of the first row, and each
// split's weight reaches every lane by readlane.  (One m and one l load per
// split in every lane, the same address across the wave, took 0.06-0.38 us
// more per layer: decode at 139,264 keys 86.50 -> 86.35, at 4,096 10.80 ->
// 10.50, verify-8 at 16K 19.91 -> 19.85, the fused decode 88.32 -> 87.94
// and the fused verify-8 25.23 -> 24.95 us; medians of 3 in-process
// rounds.)  The waves then merge through
// `scratch` (4*(D/QD+1) + 4 floats of LDS per group), each thread one head
// dim.
// PT is the type of the partial rows: float (unnormalised O) or _Float16
// (O / l, weighted by l here).  NT: the partial rows are loaded
// non-temporally, matching partials that were stored that way (the load
// policy of the combine follows the store policy of the split kernel: the
// mixed pairs measured slower).
//
// NEWKEY (the new tokens of a fused call on the stream kernel, one or two;
// the code takes up to 8): the splits cover the cached keys only.  Wave w4
// takes the new keys j = w4 and w4 + 4 that this row sees (j <= its token
// t) and folds each in as one more split: score q . k_j with the prepared
// fp32 query (tok->q_prep) and the fp16 key the split kernel appended at
// position + j, weight 1 at its own max, value the appended fp16 v_j.
template <int D, typename KV, typename PT, bool NT, bool NEWKEY = false, int QD = 1>
__device__ __forceinline__ void combine_row(const PT *part_o, const float *part_ml, int splits,
                                            int rows, int group, int q_heads, int row, int h,
                                            bool valid, int w4, int lane, float *scratch,
                                            void *out, const float *gate, int out_mode,
                                            const FusedToken *tok = nullptr, float scale_log2 = 0.f, int dq = 0) {
    constexpr int DW = D / QD;            // head dims of this workgroup: dq*DW ..
    constexpr int DV = DW / kWave;
    static_assert(DV >= 1, "a lane owns at least one head dim");
    constexpr int kBatch = 16;
    static_assert(kBatch <= 16, "a round's (m, l) pairs sit in the 16 lanes of one DPP row");
    float *part = scratch;                   // [4][DW + 1]
    float *wmax = scratch + 4 * (DW + 1);    // [4]
    const int rc = valid ? row : rows - 1;   // in-bounds reads for a padding group
    const float *ml = part_ml + (size_t)h * splits * 2 * rows + rc;
    const PT *po = part_o + ((size_t)h * splits * rows + rc) * D + dq * DW + lane * DV;
    constexpr bool kNormalised = !std::is_same<PT, float>::value;
    const size_t stride = (size_t)rows * D;

    const int t = row / group, hq = h * group + (row - t * group);
    // This thread's head dim in the final merge.  The gate of a gated
    // output is requested with the partials, so it has landed by the final
    // store instead of costing one more round trip.
    const int jd = w4 * kWave + lane;
    float gv = 0.f;
    if (out_mode == kOutGated && valid && jd < DW)
        gv = gate[((size_t)t * q_heads + hq) * 2 * D + D + dq * DW + jd];

    float M = -INFINITY, L = 0.f, acc[DV] = {};
    // NEWKEY: this wave's new keys (lane l: dims 4l .. 4l+3 of the query and
    // of each key, for the score over every head dim; dims DV*l .. +DV-1 of
    // this workgroup's head dims of each value), requested with the partials.
    constexpr int NK = 2, DQK = D / kWave;
    typedef _Float16 H4 __attribute__((ext_vector_type(4)));
    f32x4 qn = {};
    H4 kn[NK] = {};
    _Float16 vh[NK][DV] = {};
    float m_new[NK] = {-INFINITY, -INFINITY};
    bool has[NK] = {};
    if constexpr (NEWKEY) {
        static_assert(D == 4 * kWave && DQK == 4, "the fused model's 256-dim heads");
#pragma unroll
        for (int k = 0; k < NK; ++k) has[k] = w4 + 4 * k < tok->tokens && w4 + 4 * k <= t;
        if (has[0]) qn = *reinterpret_cast<const f32x4 *>(tok->q_prep + ((size_t)h * rows + rc) * D + lane * DQK);
        const _Float16 *kp = static_cast<const _Float16 *>(tok->k_pages) + (size_t)h * tok->head_stride;
        const _Float16 *vp = static_cast<const _Float16 *>(tok->v_pages) + (size_t)h * tok->head_stride;
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            if (has[k]) {
                const int pos = tok->position + w4 + 4 * k;
                // Dims 4l .. 4l+3 of a key are contiguous in its page.
                kn[k] = *reinterpret_cast<const H4 *>(kp + k_page_offset(pos, lane * DQK, D));
#pragma unroll
                for (int d = 0; d < DV; ++d) vh[k][d] = vp[v_page_offset(pos, dq * DW + lane * DV + d, D)];
            }
        }
    }
    // Rounds of 4*kBatch splits (one round for up to 64 splits).
    for (int s0 = 0; s0 < splits; s0 += 4 * kBatch) {
        // Every load is issued unconditionally (splits past the end re-read
        // the last one) so that all of them are in flight together; the
        // surplus ones are discarded afterwards.
        typedef PT OV __attribute__((ext_vector_type(DV)));
        OV ov[kBatch];
        // Lane i < kBatch: the max and sum of split s0 + w4 + 4i (two loads
        // for the wave instead of two per split).
        const int sl = min(s0 + w4 + 4 * min(lane, kBatch - 1), splits - 1);
        const float ms = ml[(size_t)sl * 2 * rows], ls = ml[(size_t)sl * 2 * rows + rows];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int sc = min(s0 + w4 + 4 * i, splits - 1);
            const OV *src = reinterpret_cast<const OV *>(po + (size_t)sc * stride);
            if constexpr (NT)
                ov[i] = __builtin_nontemporal_load(src);
            else
                ov[i] = *src;
        }
        if constexpr (NEWKEY) {
            // Round 0: the new keys' scores, while this round's partial loads
            // are in flight (their inputs were requested first).
            if (s0 == 0) {
#pragma unroll
                for (int k = 0; k < NK; ++k) {
                    if (has[k]) {
                        float dot = 0.f;
#pragma unroll
                        for (int d = 0; d < DQK; ++d) dot += qn[d] * (float)kn[k][d];
                        m_new[k] = wave_sum_dpp(dot) * scale_log2;
                    }
                }
            }
        }
        const bool live = lane < kBatch && s0 + w4 + 4 * lane < splits;
        const float mv = live ? ms : -INFINITY, lv = live ? ls : 0.f;
        // The round's max over lanes 0..15 (one row of 16 lanes), then
        // uniform.
        float bm = fmaxf(mv, dpp_get<0xb1>(mv));
        bm = fmaxf(bm, dpp_get<0x4e>(bm));
        bm = fmaxf(bm, dpp_get<0x141>(bm));
        bm = fmaxf(bm, dpp_get<0x140>(bm));
        const float rm = fmaxf(M, __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(bm))));
        const float mu = rm == -INFINITY ? 0.f : rm;
        const float f = __builtin_amdgcn_exp2f(M - mu);
        const float wl = __builtin_amdgcn_exp2f(mv - mu);
        float sl_ = wl * lv;
        sl_ = sl_ + dpp_get<0xb1>(sl_);
        sl_ = sl_ + dpp_get<0x4e>(sl_);
        sl_ = sl_ + dpp_get<0x141>(sl_);
        sl_ = sl_ + dpp_get<0x140>(sl_);
        L = L * f + __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sl_)));
#pragma unroll
        for (int d = 0; d < DV; ++d) acc[d] *= f;
        const float wo_l = kNormalised ? wl * lv : wl;
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            if (s0 + w4 + 4 * i < splits) {
                const float wo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wo_l), i));
#pragma unroll
                for (int d = 0; d < DV; ++d) acc[d] += wo * (float)ov[i][d];
            }
        }
        M = rm;
    }
    if constexpr (NEWKEY) {
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            if (has[k]) {
                // New key j = w4 + 4k as one more split: weight 1 at its own max.
                const float rm = fmaxf(M, m_new[k]);
                const float f = __builtin_amdgcn_exp2f(M - rm), e = __builtin_amdgcn_exp2f(m_new[k] - rm);
                L = L * f + e;
#pragma unroll
                for (int d = 0; d < DV; ++d) acc[d] = acc[d] * f + e * (float)vh[k][d];
                M = rm;
            }
        }
    }
    // One barrier: every wave leaves its (M, L) and its unscaled
    // accumulators in its slot; then thread j of the workgroup merges head
    // dim j of the four slots and stores it.
#pragma unroll
    for (int d = 0; d < DV; ++d) part[w4 * (DW + 1) + lane * DV + d] = acc[d];
    if (lane == 0) {
        wmax[w4] = M;
        part[w4 * (DW + 1) + DW] = L;
    }
    __syncthreads();
    if (valid && jd < DW) {
        const float G = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
        const float gu = G == -INFINITY ? 0.f : G;
        float Lt = 0.f, o = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const float f = __builtin_amdgcn_exp2f(wmax[ww] - gu);
            Lt += part[ww * (DW + 1) + DW] * f;
            o += part[ww * (DW + 1) + jd] * f;
        }
        o /= Lt;
        const size_t idx = ((size_t)t * q_heads + hq) * D + dq * DW + jd;
        if (out_mode == kOutGated) {
            static_cast<float *>(out)[idx] = o * (1.f / (1.f + expf(-gv)));
        } else if (out_mode == kOutF32) {
            static_cast<float *>(out)[idx] = o;
        } else {
            static_cast<KV *>(out)[idx] = (KV)o;
        }
    }
}

}  // namespace rs
