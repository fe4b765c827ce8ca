// Chunked prefill: many query tokens against the paged cache, on the matrix
// cores.  The reference has no prefill kernel (its server prefills 8 tokens
// at a time through attention/attention_tiled, src/kernels.cu:435-503 and
// qvelox/server.py:187-191); this is the same causal GQA formula for long
// token runs: row t sees keys 0..position+t.
//
// One workgroup owns 192 query rows of one KV head (row = token * group +
// query head within the group) as twelve 16-row tiles, one per wave (three
// per SIMD), whose query fragments stay in registers.  The tiles are dealt
// out so that every SIMD has about the same number of (row, key) pairs (see
// the kernel).  The workgroup walks the pages
// that its last row can see through two rings of four LDS buffers, one for
// K pages and one for V pages (16 KiB each at D=256), filled by direct
// global->LDS loads two K and two V pages at every second step, a pair
// ahead of the pair in use.  Since pages are stored in MFMA
// operand order, every wave reads its A operands as conflict-free 16-byte
// LDS fragments:
//   S^T[key][row] = K[key][:] . Q[row][:]     (A = K tile from LDS, B = Q)
//   O^T[dim][row] += V^T[dim][key] P^T[key][row]  (A = V^T from LDS, B = P^T,
//                                                  straight from S^T's C layout)
//
// Software pipeline: step i computes the scores of page i+1 on the matrix
// cores while the vector ALUs run the softmax of page i (whose scores the
// previous step produced), then multiplies page i's V by its P.  The two
// halves are interleaved chunk by chunk, so every wave keeps both units busy
// instead of alternating between them in step with the other waves of its
// SIMD.  Online softmax in base 2 with a lazily moved row max (see ring.hip);
// scores are scaled before they are masked and their max is taken, so any
// finite scale (zero and negative ones included) gives the softmax of the
// scaled scores.  P multiplies V as one fp16 value.  On bf16 caches a
// streaming pass (convert_v_pages) first writes the call's V pages as fp16
// into the workspace, which is exact for every bf16 value from 2^-14 to
// 65280 (the fp16 normal range), so bf16 runs one V product per fragment,
// like fp16, where P split into bf16 hi + lo parts would take two.  A KV
// head with a V value outside that range (larger, tiny but nonzero in all
// eight keys that one operand slot holds, or not finite) is flagged by the
// pass, and the workgroups of that head take the exact products instead
// (bf16 V, P as bf16 hi + lo parts; attention_prefill_bf16).
//
// Scheduling: workgroup i serves KV head i % kv_heads (with 4 KV heads the
// round-robin dispatch over the 8 XCDs keeps every head on the same two XCDs,
// whose L2s then hold that head's pages for all of its workgroups).  A call
// with too few row workgroups to occupy every CU (a short chunk on a long
// prefix) splits each row workgroup's pages into equal runs, one workgroup
// per run; their partial rows are merged by combine_prefill (below) or, for
// many runs, attention_combine, as in split-K decode.  A raw call merged by
// combine_prefill stores them as O / l in 16-bit planes (PrefillArgs::
// half_parts), the precise and gated calls and the many-run ones as fp32.
#include "combine.hpp"
#include "kernels.hpp"
#include "lds.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>

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

__device__ __forceinline__ float max3(float a, float b, float c) {
    return __builtin_fmaxf(__builtin_fmaxf(a, b), c);
}

// Two fp32 values as one dword of 16-bit values (element 0 in the low half).
__device__ __forceinline__ uint32_t pack2(float a, float b, _Float16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, h2{(_Float16)a, (_Float16)b});
}
__device__ __forceinline__ uint32_t pack2(float a, float b, __bf16) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, b2{(__bf16)a, (__bf16)b});
}
// The two halves of a packed word as fp32 values.  A bf16 low half is moved
// up with a byte permute (bytes 1:0 to 3:2, zeros below), which keeps the
// compiler from converting the fp32 input a second time instead.
__device__ __forceinline__ float unpack_lo(uint32_t w, __bf16) {
    return __uint_as_float(__builtin_amdgcn_perm(0u, w, 0x01000c0cu));
}
__device__ __forceinline__ float unpack_hi(uint32_t w, __bf16) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float unpack_lo(uint32_t w, _Float16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return (float)__builtin_bit_cast(h2, w)[0];
}
__device__ __forceinline__ float unpack_hi(uint32_t w, _Float16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return (float)__builtin_bit_cast(h2, w)[1];
}

constexpr float kLazy = 8.f;
// prefill_rows' PREP bits: the query prepared from q_gate in the kernel; the
// chunk's own keys prepared and appended in the kernel too.
constexpr int kPrepQuery = 1, kPrepKeys = 2;


struct PrefillArgs {
    const void *q;
    const void *q_lo;       // lo parts of a precise (fp32) query, or null
    const float *gate;      // q_gate of a gated output, or null
    const void *k_pages;
    const void *v_pages;
    void *out;
    // bf16 calls: the fp16 copy of the V pages (packed to the call's pages,
    // v_copy_stride elements per KV head) and the conversion pass's words,
    // flag_words per KV head (a set word: a V value outside the fp16 range).
    const void *v_copy;
    size_t v_copy_stride;
    const uint32_t *v_flags;
    int flag_words;
    size_t head_stride;       // K and V pages
    int q_heads, kv_heads, group, rows, position, n_tiles;
    float scale_log2;
    // Key splits: workgroup (split, j, h) takes the split-th of `splits`
    // equal runs of the pages its rows see, and stores fp32 partials for the
    // combine kernel: its rows unnormalised ([kv_heads][splits][rows][D]),
    // their max (base 2) and sum ([kv_heads][splits][2][rows]).  One split:
    // the rows are stored normalised.
    float *part_o;
    float *part_ml;
    int splits;
    // Raw calls merged by combine_prefill: the partial rows as O / l in two
    // 16-bit planes of the same layout, plane A at part_o and plane B right
    // after it (the fp32 rows' bytes): fp16 values in plane A for a KV head
    // whose V is fp16 (fp16 pages, or bf16 ones copied to fp16); for a head
    // that takes the exact bf16 products, the fp32 values' top 16 bits in
    // plane A and bottom 16 in plane B, and the row sums stored negated (so
    // the combine knows the format from the sums it loads anyway).
    int half_parts;
    // A fused prefill chunk that prepares its own query and keys
    // (attention_prefill_prep): the prepare kernel's inputs besides q_gate
    // (`gate`), and the chunk's token count.
    const float *key, *value, *q_norm, *k_norm;
    float epsilon;
    int tokens;
};

__device__ __forceinline__ int v_slot_token(int g, int j) {
    return j < 4 ? 4 * g + j : 16 + 4 * g + j - 4;
}

// KV: the query and K page type; VT: the V page type (fp16 for a converted
// bf16 cache), which P takes as well.  PSPLIT: P multiplies V as hi + lo
// parts of VT (the precise instance on fp16 pages, the exact instance on
// bf16 pages).  QSPLIT: the query is an fp32 one given as hi + lo fp16
// parts, both multiplied by K.  MODE: output of the KV type, fp32, or fp32
// times sigmoid(gate) (see combine.hpp).
// The rows of one workgroup; kring and vring are the kernel's two rings of
// four pages, V pages read from v_pages with v_head_stride elements per KV
// head.
// PASS: -1 for a single pass (ROWS / 16 waves, one tile each); 0 and 1 for
// the two passes of the two-pass instance (eight waves over ROWS = 192 rows:
// pass 0 gives waves 0-3 the round-0 tiles and waves 4-7 the round-1 tiles,
// pass 1 gives waves 0-3 the round-2 tiles and waves 4-7 none).
// PREP, bit kPrepQuery (the fused path's precise prefill): the query rows
// are prepared here from q_gate (RMSNorm, gamma, RoPE, hi + lo parts) rather
// than read as prepared hi + lo parts.  Bit kPrepKeys as well
// (attention_prefill_prep, the fused chunk of 9 .. 128 - position % 32
// tokens): the splits are runs over the cached keys 0 .. position-1, which
// every row sees, and the last run then attends to the chunk's own keys as
// well: it prepares them into its LDS rings (the prepare kernel's functions,
// so the same bits) and its workgroup 0 appends them to the pages.  No
// workgroup reads a key that another one appends.  (kPrepQuery: qn_stage is
// 1 KiB of LDS per wave, for the q_norm weights.)
template <int D, typename KV, typename VT, bool PSPLIT, bool QSPLIT, int MODE, int ROWS, int PASS = -1,
          int PREP = 0>
__device__ __forceinline__ void prefill_rows(const PrefillArgs &a, KV *kring, VT *vring, const void *v_pages,
                                             size_t v_head_stride, float *qn_stage = nullptr) {
    using V8 = typename Vec8<KV>::type;
    using OUT = std::conditional_t<MODE == kOutSame, KV, float>;
    typedef uint32_t U4 __attribute__((ext_vector_type(4)));
    using PT = VT;
    using PV8 = typename Vec8<PT>::type;
    constexpr int kPWaves = PASS < 0 ? ROWS / 16 : 8;
    static_assert(PASS < 0 || ROWS == 3 * 4 * 16, "two passes of eight waves over three rounds of tiles");
    constexpr bool PQ = (PREP & kPrepQuery) != 0, PK = (PREP & kPrepKeys) != 0;
    static_assert(!PQ || (D == kModelHeadDim && QSPLIT && PSPLIT && MODE == kOutGated &&
                          std::is_same<KV, _Float16>::value && std::is_same<VT, _Float16>::value),
                  "the prepared query is the fused model's: fp32 query as hi + lo parts, gated output");
    static_assert(!PK || (PQ && PASS < 0), "the chunk's own keys come with its prepared query, in one pass");
    constexpr int KS = D / 32, DT = D / 16;
    constexpr int PAGE = 32 * D;                       // elements of one K (or V) page
    constexpr int PAGE_BYTES = PAGE * 2;
    // The first kLoaders waves (two per SIMD of twelve, one per SIMD of
    // eight) copy the pages, H 1 KiB loads each per K (or V) page.
    constexpr int kLoaders = kPWaves == 12 ? 8 : kPWaves / 2;
    constexpr int H = PAGE_BYTES / 1024 / kLoaders;
    static_assert(H >= 1 && PAGE_BYTES / 1024 % kLoaders == 0, "loads divide over the loader waves");

    const int lane = threadIdx.x & 63, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave index (uniform)
    const int h = blockIdx.x % a.kv_heads;
    // Load balance.  The R rows of a KV head form T = ceil(R/16) tiles of 16
    // rows; a later tile sees more keys.  Wave w of workgroup j runs on SIMD
    // w % 4 and serves slot k = 4j + w%4 (K = 4 n_tiles slots per head) in
    // round w / 4, which deals the tiles out serpentine-wise:
    //   round 0: tile T-1-k    (the last K tiles, the latest first)
    //   round 1: tile T-2K+k   (the K before them, in rising order)
    //   round 2: tile T-3K+k   (the rest, rising)
    // Rounds 0 and 1 give every slot the same key count; round 2 rises with
    // k, while the stretch in which only the round-0 wave still has pages
    // shrinks with k.  So every SIMD, and every workgroup, has about the
    // same work.  Negative tiles are padding, and rows from R on are not
    // stored.  Workgroup j's last row lies in its round-0 tile of slot 4j.
    const int R = a.rows;
    const int rest = blockIdx.x / a.kv_heads;
    const int j = rest % a.n_tiles, split = rest / a.n_tiles;
    // kPrepKeys: the last run attends to the chunk's keys too (uniform per workgroup).
    const bool new_keys = PK && split == a.splits - 1;
    static_assert(kPWaves % 4 == 0 && kPWaves / 4 <= 3, "one to three rounds of four waves");
    const int T = (R + 15) / 16, K = 4 * a.n_tiles, slot = 4 * j + (w & 3);
    const int round = PASS == 1 ? (w < 4 ? 2 : 3) : w >> 2;   // round 3: no tile
    const int tile = round == 0 ? T - 1 - slot : round == 1 ? T - 2 * K + slot
                   : round == 2 ? T - 3 * K + slot : -1;
    const int row0 = 16 * tile;
    const int row_end = R;                                              // valid rows: [0, row_end)

    // Query fragments (B operand): k-step ks of lane l holds row row0 + l%16,
    // dims 32*ks + 8*(l/16) .. +7.  Padded rows load a valid row; their
    // results are not stored.  The first pages are requested right behind
    // them (a split workgroup runs for a few pages only), and the prologue's
    // wait covers both: loads complete in order, so a loader wave's wait for
    // the first K page covers its query, and the other waves wait for their
    // query alone.  (As compiler-tracked loads, the compiler would wait for
    // every page in flight before their first use.)
    V8 qf[KS], qlo[QSPLIT ? KS : 1];
    int limit;
    [[maybe_unused]] int row_token;
    // kPrepQuery: the row's fp32 query in the same layout (k-step ks: two float4),
    // and the q_norm weights as the prepare kernel holds them (lane l: dims
    // 64i + l); prepared once they have landed (prep_query).
    [[maybe_unused]] f32x4 qx[PQ ? KS : 1][2];
    [[maybe_unused]] float gw[4];
    // kPrepQuery: the RoPE cosines and sines of the tile's tokens (see
    // prep_query), evaluated while the query loads are in flight.
    [[maybe_unused]] float ca = 0.f, sa = 0.f, cb = 0.f, sb = 0.f;
    [[maybe_unused]] int qpos = 0, tile_pos = 0;
    {
        const int row = min(max(row0 + (lane & 15), 0), max(row_end, 1) - 1);
        const int t = row / a.group, gg = row - t * a.group;
        // kPrepKeys' cached runs: every row sees every cached key.
        row_token = t;
        limit = PK ? a.position - 1 : a.position + t;
        if constexpr (PQ) {
            qpos = a.position + t;
            // The position of the tile's first (clamped) row's token; the
            // tile's rows span at most four tokens (16 rows of 6 heads).
            tile_pos = a.position + min(max(row0, 0), max(row_end, 1) - 1) / a.group;
            const float *src = a.gate + ((size_t)t * a.q_heads + (size_t)h * a.group + gg) * 2 * D + 8 * g;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                global_load16(qx[ks][0], src + 32 * ks);
                global_load16(qx[ks][1], src + 32 * ks + 4);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) global_load4(gw[i], a.q_norm + 64 * i + lane);
        } else {
            const KV *src = static_cast<const KV *>(a.q) +
                            ((size_t)t * a.q_heads + (size_t)h * a.group + gg) * D + 8 * g;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) global_load16(qf[ks], src + 32 * ks);
            if constexpr (QSPLIT) {
                const KV *lo = static_cast<const KV *>(a.q_lo) + (src - static_cast<const KV *>(a.q));
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) global_load16(qlo[ks], lo + 32 * ks);
            }
        }
    }
    // Keys this workgroup can see: 0 .. position + (token of its last row:
    // the last valid row of tile T-1-4j, or in the second pass of tile
    // T-3K+4j+3; none when that tile is padding).
    // (kPrepKeys: the cached keys 0 .. position-1 first.)
    const int last_tile = PASS == 1 ? T - 3 * K + 4 * j + 3 : T - 1 - 4 * j;
    const int wg_keys = last_tile < 0 ? 0 : a.position + (min(16 * (last_tile + 1), R) - 1) / a.group + 1;
    int n_keys = PK && last_tile >= 0 ? a.position : wg_keys;
    const int n = (n_keys + 31) / 32;
    // This split's pages: p0 + i for i = 0 .. nl-1 (local index i, ring
    // buffer i % 4).  nl is uniform over the workgroup; nl = 0 leaves empty
    // partials (no keys: sum 0, rows 0).
    const int sp = (n + a.splits - 1) / a.splits;
    int p0 = split * sp;
    int nl = max(0, min(n, p0 + sp) - p0);
    // Pages of this wave: those its last valid row sees (none without one).
    const int wave_last = min(row0 + 15, row_end - 1);
    const int wave_keys = wave_last < max(row0, 0) ? 0 : a.position + wave_last / a.group + 1;
    int nw = min(max((PK && wave_keys ? n : (wave_keys + 31) / 32) - p0, 0), nl);
    // Pages from which on some row of this wave masks keys (every row sees
    // the keys up to position + its first row's token; kPrepKeys' cached keys:
    // up to position - 1).  Keys before key_lo are masked too (kPrepKeys'
    // chunk keys: the cached ones of their first page).
    int wave_first_limit = PK ? a.position - 1 : a.position + max(row0, 0) / a.group;
    int key_lo = 0;
    // kPrepKeys: pages come from the LDS rings as the workgroup prepared them
    // (the chunk's keys) rather than from global memory.
    [[maybe_unused]] bool from_lds = false;

    const KV *kh = static_cast<const KV *>(a.k_pages) + (size_t)h * a.head_stride;
    const VT *vh = static_cast<const VT *>(v_pages) + (size_t)h * v_head_stride;
    // Loader wave w copies 1 KiB chunks w*H .. w*H+H-1 of page p0 + i into
    // the ring's buffer i % 4.  Over a run the pages are requested in the
    // order K0 V0 K1 V1 K2 V2 ..., which the waits below count on.
    auto stage = [&](const auto *src, int i, auto *ring) __attribute__((always_inline)) {
        if (w >= kLoaders || from_lds) return;
        const auto *page = src + (size_t)(p0 + i) * PAGE + w * H * 512;       // uniform
        auto *buf = ring + (i & 3) * PAGE + w * H * 512;
#pragma unroll
        for (int c = 0; c < H; ++c)
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(page + c * 512 + lane * 8),
                                             (__attribute__((address_space(3))) void *)(buf + c * 512), 16, 0, 0);
    };
    const uint32_t kring_lane = lds_addr(kring) + lane * 16;
    const uint32_t vring_lane = lds_addr(vring) + lane * 16;

    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // m stays -inf for a row that sees no key of its pages (a split past its
    // last key).  Its exponents are taken against 0 instead (mu below), so
    // they are exp2(-inf) = 0 and the row's sum and accumulators stay 0: no
    // operation of this file makes a NaN, which matters because it is
    // compiled with -fno-honor-nans.  Such a row's partial is stored as
    // empty.
    float m = -INFINITY, l = 0.f;
    f32x4 s[2];            // scores of the page whose softmax comes next

    // ---- S^T of one page, chunk by chunk ----
    // K fragments stream through a window of KW k-steps (2 KW reads in
    // flight): the pair of k-step ks+KW is requested as soon as that of ks
    // has landed; the two key tiles are two independent accumulation chains.
    // The exact bf16 products (hi + lo P) in twelve waves keep one pair
    // ahead instead of two, which holds them within the 168 VGPRs that
    // twelve waves leave each (with two they need 171 and spill).
    constexpr int KW = PSPLIT && !QSPLIT && kPWaves == 12 ? 1 : 2;
    V8 kf[KS][2];
    auto read_k = [&](auto ks_, uint32_t kb) __attribute__((always_inline)) {
        constexpr int ks = decltype(ks_)::value;
        if constexpr (ks < KS) {
            lds_read<ks * 512 * 2>(kf[ks][0], kb);
            lds_read<(16 * D + ks * 512) * 2>(kf[ks][1], kb);
        }
    };
    auto qk_chunk = [&](auto ks_, uint32_t kb, f32x4 *sn) __attribute__((always_inline)) {
        constexpr int ks = decltype(ks_)::value;
        if constexpr (ks < KS) {
            constexpr int later = 2 * (KW - 1 < KS - 1 - ks ? KW - 1 : KS - 1 - ks);
            lds_wait<later>(kf[ks][0], kf[ks][1]);
            read_k(std::integral_constant<int, ks + KW>{}, kb);
            sn[0] = mfma(kf[ks][0], qf[ks], sn[0]);
            sn[1] = mfma(kf[ks][1], qf[ks], sn[1]);
            if constexpr (QSPLIT) {
                sn[0] = mfma(kf[ks][0], qlo[ks], sn[0]);
                sn[1] = mfma(kf[ks][1], qlo[ks], sn[1]);
            }
        }
    };

    // ---- one pipeline step: S^T of page i+1, softmax and P.V of page i ----
    // (On a workgroup's last step the scores of the page after the last are
    // computed from a stale buffer and dropped.)
    auto step = [&](int i) __attribute__((always_inline)) {
        const uint32_t kb = kring_lane + ((i + 1) & 3) * PAGE_BYTES;
        const uint32_t vb = vring_lane + (i & 3) * PAGE_BYTES;
        f32x4 sn[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
        // The S^T and softmax phase runs at raised wave priority, the P.V
        // products at the default one.  The three waves of a SIMD leave each
        // barrier in step; with the priorities the issue arbiter lets one of
        // them run ahead through its phase while another's V products fill
        // the matrix pipe (2048-token chunk: 461-469 -> 447-453 us per layer).
        __builtin_amdgcn_s_setprio(1);
        static_for<0, KW>([&](auto ks) { read_k(ks, kb); });
        // Scores of page p0 + i; keys past a row's limit are masked.
        const int key0 = (p0 + i) * 32;
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = s[j >> 2][j & 3] * a.scale_log2;
        if (key0 + 31 > wave_first_limit || (PK && key0 < key_lo)) {
            keep_branch();
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int key = key0 + 16 * (j >> 2) + 4 * g + (j & 3);
                if (key > limit || (PK && key < key_lo)) x[j] = -INFINITY;
            }
        }
        float mx = __builtin_fmaxf(max3(x[0], x[1], x[2]), max3(x[3], x[4], x[5]));
        mx = max3(mx, x[6], x[7]);
        pin(mx);
        qk_chunk(std::integral_constant<int, 0>{}, kb, sn);
        // Row max over the four lane groups (key subsets) of the row.
        mx = row_group_max(mx);
        pin(mx);
        qk_chunk(std::integral_constant<int, 1>{}, kb, sn);
        // A row that sees a key of this split sees its first one on the
        // split's first page, where its max becomes finite.
        const float bm = mx;
        float alpha = 1.f;
        // `moved` implies a finite bm, so m - bm is never -inf - (-inf).
        const bool moved = bm > m + kLazy;
        if (moved) alpha = __builtin_amdgcn_exp2f(m - bm);
        m = moved ? bm : m;
        // The exponents' reference point: m, or 0 while the row has seen no
        // key (all its scores are then -inf, and their exponents 0).
        float mu = m == -INFINITY ? 0.f : m;
        float e[8];
        pin(alpha, mu);
        qk_chunk(std::integral_constant<int, 2>{}, kb, sn);
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = __builtin_amdgcn_exp2f(x[j] - mu);
        pin(e[0], e[1], e[2], e[3]);
        qk_chunk(std::integral_constant<int, 3>{}, kb, sn);
#pragma unroll
        for (int j = 4; j < 8; ++j) e[j] = __builtin_amdgcn_exp2f(x[j] - mu);
        pin(e[4], e[5], e[6], e[7]);
        qk_chunk(std::integral_constant<int, 4>{}, kb, sn);
        // P^T as B operands: hi parts (and lo parts, bf16).
        uint32_t ph[4], pl[4] = {};
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
            ph[j / 2] = pack2(e[j], e[j + 1], PT{});
            if constexpr (PSPLIT) {
                pl[j / 2] = pack2(e[j] - unpack_lo(ph[j / 2], PT{}), e[j + 1] - unpack_hi(ph[j / 2], PT{}), PT{});
            }
        }
        pin(ph[0], ph[1]);
        if constexpr (PSPLIT) pin(pl[0], pl[1]);
        qk_chunk(std::integral_constant<int, 5>{}, kb, sn);
#pragma unroll
        for (int j = 4; j < 8; j += 2) {
            ph[j / 2] = pack2(e[j], e[j + 1], PT{});
            if constexpr (PSPLIT) {
                pl[j / 2] = pack2(e[j] - unpack_lo(ph[j / 2], PT{}), e[j + 1] - unpack_hi(ph[j / 2], PT{}), PT{});
            }
        }
        pin(ph[2], ph[3]);
        if constexpr (PSPLIT) pin(pl[2], pl[3]);
        qk_chunk(std::integral_constant<int, 6>{}, kb, sn);
        l = l * alpha + (((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7])));
        pin(l);
        qk_chunk(std::integral_constant<int, 7>{}, kb, sn);
        static_for<8, KS>([&](auto ks) { qk_chunk(ks, kb, sn); });
        const PV8 p_hi = __builtin_bit_cast(PV8, U4{ph[0], ph[1], ph[2], ph[3]});
        const PV8 p_lo = __builtin_bit_cast(PV8, U4{pl[0], pl[1], pl[2], pl[3]});

        // ---- O^T += V^T P^T for page i ----
        // V fragments stream through a window of VW reads.
        constexpr int VW = 4;
        PV8 vf[DT];
        auto read_v = [&](auto dt_) __attribute__((always_inline)) {
            constexpr int dt = decltype(dt_)::value;
            if constexpr (dt < DT) lds_read<dt * 1024>(vf[dt], vb);
        };
        static_for<0, VW>(read_v);
        if (__any(moved)) {
            keep_branch();
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
        }
        // Pairs of tiles: the hi and lo products of a tile accumulate into
        // the same registers, so they are issued two apart.
        __builtin_amdgcn_s_setprio(0);
        static_for<0, DT / 2>([&](auto dp_) {
            constexpr int dt = 2 * decltype(dp_)::value;
            constexpr int later = dt + 2 + VW <= DT + 2 ? VW - 2 : DT - 2 - dt;
            lds_wait<later>(vf[dt], vf[dt + 1]);
            read_v(std::integral_constant<int, dt + VW>{});
            read_v(std::integral_constant<int, dt + VW + 1>{});
            acc[dt] = mfma(vf[dt], p_hi, acc[dt]);
            acc[dt + 1] = mfma(vf[dt + 1], p_hi, acc[dt + 1]);
            if constexpr (PSPLIT) {
                acc[dt] = mfma(vf[dt], p_lo, acc[dt]);
                acc[dt + 1] = mfma(vf[dt + 1], p_lo, acc[dt + 1]);
            }
        });
        s[0] = sn[0];
        s[1] = sn[1];
    };

    // ---- kPrepQuery: the query's hi + lo fragments from its fp32 row ----
    // RMSNorm over the row's 256 dims (each lane holds 64 of them; the four
    // lanes of a row sum theirs with lane swaps), times q_norm, RoPE on the
    // pairs (i, i+32), i < 32 (dims 8g + e of k-step 0 and 1 of the same
    // lane), with the prepare kernel's formulas and angles.  The prepare
    // kernel sums the squares in another order, so a value may differ from
    // its in the last bit of fp32.  The q_norm weights pass through the
    // wave's LDS slot into the fragment layout.  Each lane evaluates two
    // angles, pair lane % 32 of the tile's tokens 0 + lane / 32 and
    // 2 + lane / 32, and every lane takes its eight from those lanes.
    [[maybe_unused]] auto prep_query = [&]() __attribute__((always_inline)) {
      if constexpr (PQ) {
#pragma clang fp contract(off)
        static_for<0, KS>([&](auto ks) { pin(qx[ks][0], qx[ks][1]); });
        pin(gw[0], gw[1], gw[2], gw[3]);
        const uint32_t slot = lds_addr(qn_stage) + w * 1024;
#pragma unroll
        for (int i = 0; i < 4; ++i) lds_write4(slot + (64 * i + lane) * 4, gw[i]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        f32x4 qg[KS][2];
        static_for<0, 2>([&](auto half_) {
            constexpr int K0 = decltype(half_)::value * KS / 2;
            static_for<0, KS / 2>([&](auto k_) {
                constexpr int ks = K0 + decltype(k_)::value;
                lds_read<ks * 128>(qg[ks][0], slot + 32 * g);
                lds_read<ks * 128 + 16>(qg[ks][1], slot + 32 * g);
            });
            static_for<0, KS / 2>([&](auto k_) {
                constexpr int ks = K0 + decltype(k_)::value;
                lds_wait<2 * (KS / 2 - 1 - decltype(k_)::value)>(qg[ks][0], qg[ks][1]);
            });
        });
        float sq = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e) sq = (sq + (qx[ks][e >> 2][e & 3] * qx[ks][e >> 2][e & 3]));
        const float inv = rsqrtf((row_group_sum(sq) * (1.f / D)) + a.epsilon);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e) qx[ks][e >> 2][e & 3] = ((qx[ks][e >> 2][e & 3] * inv) * qg[ks][e >> 2][e & 3]);
        const int dt = qpos - tile_pos;                    // 0 .. 3
        const bool later = dt >= 2;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int src = ((dt & 1) << 5) + 8 * g + e;
            const float c0 = __shfl(ca, src, kWave), c1 = __shfl(cb, src, kWave);
            const float s0 = __shfl(sa, src, kWave), s1 = __shfl(sb, src, kWave);
            const float c = later ? c1 : c0, sn = later ? s1 : s0;
            const float x0 = qx[0][e >> 2][e & 3], x1 = qx[1][e >> 2][e & 3];
            qx[0][e >> 2][e & 3] = ((x0 * c) - (x1 * sn));
            qx[1][e >> 2][e & 3] = ((x0 * sn) + (x1 * c));
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = qx[ks][e >> 2][e & 3];
                const _Float16 hi = (_Float16)x;
                qf[ks][e] = hi;
                qlo[ks][e] = (_Float16)(x - (float)hi);
            }
      }
    };
    // ---- kPrepKeys, the last run: the chunk's keys in the rings ----
    // The K and V buffers of those pages (at most four) are zeroed, then wave
    // w prepares keys w, w+8, ... (lane l: dims 64i + l, the prepare
    // kernel's functions, so the bits it appends) and writes those this
    // workgroup's rows see at their slots; slots of cached keys (before
    // `position`) and past the last stay zero and are masked.  Workgroup 0
    // (whose rows include the chunk's last) prepares every key and appends
    // them to the pages; the cached runs mask and zero the slots from
    // `position` on of the page they share, so reading them while they are
    // written is harmless.
    [[maybe_unused]] auto prep_new_keys = [&]() __attribute__((always_inline)) {
      if constexpr (PK) {
            U4 *kz = reinterpret_cast<U4 *>(kring), *vz = reinterpret_cast<U4 *>(vring);
            for (int e = threadIdx.x; e < nl * PAGE / 8; e += kPWaves * kWave) {
                kz[e] = U4{0u, 0u, 0u, 0u};
                vz[e] = U4{0u, 0u, 0u, 0u};
            }
            lds_barrier();
            const int seen = wg_keys - a.position, todo = j == 0 ? a.tokens : seen;
            float gk[4];
    #pragma unroll
            for (int i = 0; i < 4; ++i) gk[i] = a.k_norm[64 * i + lane];
            const double fq = rope_freq(lane);
            _Float16 *kpg = const_cast<_Float16 *>(static_cast<const _Float16 *>(a.k_pages)) + (size_t)h * a.head_stride;
            _Float16 *vpg = const_cast<_Float16 *>(static_cast<const _Float16 *>(a.v_pages)) + (size_t)h * a.head_stride;
            for (int jj = w; jj < todo; jj += kPWaves) {
                const size_t krow = ((size_t)jj * a.kv_heads + h) * D + lane;
                float xk[1][4], xv[4];
    #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    xk[0][i] = a.key[krow + 64 * i];
                    xv[i] = a.value[krow + 64 * i];
                }
                const int key = a.position + jj;
                float c[1] = {1.f}, sn[1] = {0.f};
                if (lane < 32) rope_cos_sin(key, fq, c[0], sn[0]);
                norm_rope_rows<1>(xk, gk, c, sn, a.epsilon, lane);
                const int buf = key / 32 - p0;
    #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int d = 64 * i + lane;
                    const _Float16 kv = cache_half(xk[0][i]), vv = cache_half(xv[i]);
                    if (jj < seen) {
                        kring[buf * PAGE + k_page_offset(key & 31, d, D)] = kv;
                        vring[buf * PAGE + v_page_offset(key & 31, d, D)] = vv;
                    }
                    if (j == 0) {
                        kpg[k_page_offset(key, d, D)] = kv;
                        vpg[v_page_offset(key, d, D)] = vv;
                    }
                }
            }
            lds_barrier();
          }
    };

    // ---- prologue: K0 V0 K1 V1 K2 requested, S^T of page 0 ----
    s[0] = s[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (nl > 0) {
        stage(kh, 0, kring);
        stage(vh, 0, vring);
        if (nl > 1) { stage(kh, 1, kring); stage(vh, 1, vring); }
        if (nl > 2) stage(kh, 2, kring);
    }
    if constexpr (PQ) {
        // Each lane's two RoPE angles depend on the tile's position only, so
        // they are evaluated before the wait for the query rows (fused
        // 64-token chunk at 16,384: 62.75 -> 62.52 us per layer, medians of
        // 7 in-process rounds; 66.12 -> 65.79 on another box).
        {
#pragma clang fp contract(off)
            const double fq = rope_freq(lane & 31);
            rope_cos_sin(tile_pos + (lane >> 5), fq, ca, sa);
            rope_cos_sin(tile_pos + 2 + (lane >> 5), fq, cb, sb);
        }
        // The query's loads precede the pages' (loads complete in order):
        // wait for them alone and prepare the query while the pages are in
        // flight.
        if (w >= kLoaders || nl == 0) wait_vmcnt<0>();
        else if (nl > 2) wait_vmcnt<5 * H>();
        else if (nl > 1) wait_vmcnt<4 * H>();
        else wait_vmcnt<2 * H>();
        prep_query();
    }
    // S^T of the run's first page once it is in its buffer (every wave
    // meets first).
    auto first_scores = [&]() __attribute__((always_inline)) {
        ring_barrier();
        static_for<0, KW>([&](auto ks) { read_k(ks, kring_lane); });
        static_for<0, KS>([&](auto ks) { qk_chunk(ks, kring_lane, s); });
    };
    if (nl > 0) {
        // Loader waves: K0 has landed, and the query loads before it.  The
        // others issued no page loads: their query loads.
        if (w >= kLoaders) wait_vmcnt<0>();
        else if (nl > 2) wait_vmcnt<4 * H>();
        else if (nl > 1) wait_vmcnt<3 * H>();
        else wait_vmcnt<H>();
        first_scores();
    } else if constexpr (!PQ) {
        wait_vmcnt<0>();   // no page of this split: the query loads only
    }

    // The waves meet every second step (i even): K(i+1), K(i+2), V(i) and
    // V(i+1) have landed (every request), the waves meet (K(i-1), K(i),
    // V(i-2) and V(i-1) are consumed), and K(i+3), K(i+4), V(i+2) and V(i+3)
    // are requested into those buffers; steps i and i+1 then run in the waves
    // whose rows see those pages.  Every wave takes part in every barrier.
    // Meeting once per page instead, with three pages in flight, took 2.5%
    // longer on a 2048-token chunk (458.6 against 447.6 us).
    // At a meeting, on the workgroup's last page, each loader wave zeroes
    // the V slots past its last key in its own chunks once they have landed
    // (stale slots may hold anything, and a masked key's P of 0 times NaN is
    // NaN).  Chunk c of a page is dims 16c .. 16c+15 of all 32 keys; lane l
    // holds dim l%16, key group g = (l/16)%4 (keys 4g + j and 16 + 4g + j - 4).
    const int tail_page = n_keys % 32 ? n_keys / 32 : -1;
    auto prepare_v = [&](int i) __attribute__((always_inline)) {
        const int p = p0 + i;
        if (w >= kLoaders || i >= nl || p != tail_page || from_lds) return;
#pragma unroll
        for (int c = 0; c < H; ++c) {
            U4 *slot = reinterpret_cast<U4 *>(vring + (i & 3) * PAGE + (w * H + c) * 512) + lane;
            U4 v = *slot;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (p * 32 + v_slot_token(g, j) >= n_keys) v[j >> 1] &= (j & 1) ? 0x0000ffffu : 0xffff0000u;
            *slot = v;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };
    auto run_pages = [&]() __attribute__((always_inline)) {
        for (int i = 0; i < nl; ++i) {
            if ((i & 1) == 0) {
                wait_vmcnt<0>();
                prepare_v(i);
                prepare_v(i + 1);
                ring_barrier();
                if (i + 3 < nl) stage(kh, i + 3, kring);
                if (i + 4 < nl) stage(kh, i + 4, kring);
                if (i + 2 < nl) stage(vh, i + 2, vring);
                if (i + 3 < nl) stage(vh, i + 3, vring);
            }
            if (i < nw) step(i);
        }
    };
    run_pages();

    if constexpr (PK) {
        if (new_keys) {
            // ---- the last run: then the chunk's keys, from its rings ----
            // Once every wave is done with the rings, the keys of the
            // workgroup's rows (pages from the one holding key `position`
            // on) are prepared into them, and the same loop runs over them
            // with the rows' causal limits; keys before `position` are the
            // cached runs' and are masked.  The softmax state carries on.
            wait_vmcnt<0>();
            lds_barrier();
            from_lds = true;
            p0 = a.position / 32;
            n_keys = wg_keys;
            nl = max(0, (wg_keys + 31) / 32 - p0);
            nw = min(max((wave_keys + 31) / 32 - p0, 0), nl);
            limit = a.position + row_token;
            wave_first_limit = a.position + max(row0, 0) / a.group;
            key_lo = a.position;
            prep_new_keys();
            s[0] = s[1] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (nl > 0) first_scores();
            run_pages();
        }
    }

    l = row_group_sum(l);
    const int row = row0 + (lane & 15);
    if (a.splits > 1) {
        // ---- partial rows: unnormalised, with their max and sum ----
        if (row >= 0 && row < row_end) {
            const size_t part = (size_t)h * a.splits + split;
            const bool none = m == -INFINITY;   // no key of this split: empty
            constexpr bool EXACT_V = std::is_same<VT, __bf16>::value;
            if (!QSPLIT && a.half_parts) {
                // O / l (a convex combination of V rows: fp16 holds it to
                // 2^-11 relative when V is fp16).  As in the other 16-bit
                // partials, lane groups g and g^1 swap halves of each pair
                // of 16-dim tiles so that every lane stores 8 consecutive
                // dims (16 B; 64 contiguous bytes per row).  Swap partners
                // share their row, so both take part or neither does.
                typedef unsigned U2 __attribute__((ext_vector_type(2)));
                typedef _Float16 H4 __attribute__((ext_vector_type(4)));
                const float inv = none ? 0.f : 1.f / l;
                uint16_t *pa = reinterpret_cast<uint16_t *>(a.part_o) + (part * R + row) * D + 16 * (g & 1) + 4 * (g & 2);
                uint16_t *pb = pa + (size_t)a.kv_heads * a.splits * R * D;
                auto store_pair = [&](uint16_t *dst, U2 x, U2 y) __attribute__((always_inline)) {
                    const auto s0 = __builtin_amdgcn_permlane16_swap(x[0], y[0], false, false);
                    const auto s1 = __builtin_amdgcn_permlane16_swap(x[1], y[1], false, false);
                    *reinterpret_cast<U4 *>(dst) = U4{s0[0], s1[0], s0[1], s1[1]};
                };
#pragma unroll
                for (int dt = 0; dt < DT; dt += 2) {
                    const f32x4 x = acc[dt] * inv, y = acc[dt + 1] * inv;
                    if constexpr (EXACT_V) {
                        const U4 bx = __builtin_bit_cast(U4, x), by = __builtin_bit_cast(U4, y);
                        store_pair(pa + dt * 16, U2{(bx[0] >> 16) | (bx[1] & 0xFFFF0000u), (bx[2] >> 16) | (bx[3] & 0xFFFF0000u)},
                                   U2{(by[0] >> 16) | (by[1] & 0xFFFF0000u), (by[2] >> 16) | (by[3] & 0xFFFF0000u)});
                        store_pair(pb + dt * 16, U2{(bx[0] & 0xFFFFu) | (bx[1] << 16), (bx[2] & 0xFFFFu) | (bx[3] << 16)},
                                   U2{(by[0] & 0xFFFFu) | (by[1] << 16), (by[2] & 0xFFFFu) | (by[3] << 16)});
                    } else {
                        store_pair(pa + dt * 16,
                                   __builtin_bit_cast(U2, H4{(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]}),
                                   __builtin_bit_cast(U2, H4{(_Float16)y[0], (_Float16)y[1], (_Float16)y[2], (_Float16)y[3]}));
                    }
                }
            } else {
                float *po = a.part_o + (part * R + row) * D + 4 * g;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
                    *reinterpret_cast<f32x4 *>(po + dt * 16) = none ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[dt];
            }
            if (g == 0) {
                const float sum = none ? 0.f : l;
                a.part_ml[part * 2 * R + row] = m;
                a.part_ml[part * 2 * R + R + row] = !QSPLIT && a.half_parts && EXACT_V ? -sum : sum;
            }
        }
        return;
    }
    // ---- normalise and store rows ----
    if (row >= 0 && row < row_end) {
        const int t = row / a.group, gg = row - t * a.group;
        OUT *dst = static_cast<OUT *>(a.out) + ((size_t)t * a.q_heads + (size_t)h * a.group + gg) * D + 4 * g;
        const float inv = 1.f / l;
        // Gated output: times sigmoid(q_gate[t][head][D + d]) (rows of 2D).
        const float *gate = MODE == kOutGated
            ? a.gate + ((size_t)t * a.q_heads + (size_t)h * a.group + gg) * 2 * D + D + 4 * g : nullptr;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            typedef OUT OUT4 __attribute__((ext_vector_type(4)));
            OUT4 o;
#pragma unroll
            for (int r = 0; r < 4; ++r) o[r] = (OUT)(acc[dt][r] * inv);
            if constexpr (MODE == kOutGated) {
                const f32x4 gv = *reinterpret_cast<const f32x4 *>(gate + dt * 16);
#pragma unroll
                for (int r = 0; r < 4; ++r) o[r] *= 1.f / (1.f + expf(-gv[r]));
            }
            *reinterpret_cast<OUT4 *>(dst + dt * 16) = o;
        }
    }
}

// PREP = kPrepQuery: the fused path's chunk, its query prepared from q_gate
// (its keys appended by a launch before).
template <int D, typename KV, typename VT, bool PSPLIT, bool QSPLIT, int MODE, int ROWS, int PREP = 0>
__global__ __launch_bounds__(ROWS / 16 * kWave, 1)
void attention_prefill(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) KV kring[4 * 32 * D];
    __shared__ __attribute__((aligned(16))) VT vring[4 * 32 * D];
    __shared__ __attribute__((aligned(16))) float qn_stage[PREP ? ROWS / 16 : 1][PREP ? D : 1];
    prefill_rows<D, KV, VT, PSPLIT, QSPLIT, MODE, ROWS, -1, PREP>(a, kring, vring, a.v_pages, a.head_stride,
                                                                  &qn_stage[0][0]);
}

// The fused prefill chunk that prepares its own query and keys (PREP in
// prefill_rows): fp16 pages, precise query, gated output, 128 rows per
// workgroup.
__global__ __launch_bounds__(kPreciseRows / 16 * kWave, 1)
void attention_prefill_prep(PrefillArgs a) {
    constexpr int D = kModelHeadDim;
    __shared__ __attribute__((aligned(16))) _Float16 kring[4 * 32 * D];
    __shared__ __attribute__((aligned(16))) _Float16 vring[4 * 32 * D];
    __shared__ __attribute__((aligned(16))) float qn_stage[kPreciseRows / 16][D];
    prefill_rows<D, _Float16, _Float16, true, true, kOutGated, kPreciseRows, -1, kPrepQuery | kPrepKeys>(
        a, kring, vring, a.v_pages, a.head_stride, &qn_stage[0][0]);
}

// The precise rows in two passes of eight waves (192 rows per workgroup):
// one round of workgroups where 128-row ones would take two.  Between the
// passes every wave's output stores complete (the second pass's waits count
// its page loads only) and every wave has finished reading the rings.
template <int D, typename KV, typename VT, bool PSPLIT, bool QSPLIT, int MODE, int PREP = 0>
__global__ __launch_bounds__(8 * kWave, 1)
void attention_prefill_2pass(PrefillArgs a) {
    constexpr int ROWS = kPreciseTwoPassRows;
    __shared__ __attribute__((aligned(16))) KV kring[4 * 32 * D];
    __shared__ __attribute__((aligned(16))) VT vring[4 * 32 * D];
    __shared__ __attribute__((aligned(16))) float qn_stage[PREP ? 8 : 1][PREP ? D : 1];
    prefill_rows<D, KV, VT, PSPLIT, QSPLIT, MODE, ROWS, 0, PREP>(a, kring, vring, a.v_pages, a.head_stride,
                                                                 &qn_stage[0][0]);
    wait_vmcnt<0>();
    ring_barrier();
    prefill_rows<D, KV, VT, PSPLIT, QSPLIT, MODE, ROWS, 1, PREP>(a, kring, vring, a.v_pages, a.head_stride,
                                                                 &qn_stage[0][0]);
}

// bf16 pages: the workgroups of a KV head that the conversion pass did not
// flag multiply by the fp16 copy of V with one fp16 P; a flagged head's take
// the exact products (bf16 V, P as bf16 hi + lo parts).  Every wave reads
// the same words, so the choice is uniform.
template <int D, int MODE, int ROWS>
__global__ __launch_bounds__(ROWS / 16 * kWave, 1)
void attention_prefill_bf16(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) __bf16 kring[4 * 32 * D];
    __shared__ __attribute__((aligned(16))) uint16_t vring[4 * 32 * D];
    const uint32_t *f = a.v_flags + (size_t)(blockIdx.x % a.kv_heads) * a.flag_words;
    uint32_t any = 0;
    for (int i = threadIdx.x & 63; i < a.flag_words; i += 64) any |= f[i];
    if (__any(any != 0))
        prefill_rows<D, __bf16, __bf16, true, false, MODE, ROWS>(a, kring, reinterpret_cast<__bf16 *>(vring),
                                                                 a.v_pages, a.head_stride);
    else
        prefill_rows<D, __bf16, _Float16, false, false, MODE, ROWS>(a, kring, reinterpret_cast<_Float16 *>(vring),
                                                                    a.v_copy, a.v_copy_stride);
}

// Rows per workgroup (kPrefillRows, kernels.hpp): 192 (twelve waves, three
// per SIMD; 2048 tokens of six query heads per KV head make 64 workgroups
// per KV head, one round on 256 CUs).  A precise query (hi + lo parts) needs
// twice the query registers: kPreciseRows = 128 (eight waves, two per SIMD),
// or kPreciseTwoPassRows = 192 on the same eight waves in two passes
// (attention_prefill_2pass) when that saves rounds of workgroups.

// The raw instances: fp16 pages; bf16 pages, V through the conversion pass
// below (attention_prefill_bf16).
template <int D>
const void *prefill_kernel(Dtype dtype, bool out_f32) {
    constexpr int R = kPrefillRows;
    if (dtype == Dtype::BF16)
        return out_f32 ? (const void *)&attention_prefill_bf16<D, kOutF32, R>
                       : (const void *)&attention_prefill_bf16<D, kOutSame, R>;
    return out_f32 ? (const void *)&attention_prefill<D, _Float16, _Float16, false, false, kOutF32, R>
                   : (const void *)&attention_prefill<D, _Float16, _Float16, false, false, kOutSame, R>;
}

// The fused model path: fp16 pages, fp32 query as hi + lo parts, hi + lo P
// (the same precision as the split kernels' precise instance).
template <int D>
const void *precise_prefill_kernel(bool gated, int passes) {
    if (passes == 2)
        return gated ? (const void *)&attention_prefill_2pass<D, _Float16, _Float16, true, true, kOutGated>
                     : (const void *)&attention_prefill_2pass<D, _Float16, _Float16, true, true, kOutF32>;
    return gated ? (const void *)&attention_prefill<D, _Float16, _Float16, true, true, kOutGated, kPreciseRows>
                 : (const void *)&attention_prefill<D, _Float16, _Float16, true, true, kOutF32, kPreciseRows>;
}


// ---- V conversion pass (bf16 calls) ----
// The call's V pages (keys 0 .. position+tokens-1) of every KV head as fp16
// pages in the workspace, [kv_heads][pages][32*D], the slots past the last
// key zeroed.  Block (head, page) converts one page, every thread its 16-byte
// slots (all loads issued first), and writes one word: 1 if some slot (8
// keys of one dim, an operand's lane) is neither all zero nor has its
// largest magnitude in [2^-14, 65280] (a value the conversion cannot hold,
// or whose slot would lose precision).  Loads are non-temporal (each bf16
// page is read once); the fp16 copy keeps the default policy, the prefill
// kernel reads it next.
constexpr int kConvThreads = 256;

template <int D>
__global__ __launch_bounds__(kConvThreads)
void convert_v_pages(const __bf16 *v_pages, size_t head_stride, _Float16 *out, uint32_t *flags, int pages,
                     int n_keys) {
    typedef uint32_t U4 __attribute__((ext_vector_type(4)));
    constexpr int PAGE = 32 * D, SLOTS = PAGE / 8;   // 16-byte slots per page
    constexpr int PER = SLOTS / kConvThreads;
    static_assert(PER * kConvThreads == SLOTS, "slots divide over the threads");
    const int h = blockIdx.x / pages, p = blockIdx.x - h * pages;
    const U4 *src = reinterpret_cast<const U4 *>(v_pages + (size_t)h * head_stride + (size_t)p * PAGE);
    U4 *dst = reinterpret_cast<U4 *>(out + ((size_t)h * pages + p) * PAGE);
    U4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = __builtin_nontemporal_load(src + threadIdx.x + i * kConvThreads);
    bool ok = true;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = threadIdx.x + i * kConvThreads, g = (e >> 4) & 3;   // slot e: lane e % 64 of its 1 KiB chunk
        if (p * 32 + 32 > n_keys) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (p * 32 + v_slot_token(g, j) >= n_keys) v[i][j >> 1] &= (j & 1) ? 0x0000ffffu : 0xffff0000u;
        }
        uint32_t mx = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t m = v[i][k] & 0x7fff7fffu;
            mx = max(mx, max(m & 0xffffu, m >> 16));
        }
        ok = ok && (mx == 0 || (mx >= 0x3880u && mx <= 0x477fu));
#pragma unroll
        for (int k = 0; k < 4; ++k)
            v[i][k] = pack2(__uint_as_float(v[i][k] << 16), __uint_as_float(v[i][k] & 0xffff0000u), _Float16{});
        dst[e] = v[i];
    }
    const int bad = __syncthreads_or(!ok);
    if (threadIdx.x == 0) flags[blockIdx.x] = bad ? 1u : 0u;
}

// Workspace of a bf16 call: the fp16 copy, then one word per page.
struct ConvPlan {
    int pages;
    size_t flag_offset, bytes;
};

ConvPlan conv_plan(const Shape &s) {
    ConvPlan c;
    c.pages = (s.n_keys() + 31) / 32;
    const size_t copy = (size_t)s.kv_heads * c.pages * 32 * s.head_dim * 2;
    c.flag_offset = (copy + 255) / 256 * 256;
    c.bytes = c.flag_offset + ((size_t)s.kv_heads * c.pages * 4 + 255) / 256 * 256;
    return c;
}

// Key splits.  A prefill workgroup fills a CU (its LDS rings), so a call with
// fewer row workgroups (rows / 192, or / 128, times kv_heads) than the device
// has CUs leaves the rest idle: a 64-token chunk on a 16K prefix runs in 12
// workgroups.  Such a call splits every row workgroup's pages into up to
// CUs / row workgroups equal runs of at least kPrefillMinSplitPages pages,
// and combine_prefill merges the partial rows.  A call over fewer than
// kPrefillMinSplitKeyPages pages stays whole: a workgroup's fixed costs (its query
// load, first page loads and partial stores) outweigh the pages it would
// shed (300 tokens at 300: 27.8 us whole, 26 us for the split kernel alone).
// Neither does a call with at least as many row workgroups as CUs split:
// the precise 2048-token chunk (384 workgroups, 1.5 rounds) measured
// 610-709 us split in two against 669 us whole.

size_t split_partial_bytes(const Shape &s, int splits) {
    return splits > 1
        ? ((size_t)s.kv_heads * splits * s.group() * s.tokens * (s.head_dim + 2) * sizeof(float) + 255) / 256 * 256
        : 0;
}

}  // namespace

PrefillPlan plan_prefill_for(const Shape &s, Dtype dtype, bool precise, int cus) {
    PrefillPlan p;
    p.rows = precise ? kPreciseRows : kPrefillRows;
    p.row_wgs = (s.group() * s.tokens + p.rows - 1) / p.rows;
    const long long pages = ((long long)s.n_keys() + 31) / 32;
    const long long base = (long long)p.row_wgs * s.kv_heads;
    p.splits = 1;
    if (pages >= kPrefillMinSplitKeyPages && base < cus)
        p.splits = (int)std::max(1LL, std::min<long long>({cus / base, pages / kPrefillMinSplitPages,
                                                           kPrefillMaxSplits}));
    p.passes = 1;
    if (precise && p.splits == 1) {
        const long long rows = (long long)s.group() * s.tokens;
        const long long wgs2 = (rows + kPreciseTwoPassRows - 1) / kPreciseTwoPassRows;
        const long long rounds1 = (base + cus - 1) / cus, rounds2 = (wgs2 * s.kv_heads + cus - 1) / cus;
        if (3 * rounds2 < 2 * rounds1) {
            p.rows = kPreciseTwoPassRows;
            p.row_wgs = (int)wgs2;
            p.passes = 2;
        }
    }
    p.part_offset = dtype == Dtype::BF16 && !precise ? conv_plan(s).bytes : 0;
    p.bytes = p.part_offset + split_partial_bytes(s, p.splits);
    return p;
}

namespace {
PrefillPlan plan_prefill(const Shape &s, Dtype dtype, bool precise) {
    return plan_prefill_for(s, dtype, precise, device_cu_count());
}

// ---- combine of split prefill partials ----
// One wave per (row, KV head), lane l head dims DV*l .. DV*l+DV-1: the
// splits' (m, l) pairs (lane s holding split s's) and partial rows (fp32, or
// the 16-bit planes of PrefillArgs::half_parts, BATCH at a time, all in
// flight together) are merged in base 2 against the splits' largest max.
// A split that saw no key of the row stored max -inf, sum 0 and a zero row,
// and weighs 0.  Up to 64 splits (one per lane); the launcher sends at most
// kCombineWideBatch.  (Loading every split's m and l in every lane, the
// same address across the wave, took 72 loads per wave at 24 splits, each
// with a 64-bit address of its own, and the compiler then issued the rows in
// several rounds.  Fused 64-token chunk at 16,384, 21 splits: 63.36 -> 62.73
// us per layer; 512 bf16 tokens at 6144, 4 splits: 99.33 -> 97.89 us;
// medians of 5 in-process rounds each.)
struct CombinePrefillArgs {
    const float *part_o;
    const float *part_ml;
    void *out;
    const float *gate;
    int q_heads, group, rows, kv_heads, splits;
};
// Up to kCombineNarrowBatch splits take one round of 4 loads (no surplus
// loads, fewer registers: the 512-token bf16 chunk's 4-split combine took
// 6.84 against 7.16 us per call with rounds of 8, by a kernel trace of both
// in one process), up to 2 kCombineBatch rounds of 8, up to
// kCombineWideBatch one round of all of them (more registers per wave).
constexpr int kCombineBatch = 8, kCombineWideBatch = 24, kCombineNarrowBatch = 4, kCombineThreads = 256;
static_assert(kCombineWideBatch <= kWave, "combine_prefill holds one split's (m, l) per lane");

// HALF: the partial rows are PrefillArgs::half_parts planes (raw calls).
// Lane s < splits loads split s's max and sum (one load each for the wave),
// so the row loads are the wave's only other loads and all of them are in
// flight together: the global max and the weights exp2(m_s - M) come from
// lane reductions, and each split's weight reaches every lane by readlane.
template <int D, typename KV, int MODE, int BATCH, bool HALF>
__global__ __launch_bounds__(kCombineThreads)
void combine_prefill(CombinePrefillArgs c) {
    constexpr int DV = D / kWave;
    typedef float FV __attribute__((ext_vector_type(DV)));
    const int wave = blockIdx.x * (kCombineThreads / kWave) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (wave >= c.rows * c.kv_heads) return;
    const int h = wave / c.rows, row = wave - h * c.rows;
    typedef uint16_t HV __attribute__((ext_vector_type(DV)));
    const float *ml = c.part_ml + (size_t)h * c.splits * 2 * c.rows + row;
    const size_t e0 = ((size_t)h * c.splits * c.rows + row) * D + lane * DV;
    const float *po = c.part_o + e0;
    const uint16_t *pa = reinterpret_cast<const uint16_t *>(c.part_o) + e0;
    const uint16_t *pb = pa + (size_t)c.kv_heads * c.splits * c.rows * D;
    const size_t stride = (size_t)c.rows * D;
    const int sl = min(lane, c.splits - 1);
    const float ms = ml[(size_t)sl * 2 * c.rows];
    const float ls = ml[(size_t)sl * 2 * c.rows + c.rows];
    FV acc = {};
    float L = 0.f;
    for (int s0 = 0; s0 < c.splits; s0 += BATCH) {
        FV ov[BATCH];
        HV av[BATCH];
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
            const int sc = min(s0 + i, c.splits - 1);
            if constexpr (HALF) av[i] = *reinterpret_cast<const HV *>(pa + sc * stride);
            else ov[i] = *reinterpret_cast<const FV *>(po + sc * stride);
        }
        // The weights (the same every round).
        const float mv = lane < c.splits ? ms : -INFINITY;
        float M = fmaxf(mv, dpp_get<0xb1>(mv));
        M = fmaxf(M, dpp_get<0x4e>(M));
        M = fmaxf(M, dpp_get<0x141>(M));
        M = fmaxf(M, dpp_get<0x140>(M));
        M = row_group_max(M);
        const float mu = M == -INFINITY ? 0.f : M;
        // A negative sum (every split of a KV head alike) says the planes
        // hold fp32 halves.
        const bool exact = HALF && __builtin_signbit(__int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(ls))));
        const float lv = lane < c.splits ? (exact ? -ls : ls) : 0.f;
        const float wl = lane < c.splits ? __builtin_amdgcn_exp2f(mv - mu) : 0.f;
        if (s0 == 0) L = wave_sum_dpp(wl * lv);
        // HALF rows are O / l: weighted by l as well.
        const float wo = HALF ? wl * lv : wl;
        if constexpr (HALF) {
            if (exact) {
                HV bv[BATCH];
#pragma unroll
                for (int i = 0; i < BATCH; ++i)
                    bv[i] = *reinterpret_cast<const HV *>(pb + min(s0 + i, c.splits - 1) * stride);
#pragma unroll
                for (int i = 0; i < BATCH; ++i)
#pragma unroll
                    for (int d = 0; d < DV; ++d)
                        ov[i][d] = __uint_as_float(((uint32_t)av[i][d] << 16) | bv[i][d]);
            } else {
                typedef _Float16 FH __attribute__((ext_vector_type(DV)));
#pragma unroll
                for (int i = 0; i < BATCH; ++i) {
                    const FH fh = __builtin_bit_cast(FH, av[i]);
#pragma unroll
                    for (int d = 0; d < DV; ++d) ov[i][d] = (float)fh[d];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
            if (s0 + i < c.splits) {
                const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wo), s0 + i));
                acc += w * ov[i];
            }
        }
    }
    const float inv = 1.f / L;
    const int t = row / c.group, hq = h * c.group + (row - t * c.group);
    const size_t idx = ((size_t)t * c.q_heads + hq) * D + lane * DV;
    if constexpr (MODE == kOutSame) {
        typedef KV KVV __attribute__((ext_vector_type(DV)));
        KVV o;
#pragma unroll
        for (int d = 0; d < DV; ++d) o[d] = (KV)(acc[d] * inv);
        *reinterpret_cast<KVV *>(static_cast<KV *>(c.out) + idx) = o;
    } else {
        FV o = acc * inv;
        if constexpr (MODE == kOutGated) {
            const FV g = *reinterpret_cast<const FV *>(c.gate + ((size_t)t * c.q_heads + hq) * 2 * D + D + lane * DV);
#pragma unroll
            for (int d = 0; d < DV; ++d) o[d] *= 1.f / (1.f + expf(-g[d]));
        }
        *reinterpret_cast<FV *>(static_cast<float *>(c.out) + idx) = o;
    }
}

template <int D, int B>
const void *combine_prefill_pick(Dtype dtype, bool out_f32, bool gated, bool half) {
    // Gated (fused) and precise calls store fp32 rows, raw calls the planes.
    if (gated) return half ? nullptr : (const void *)&combine_prefill<D, float, kOutGated, B, false>;
    if (out_f32)
        return half ? (const void *)&combine_prefill<D, float, kOutF32, B, true>
                    : (const void *)&combine_prefill<D, float, kOutF32, B, false>;
    if (!half) return nullptr;
    return dtype == Dtype::BF16 ? (const void *)&combine_prefill<D, __bf16, kOutSame, B, true>
                                : (const void *)&combine_prefill<D, _Float16, kOutSame, B, true>;
}

template <int D>
const void *combine_prefill_kernel(Dtype dtype, bool out_f32, bool gated, int splits, bool half) {
    return splits > 2 * kCombineBatch ? combine_prefill_pick<D, kCombineWideBatch>(dtype, out_f32, gated, half)
         : splits > kCombineNarrowBatch ? combine_prefill_pick<D, kCombineBatch>(dtype, out_f32, gated, half)
                                        : combine_prefill_pick<D, kCombineNarrowBatch>(dtype, out_f32, gated, half);
}

}  // namespace

size_t prefill_workspace_bytes(const Shape &s, Dtype dtype, bool precise) {
    return plan_prefill(s, dtype, precise).bytes;
}

namespace {
// The combine of a call whose rows' keys were split into `splits` runs.  Up
// to kCombineWideBatch splits (many rows): combine_prefill, a wave per row,
// in rounds of 8 splits up to 16 and in one round of up to 24 beyond (the
// fused 64-token chunk at 16,384, 21 splits: 66.3 against 68.1 us per layer
// with attention_combine; the wide batch gave nothing at 9-16 splits).  More
// splits (then few row workgroups, few rows): attention_combine, whose four
// waves per row request up to 64 splits in one round (62 splits of 96 rows:
// 27.5 us per call against 31.1 us with combine_prefill's batches in turn).
void launch_prefill_combine(const Shape &s, Dtype dtype, const float *part_o, const float *part_ml, int splits,
                            bool half_parts, void *out, bool out_f32, const float *gate, hipStream_t stream) {
    const int rows = s.group() * s.tokens;
    if (splits > kCombineWideBatch) {
        require(!half_parts, "16-bit partial rows go to combine_prefill");
        SplitPlan cp = {};
        cp.kind = SplitKind::Stream;   // fp32 partial rows, default-policy stores
        cp.rows = rows;
        cp.splits = splits;
        launch_combine(s, cp, dtype, part_o, out, out_f32, gate, stream);
        return;
    }
    CombinePrefillArgs c;
    c.part_o = part_o;
    c.part_ml = part_ml;
    c.out = out;
    c.gate = gate;
    c.q_heads = s.q_heads;
    c.group = s.group();
    c.rows = rows;
    c.kv_heads = s.kv_heads;
    c.splits = splits;
    const long long waves = (long long)rows * s.kv_heads;
    const long long blocks = (waves + kCombineThreads / kWave - 1) / (kCombineThreads / kWave);
    require(blocks < (1LL << 31), "prefill combine exceeds the grid");
    const void *kernel = s.head_dim == 256 ? combine_prefill_kernel<256>(dtype, out_f32, gate != nullptr, splits, half_parts)
                                           : combine_prefill_kernel<128>(dtype, out_f32, gate != nullptr, splits, half_parts);
    require(kernel != nullptr, "no prefill combine for this partial format");
    void *cargs[] = {&c};
    check(hipLaunchKernel(kernel, dim3((unsigned)blocks), dim3(kCombineThreads), cargs, 0, stream));
}
}  // namespace

bool prefill_prep_fits(int tokens, int position) {
    return tokens > kMaxFusedSplitTokens && position >= 0 &&
           tokens + position % kPageTokens <= kPrepNewKeyPages * kPageTokens;
}

PrefillPlan plan_prefill_prep_for(int tokens, int position, int cus) {
    const Shape s{kModelQHeads, kModelKvHeads, kModelHeadDim, tokens, position, 0};
    PrefillPlan p;
    p.rows = kPreciseRows;
    p.row_wgs = (s.group() * tokens + p.rows - 1) / p.rows;
    p.passes = 1;
    // Runs over the cached pages as plan_prefill_for splits a call's pages
    // (the last run, the shortest, also takes the chunk's keys).
    const long long cached = ((long long)position + kPageTokens - 1) / kPageTokens;
    const long long base = (long long)p.row_wgs * s.kv_heads;
    p.splits = 1;
    if (cached >= kPrefillMinSplitKeyPages && base < cus)
        p.splits = (int)std::max(1LL, std::min<long long>({cus / base, cached / kPrefillMinSplitPages,
                                                           kPrefillMaxSplits}));
    p.part_offset = 0;
    p.bytes = split_partial_bytes(s, p.splits);
    return p;
}

size_t prefill_prep_workspace_bytes(int tokens, int position) {
    return prefill_prep_fits(tokens, position) ? plan_prefill_prep_for(tokens, position, device_cu_count()).bytes : 0;
}

void launch_prefill_prep(const FusedToken &tok, float *out, void *workspace, hipStream_t stream) {
    require(prefill_prep_fits(tok.tokens, tok.position), "the chunk's keys do not fit the prepared prefill's rings");
    const Shape s{kModelQHeads, kModelKvHeads, kModelHeadDim, tok.tokens, tok.position, 0};
    const PrefillPlan plan = plan_prefill_prep_for(tok.tokens, tok.position, device_cu_count());
    require(plan.bytes == 0 || workspace != nullptr, "this prefill needs its workspace");
    PrefillArgs a = {};
    a.gate = tok.q_gate;
    a.k_pages = tok.k_pages;
    a.v_pages = tok.v_pages;
    a.out = out;
    a.head_stride = tok.head_stride;
    a.q_heads = s.q_heads;
    a.kv_heads = s.kv_heads;
    a.group = s.group();
    a.rows = s.group() * s.tokens;
    a.position = s.position;
    a.n_tiles = plan.row_wgs;
    a.scale_log2 = (1.0f / 16.0f) * 1.4426950408889634f;
    a.splits = plan.splits;
    a.key = tok.key;
    a.value = tok.value;
    a.q_norm = tok.q_norm;
    a.k_norm = tok.k_norm;
    a.epsilon = tok.epsilon;
    a.tokens = tok.tokens;
    if (plan.splits > 1) {
        a.part_o = static_cast<float *>(workspace);
        a.part_ml = a.part_o + (size_t)s.kv_heads * plan.splits * a.rows * s.head_dim;
    }
    const long long grid = (long long)plan.row_wgs * s.kv_heads * plan.splits;
    void *args[] = {&a};
    check(hipLaunchKernel((const void *)&attention_prefill_prep, dim3((unsigned)grid), dim3(kPreciseRows / 16 * kWave),
                          args, 0, stream));
    if (plan.splits > 1)
        launch_prefill_combine(s, Dtype::F16, a.part_o, a.part_ml, plan.splits, false, out, true, tok.q_gate, stream);
}

void launch_prefill_fused(const FusedToken &tok, float *out, void *workspace, hipStream_t stream) {
    const Shape s{kModelQHeads, kModelKvHeads, kModelHeadDim, tok.tokens, tok.position, 0};
    const PrefillPlan plan = plan_prefill(s, Dtype::F16, true);
    require(plan.bytes == 0 || workspace != nullptr, "this prefill needs its workspace");
    PrefillArgs a = {};
    a.gate = tok.q_gate;
    a.k_pages = tok.k_pages;
    a.v_pages = tok.v_pages;
    a.out = out;
    a.head_stride = tok.head_stride;
    a.q_heads = s.q_heads;
    a.kv_heads = s.kv_heads;
    a.group = s.group();
    a.rows = s.group() * s.tokens;
    a.position = s.position;
    a.n_tiles = plan.row_wgs;
    a.scale_log2 = (1.0f / 16.0f) * 1.4426950408889634f;
    a.splits = plan.splits;
    a.q_norm = tok.q_norm;
    a.k_norm = tok.k_norm;
    a.epsilon = tok.epsilon;
    a.tokens = tok.tokens;
    if (plan.splits > 1) {
        a.part_o = reinterpret_cast<float *>(static_cast<char *>(workspace) + plan.part_offset);
        a.part_ml = a.part_o + (size_t)s.kv_heads * plan.splits * a.rows * s.head_dim;
    }
    const int threads = (plan.passes == 2 ? 8 : plan.rows / 16) * kWave;
    const long long grid = (long long)plan.row_wgs * s.kv_heads * plan.splits;
    require(grid * threads < (1LL << 32), "prefill launch exceeds 2^32 work-items");
    constexpr int D = kModelHeadDim;
    const void *kernel =
        plan.passes == 2
            ? (const void *)&attention_prefill_2pass<D, _Float16, _Float16, true, true, kOutGated, kPrepQuery>
            : (const void *)&attention_prefill<D, _Float16, _Float16, true, true, kOutGated, kPreciseRows, kPrepQuery>;
    void *args[] = {&a};
    check(hipLaunchKernel(kernel, dim3((unsigned)grid), dim3(threads), args, 0, stream));
    if (plan.splits > 1)
        launch_prefill_combine(s, Dtype::F16, a.part_o, a.part_ml, plan.splits, false, out, true, tok.q_gate, stream);
}

void launch_prefill(const Shape &s, Dtype dtype, bool precise, float scale, const void *q,
                    const void *q_lo, const void *k_pages, const void *v_pages, void *out, bool out_f32,
                    const float *gate, void *workspace, hipStream_t stream) {
    require(!gate || precise, "a gated prefill needs the precise query");
    require(!precise || (dtype == Dtype::F16 && out_f32 && q_lo), "a precise prefill runs on fp16 pages with fp32 output");
    require(s.head_dim == 256 || s.head_dim == 128, "unsupported head_dim for the prefill kernel");
    const PrefillPlan plan = plan_prefill(s, dtype, precise);
    require(plan.bytes == 0 || workspace != nullptr, "this prefill needs its workspace");
    PrefillArgs a = {};
    a.q = q;
    a.q_lo = q_lo;
    a.gate = gate;
    a.k_pages = k_pages;
    a.v_pages = v_pages;
    a.out = out;
    a.head_stride = (size_t)s.capacity * s.head_dim;
    a.q_heads = s.q_heads;
    a.kv_heads = s.kv_heads;
    a.group = s.group();
    a.rows = s.group() * s.tokens;
    a.position = s.position;
    a.n_tiles = plan.row_wgs;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.splits = plan.splits;
    if (plan.splits > 1) {
        a.part_o = reinterpret_cast<float *>(static_cast<char *>(workspace) + plan.part_offset);
        a.part_ml = a.part_o + (size_t)s.kv_heads * plan.splits * a.rows * s.head_dim;
        // Raw rows that combine_prefill merges travel as 16-bit planes.
        a.half_parts = !precise && plan.splits <= kCombineWideBatch;
    }
    const bool d256 = s.head_dim == 256;
    const int threads = (plan.passes == 2 ? 8 : plan.rows / 16) * kWave;
    const long long grid = (long long)plan.row_wgs * s.kv_heads * plan.splits;
    require(grid * threads < (1LL << 32), "prefill launch exceeds 2^32 work-items");
    void *args[] = {&a};
    auto combine = [&] {
        if (plan.splits > 1)
            launch_prefill_combine(s, dtype, a.part_o, a.part_ml, plan.splits, a.half_parts != 0, out, out_f32, gate,
                                   stream);
    };
    if (precise) {
        const void *kernel = d256 ? precise_prefill_kernel<256>(gate != nullptr, plan.passes)
                                  : precise_prefill_kernel<128>(gate != nullptr, plan.passes);
        check(hipLaunchKernel(kernel, dim3((unsigned)grid), dim3(threads), args, 0, stream));
        combine();
        return;
    }
    if (dtype == Dtype::BF16) {
        // V pages to fp16 with their range words, then the prefill (which
        // takes the exact products on a flagged KV head).
        const ConvPlan c = conv_plan(s);
        _Float16 *copy = static_cast<_Float16 *>(workspace);
        uint32_t *flags = reinterpret_cast<uint32_t *>(static_cast<char *>(workspace) + c.flag_offset);
        const int conv_blocks = c.pages * s.kv_heads;
        if (d256)
            convert_v_pages<256><<<conv_blocks, kConvThreads, 0, stream>>>(
                static_cast<const __bf16 *>(v_pages), a.head_stride, copy, flags, c.pages, s.n_keys());
        else
            convert_v_pages<128><<<conv_blocks, kConvThreads, 0, stream>>>(
                static_cast<const __bf16 *>(v_pages), a.head_stride, copy, flags, c.pages, s.n_keys());
        check(hipGetLastError());
        a.v_copy = copy;
        a.v_copy_stride = (size_t)c.pages * 32 * s.head_dim;
        a.v_flags = flags;
        a.flag_words = c.pages;
    }
    const void *kernel = d256 ? prefill_kernel<256>(dtype, out_f32) : prefill_kernel<128>(dtype, out_f32);
    check(hipLaunchKernel(kernel, dim3((unsigned)grid), dim3(threads), args, 0, stream));
    combine();
}

}  // namespace rs
