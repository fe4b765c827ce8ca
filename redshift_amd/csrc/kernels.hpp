// Host-side launchers shared by the C-ABI layer (abi.cpp) and the kernel
// translation units.  All launches are asynchronous on the given stream.
#pragma once
#include "common.hpp"

namespace rs {

enum class Dtype { F16 = 1, BF16 = 2 };

// Geometry of one raw attention call: `tokens` query tokens whose first token
// sits at `position`; row t (0-based) sees keys 0 .. position + t.
struct Shape {
    int q_heads, kv_heads, head_dim, tokens, position, capacity;
    int group() const { return q_heads / kv_heads; }
    int n_keys() const { return position + tokens; }
};

enum class SplitKind { Stream, Ring };

// What a split kernel or the combine writes: the KV type, fp32, or fp32
// times sigmoid(gate) (gate = q_gate[t][h][D + d], rows of 2D floats); or,
// for a split kernel, its partial rows (the combine then writes the output).
enum { kOutSame = 0, kOutF32 = 1, kOutGated = 2, kOutPartials = 3 };

// The new tokens of a fused call (the reference's attn_prepare inputs for
// the 24/4/256 model), token t seeing new keys 0..t.  The split kernel
// prepares the query and attends to the cached keys; its first split's
// workgroups also prepare the new keys and values and append them to the
// pages.  One or two tokens (the stream kernel): the first split publishes
// the prepared query rows in q_prep, and the combine adds the new keys from
// the pages and q_prep.  3..8 tokens (the ring kernel): the first split
// attends to the new keys itself.
struct FusedToken {
    const float *q_gate;   // [tokens][q_heads][2D]: q, then the gate
    const float *key;      // [tokens][kv_heads][D]
    const float *value;    // [tokens][kv_heads][D]
    const float *q_norm;   // [D]
    const float *k_norm;   // [D]
    void *k_pages;
    void *v_pages;
    size_t head_stride;
    float epsilon;
    int position;          // token 0's position: RoPE angles and page slots
    int tokens;
    float *q_prep;         // [kv_heads][tokens * group][D] prepared fp32 queries
};

// Arguments of every split-K partial kernel.
struct SplitArgs {
    const void *q;        // [tokens][q_heads][D] 16-bit (hi part when QSPLIT)
    const void *q_lo;     // QSPLIT: lo part, same layout
    const void *k_pages;
    const void *v_pages;
    float *part_o;    // [kv_heads][splits][rows][D]   unnormalised, base-2 max m
    float *part_ml;   // [kv_heads][splits][2][rows]   m (log2 domain), then l
    size_t head_stride;
    int q_heads, kv_heads, group, rows, position, n_keys, n_pages, splits;
    float scale_log2;
    FusedToken tok;       // the prepared-query instances' inputs (stream: 1-2 tokens, ring: 3-8)
    void *out;            // direct output: [tokens][q_heads][D] (one split per KV head)
};

// attention_ring instance (ring.hip) for head_dim D (128 or 256), nqt query
// tiles (1..3) and output mode (kOutPartials, or a direct output: kOutSame
// and kOutF32 for 16-bit queries, kOutF32 for precise ones);
// precise (fp32 hi + lo) queries run on fp16 pages only.  nullptr for other
// combinations.  It takes kRingThreads threads and SplitArgs.
constexpr int kRingThreads = 512;
const void *ring_kernel(int D, int nqt, Dtype dtype, bool precise, int out_mode);
// The fused verification's ring instance (24/4/256, fp16 pages, 2 or 3
// query tiles): the query prepared in the kernel from SplitArgs::tok, every
// row over the cached keys 0 .. position only, fp32 partials.
const void *ring_prep_kernel(int nqt);

// The split-K decomposition chosen for one launch of the partial kernel.
struct SplitPlan {
    SplitKind kind;  // attention_stream (one query tile) or attention_ring
    int nqt;         // 16-row query tiles per KV head (rows = group * tokens)
    int rows;        // valid query rows per KV head
    int n_pages;     // 32-key pages per KV head holding keys 0..n_keys-1
    int splits;      // workgroups per KV head
    bool half_parts; // partial rows stored as fp16 O / l (the raw fp16 ring kernel)
    bool direct;     // one split per KV head that writes the output itself (no combine)
};

// Contexts of up to kDirectStreamPages (decode) or kDirectRingPages
// (verification) pages per KV head run in one workgroup per KV head, which
// writes the output rows directly: a short context is bound by latency, and
// the combine launch costs more than the split-K parallelism gains.  Measured
// on 16 layers in a graph (fp16, 24/4/256): one token at 16..240 cached keys
// 5.2..8.4 us against 8.7..9.8 us with split + combine; eight tokens at 16,
// 64, 128, 240 keys 6.0, 7.9, 9.4, 12.2 us against 9.1, 9.2, 9.4, 9.5 us.
constexpr int kDirectStreamPages = 8, kDirectRingPages = 4;

// Largest number of query rows (group * tokens) per KV head that one launch of
// the split kernel holds; longer token runs are processed in chunks.
constexpr int kMaxRows = 48;
// Largest q_heads * tokens of one raw attention call.
constexpr long long kMaxQueryRows = 1LL << 28;

int device_cu_count();
// allow_direct: the caller writes the output with the split kernel when the
// plan is direct (qv_attention's ungated calls); the two-phase entry points
// and gated outputs always combine (the combine requests the gate with the
// partials, where a direct split would wait one more round trip for it).
SplitPlan plan_split(const Shape &s, int chunk_tokens, Dtype dtype, bool precise, bool allow_direct = false);
// plan_split on `cus` CUs of which each holds resident_per_cu(plan, D,
// dtype, precise) workgroups of the chosen split kernel: no device query
// (plan_split passes the current device's figures).
SplitPlan plan_split_for(const Shape &s, int chunk_tokens, Dtype dtype, bool precise, bool allow_direct,
                         int cus, int (*resident_per_cu)(const SplitPlan &, int D, Dtype, bool));
// Tokens per chunk for a shape (chunk_tokens * group <= kMaxRows).
int chunk_tokens(const Shape &s);
// Workspace bytes for qv_attention on this shape (largest chunk, as if every
// chunk combined its partials: an upper bound that also serves the two-phase
// entry points).
size_t attention_workspace_bytes(const Shape &s, Dtype dtype, bool precise);

// Split-K partial kernel over the pages of every KV head.  q is 16-bit of
// `dtype`, [tokens][q_heads][D]; when `precise` (fp16 only) q and q_lo are
// the hi and lo parts of an fp32 query.
// Partial buffers of one plan: o [kv_heads][splits][rows][D] float32
// (unnormalised), or fp16 O / l in the first half of that region when
// plan.half_parts, then m and l [kv_heads][splits][2][rows] float32.
size_t plan_bytes(const Shape &s, const SplitPlan &p);
// A direct plan writes out (fp32 when out_f32, else `dtype`) instead of
// the workspace.
void launch_split(const Shape &s, const SplitPlan &plan, Dtype dtype, bool precise,
                  float scale, const void *q, const void *q_lo, const void *k_pages,
                  const void *v_pages, void *workspace, hipStream_t stream,
                  void *out = nullptr, bool out_f32 = false);
// Log-sum-exp combine of the partials into out.  Raw mode writes `dtype`
// [tokens][q_heads][D]; fused mode (gate != nullptr) writes float32 and
// multiplies by sigmoid(gate), gate being q_gate[t][h][D + d] (row stride 2D).
void launch_combine(const Shape &s, const SplitPlan &plan, Dtype dtype,
                    const void *workspace, void *out, bool out_f32, const float *gate,
                    hipStream_t stream);

// Fused decode or verification of tok.tokens new tokens (up to
// kMaxFusedSplitTokens) at tok.position >= 1 (24/4/256, fp16 pages) in two
// launches: the split kernel prepares the query itself (RMSNorm, gamma,
// RoPE, hi + lo parts) while its first pages are in flight and attends to
// the cached keys 0 .. position-1, its first split appending the new keys
// and values; the combine merges and applies the gate.  No prepare launch.
// One or two tokens run the stream kernel, and the combine adds the new
// keys (from the pages and the published query rows); 3..8 tokens run the
// ring kernel, whose first split attends to the new keys as one more block.
// The workspace holds the split's partials and the prepared query rows
// (fused_tokens_workspace_bytes).
void launch_fused_tokens(const FusedToken &tok, int capacity, void *workspace, float *out, hipStream_t stream);
size_t fused_tokens_workspace_bytes(int tokens, int position);
constexpr int kMaxFusedSplitTokens = 8;

// The fused k_attention of up to kShortMaxTokens new tokens when position +
// tokens <= kShortFusedKeys (short.hip): one launch, one workgroup per (token,
// KV head) that prepares its query rows and the new keys, appends its token's
// key and value, attends to the cached and the new keys and gates the rows.
// No workspace.
constexpr int kShortMaxTokens = 8, kShortFusedKeys = 256;
void launch_fused_short(const FusedToken &tok, float *out, hipStream_t stream);

// Chunked prefill: all group*tokens query rows against the pages; `dtype` q
// and out, [tokens][q_heads][D].  A precise call (fp16 pages) takes the query
// as hi + lo fp16 parts and writes fp32, times sigmoid of the gate half of
// q_gate [tokens][q_heads][2D] when `gate` is given.  A raw bf16 call first
// converts the call's V pages to fp16 in the workspace, with one range word
// per page (the prefill kernel takes the exact bf16 products on a KV head
// whose V leaves the fp16 range).  A call with too few row workgroups to fill
// the device splits their pages over more workgroups, whose fp32 partial
// rows (in the workspace, after the V copy) the combine kernel merges.
// prefill_workspace_bytes: the workspace of a call (0 when it needs none).
size_t prefill_workspace_bytes(const Shape &s, Dtype dtype, bool precise);

// The prefill's launch plan for a device of `cus` CUs: rows per workgroup
// (kPrefillRows, or kPreciseRows for a precise query), row workgroups per
// KV head, key splits (1, or up to kPrefillMaxSplits runs of at least
// kPrefillMinSplitPages pages when the row workgroups number fewer than the
// CUs and the call covers at least kPrefillMinSplitKeyPages pages; at most
// one workgroup per CU then), and its workspace: a raw bf16 call's fp16 V
// copy and range words, then (at part_offset) the split partials.  A
// precise call without key splits whose 128-row workgroups would need more
// rounds over the CUs than 1.5 times those of 192-row ones takes
// kPreciseTwoPassRows rows per workgroup in two passes of its eight waves
// (passes = 2): the later 128 rows first, then the earliest 64 rows, which
// see the fewest keys, on four of the waves.
constexpr int kPrefillRows = 192, kPreciseRows = 128, kPreciseTwoPassRows = 192;
constexpr int kPrefillMinSplitPages = 8, kPrefillMinSplitKeyPages = 32, kPrefillMaxSplits = 64;
struct PrefillPlan {
    int rows;            // query rows per workgroup
    int row_wgs;         // workgroups of rows per KV head
    int splits;
    int passes;          // 1, or 2 (a precise call, eight waves over 192 rows)
    size_t part_offset;  // split partials in the workspace
    size_t bytes;        // workspace
};
PrefillPlan plan_prefill_for(const Shape &s, Dtype dtype, bool precise, int cus);
void launch_prefill(const Shape &s, Dtype dtype, bool precise, float scale, const void *q,
                    const void *q_lo, const void *k_pages, const void *v_pages, void *out, bool out_f32,
                    const float *gate, void *workspace, hipStream_t stream);

// The fused prefill chunk of tok.tokens new tokens (more than
// kMaxFusedSplitTokens) whose keys fit kPrepNewKeyPages pages from the one
// holding key tok.position (prefill_prep_fits), in at most two launches and
// no prepare launch: attention_prefill_prep's workgroups prepare their own
// query rows (RMSNorm, gamma, RoPE, hi + lo parts) and attend to runs of the
// cached keys 0 .. position-1 (split as plan_prefill_for splits a call's
// pages); the last run then prepares the chunk's keys into its LDS rings
// (its workgroup 0 appends them) and attends to them; the gated combine
// merges the runs (none for one run).  plan_prefill_prep_for gives the plan
// on `cus` CUs; the workspace holds the fp32 partials.
constexpr int kPrepNewKeyPages = 4;
bool prefill_prep_fits(int tokens, int position);
PrefillPlan plan_prefill_prep_for(int tokens, int position, int cus);
size_t prefill_prep_workspace_bytes(int tokens, int position);
void launch_prefill_prep(const FusedToken &tok, float *out, void *workspace, hipStream_t stream);
// A fused prefill chunk too long for launch_prefill_prep, after its keys and
// values were appended (launch_prepare, keys_only): the precise, gated
// prefill with its query prepared from q_gate in the kernel, then the gated
// combine when its keys are split.  workspace: prefill_workspace_bytes of
// the chunk's precise fp16 shape.
void launch_prefill_fused(const FusedToken &tok, float *out, void *workspace, hipStream_t stream);

// Whole pages 0 .. pages-1 of every KV head, K and V, from caches of
// src_capacity tokens to caches of dst_capacity tokens (checkpoint/restore).
void launch_copy(void *dst_k, void *dst_v, const void *src_k, const void *src_v, int kv_heads,
                 int head_dim, int dst_capacity, int src_capacity, int pages, hipStream_t stream);

// Token-major rows [count][kv_heads][D] <-> pages, for tokens first..first+count.
void launch_pack(void *k_pages, void *v_pages, const void *k_rows, const void *v_rows,
                 int kv_heads, int head_dim, int capacity, int first, int count,
                 hipStream_t stream);
void launch_unpack(void *k_rows, void *v_rows, const void *k_pages, const void *v_pages,
                   int kv_heads, int head_dim, int capacity, int first, int count,
                   hipStream_t stream);

// An fp32 query [n] as two fp16 arrays [2][n]: hi = fp16(q), lo = fp16(q -
// hi) (the B operands of the precise kernel instances).
void launch_split_query(void *q_hilo, const float *q, size_t n, hipStream_t stream);

// RMSNorm + RoPE of q and k, fp16 append of k and v into the pages at
// position..position+batch-1 (the reference's attn_prepare semantics for the
// fixed 24/4/256 model).  Writes the prepared fp32 q as two fp16 arrays
// [2][batch][24][256]: hi = fp16(q), lo = fp16(q - hi); keys_only: k and v
// alone (q_hilo unused), for a prefill that prepares its query itself.
void launch_prepare(void *q_hilo, void *k_pages, void *v_pages, const float *q_gate,
                    const float *key, const float *value, const float *q_norm,
                    const float *k_norm, int batch, int position, int capacity,
                    float epsilon, hipStream_t stream, bool keys_only = false);

}  // namespace rs
