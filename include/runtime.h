#ifndef QVELOX_RUNTIME_H
#define QVELOX_RUNTIME_H
/* libredshift_hip: the full-attention path of the qvelox runtime for AMD
 * Instinct MI355X (gfx950).
 *
 * The first part keeps the reference's C ABI byte for byte (src/runtime.h:9-74
 * of the reference); qv_test_attention has its full semantics and the entry
 * points outside the attention path are exported so that the reference's
 * ctypes loader (qvelox/runtime.py:6-22) resolves them, but return -1 with a
 * message.  The second part adds device-pointer, stream-ordered entry points
 * for the raw attention core on the paged KV cache. */
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Synchronous kernel validation ABI. All pointers refer to host memory.
 * Returns 0 on success, -1 on failure. qv_error() describes the last failure
 * on the calling thread, until its next ABI call. Caller owns buffer lengths.
 * These entry points include allocation and transfers: do not time them as
 * model inference. Batch sizes are 1..8. */
/* Replaces qv_error, src/runtime.cu:79 (thread-local message, "" after success). */
const char *qv_error(void);
/* Exported for loader compatibility (src/runtime.cu:81-114): quantized
 * projections are not part of this library; always returns -1. */
int qv_test_mm(float *out, const void *weights, const float *x,
               int kind, int batch, int width, int rows);
int qv_test_mm_fast(float *out, const void *weights, const float *x,
               int kind, int batch, int width, int rows);
/* Exported for loader compatibility (src/runtime.cu:116-129); returns -1. */
int qv_test_norm(float *out, const float *x, const float *weights,
                 int batch, int width, float epsilon);
/* Exported for loader compatibility (src/runtime.cu:131-165); returns -1. */
int qv_test_delta(float *out, float *state, float *history,
                  const float *qkv, const float *gate,
                  const float *alpha, const float *beta,
                  const float *conv, const float *decay,
                  const float *bias, const float *norm,
                  int batch, int key_heads, int value_heads, int dim,
                  float epsilon);

/* Fixed model attention: 24 query heads, 4 KV heads, head dimension 256.
 * out: [batch,24,256]; q_gate: [batch,24,512]; key/value: [batch,4,256];
 * q_norm/k_norm: [256]. Caches (in/out) hold IEEE float16 bits as
 * [position+batch,4,256]. Only the prefix [0,position) is read from host.
 * 0 <= position and position+batch <= 139264.
 * Replaces qv_test_attention, src/runtime.cu:167-197 (same validation order:
 * batch, epsilon, position, null pointers, all before any buffer is read). */
int qv_test_attention(float *out, void *key_cache, void *value_cache,
                      const float *q_gate, const float *key, const float *value,
                      const float *q_norm, const float *k_norm,
                      int batch, int position, float epsilon);

/* Model ABI (src/runtime.h:47-74 of the reference). The model session needs
 * the quantized projections and recurrent layers, which are not part of this
 * library: every call returns -1 (qv_create also stores NULL in *handle) and
 * qv_destroy does nothing. Declared so the header stays a drop-in. */
int qv_create(void **handle, const char *path, int context, float epsilon);
int qv_upload(void *handle, int slot, uint64_t offset, uint64_t length);
int qv_evaluate(void *handle, const int *tokens, int batch, float *out);
int qv_verify(void *handle, const int *tokens, int batch, float *out);
int qv_commit(void *handle, int accepted);
int qv_advance(void *handle, const int *tokens, int batch, int *next);
int qv_reset(void *handle);
int qv_checkpoint(void *handle);
int qv_restore(void *handle);
int qv_position(void *handle, int *position);
void qv_destroy(void *handle);

/* ------------------------------------------------------------------------
 * Device ABI (additive; no counterpart in the reference, whose kernels are
 * reachable only through the host-pointer test entry and the model session).
 * All pointers are device memory on the current HIP device, 16-byte aligned.
 * `stream` is a hipStream_t (NULL = the null stream). Calls only enqueue work:
 * they return before it runs and do not synchronize. Returns 0 or -1 with
 * qv_error() set; validation happens before anything is enqueued.
 *
 * KV cache: per KV head a contiguous run of `capacity` tokens (a multiple of
 * 32) in 32-token pages laid out in matrix-core operand order; K and V are
 * separate allocations of qv_kv_bytes() bytes each. Element type is 16-bit
 * (fp16 or bf16, chosen by the caller per call). Element (token p, dim d)
 * of KV head h sits at h*capacity*D plus
 *   K: (p/32)*32*D + (p%32/16)*16*D + (d/8)*128 + (p%16)*8 + d%8
 *   V: (p/32)*32*D + (d/16)*512 + ((p/4)%4)*128 + (d%16)*8 + (p%32/16)*4 + p%4
 * (elements, not bytes); qv_kv_pack / qv_kv_unpack convert token-major rows.
 * Query row t (0-based) of a call at `position` sees keys 0..position+t.
 * ---------------------------------------------------------------------- */
#define QV_F16 1
#define QV_BF16 2
#define QV_F32 3 /* output type only */

/* Bytes of one K (or V) cache: kv_heads * capacity * head_dim * 2. */
int qv_kv_bytes(uint64_t *bytes, int kv_heads, int head_dim, int capacity);
/* Copy token-major rows [count][kv_heads][head_dim] (16-bit) into the pages
 * of tokens first..first+count-1; either K or V side may be NULL. */
int qv_kv_pack(void *k_pages, void *v_pages, const void *k_rows, const void *v_rows,
               int kv_heads, int head_dim, int capacity, int first, int count,
               void *stream);
/* Inverse of qv_kv_pack. */
int qv_kv_unpack(void *k_rows, void *v_rows, const void *k_pages, const void *v_pages,
                 int kv_heads, int head_dim, int capacity, int first, int count,
                 void *stream);

/* Checkpoint / restore of the valid prefix (the reference's copy_state for
 * the full-attention layers, src/runtime.cu:455-485, which copies
 * prefix*kv_heads*head_dim fp16 values of each cache): copies the pages that
 * hold tokens 0..tokens-1 of every KV head, K and V, from caches of
 * src_capacity tokens to caches of dst_capacity tokens (whole pages, so up to
 * 31 tokens past the prefix come along; they are unreachable, as in the
 * reference). A snapshot needs capacity tokens rounded up to 32 only. */
int qv_kv_copy(void *dst_k, void *dst_v, const void *src_k, const void *src_v,
               int kv_heads, int head_dim, int dst_capacity, int src_capacity, int tokens,
               void *stream);

/* Workspace bytes that qv_attention needs for this shape on the current
 * device: split-K partials, or a prefill's fp16 V copy (bf16 pages) and key
 * split partials; the larger of the fp16 and bf16 page types. */
int qv_attention_workspace(uint64_t *bytes, int q_heads, int kv_heads, int head_dim,
                           int tokens, int position);
/* Raw causal GQA attention core, the reference's attention / attention_tiled
 * (src/kernels.cu:435-456,466-503) without prepare and gate, generalised to
 * q_heads/kv_heads/head_dim/scale: out[t][h] = softmax_p(q[t][h] . k[p][h/G] *
 * scale, p <= position+t) . v[p][h/G], G = q_heads/kv_heads.
 * q: [tokens][q_heads][head_dim] of `dtype` (QV_F16 or QV_BF16), like the
 * pages; out: same shape, of `out_dtype` (`dtype`, or QV_F32 as the
 * reference's float output); fp32 softmax and accumulation. head_dim 128 or
 * 256; G <= 48; 1 <= tokens; q_heads*tokens <= 2^28; position+tokens <=
 * capacity. Up to 48 query
 * rows per KV head (G*tokens): split-K over all CUs plus a log-sum-exp
 * combine (qv_attention_split then qv_attention_combine). More rows (chunked
 * prefill): one workgroup per 192 rows streams the visible pages through LDS.
 * Its workspace holds, for bf16 pages, an fp16 copy of the call's V pages,
 * and, for a call with fewer such workgroups than the device has CUs (a short
 * chunk on a long prefix), the fp32 partial rows of its key splits; an fp16
 * call that needs neither takes 0 bytes and the pointer may be NULL. */
int qv_attention(void *out, const void *q, const void *k_pages, const void *v_pages,
                 int dtype, int out_dtype, int q_heads, int kv_heads, int head_dim,
                 int tokens, int position, int capacity, float scale,
                 void *workspace, uint64_t workspace_bytes, void *stream);
/* The two phases of qv_attention for one token chunk (G*tokens <= 48), for
 * callers that time or schedule them separately. The workspace carries each
 * split's row max and sum (fp32) and its partial output rows: fp32, or, on
 * fp16 pages with 17..48 rows per KV head, fp16 rows normalised by their sum
 * (2^-11 relative, like the fp16 output). A combine reads what the split of
 * the same shape and dtype wrote. */
int qv_attention_split(const void *q, const void *k_pages, const void *v_pages,
                       int dtype, int q_heads, int kv_heads, int head_dim,
                       int tokens, int position, int capacity, float scale,
                       void *workspace, uint64_t workspace_bytes, void *stream);
int qv_attention_combine(void *out, int dtype, int out_dtype, int q_heads, int kv_heads, int head_dim,
                         int tokens, int position, const void *workspace,
                         uint64_t workspace_bytes, void *stream);

/* qv_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  It
 * runs the same kernels, and gives the same bits, as qv_attention; the
 * workspace (split-K partials, a bf16 prefill's fp16 copy of its V pages,
 * a split prefill's partials) lives in a static device array of 64 MiB per
 * GPU, held until the process ends (the largest split-K plan on a 256-CU
 * MI355X takes 12.1 MiB, a bf16 prefill kv_heads*keys*head_dim*2 bytes, a
 * split prefill's partials at most about 51 MB at head_dim 256; a shape that
 * needs more is refused).  The call itself allocates
 * nothing.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (concurrent streams, or threads) race on it, so
 * serialise them.  No kernel reads a partial it has not written in the same
 * call, so the array needs no clearing. */
int qv_attention_noalloc(void *out, const void *q, const void *k_pages, const void *v_pages,
                         int dtype, int out_dtype, int q_heads, int kv_heads, int head_dim,
                         int tokens, int position, int capacity, float scale, void *stream);

/* Workspace bytes of qv_attention_precise for this shape. */
int qv_attention_precise_workspace(uint64_t *bytes, int q_heads, int kv_heads, int head_dim,
                                   int tokens, int position);
/* The raw core at the reference's own precision: an fp32 query on fp16
 * pages, fp32 output.  The reference's attention kernels read q as fp32
 * (written by attn_prepare, src/kernels.cu:416-434, read at :435-503) from
 * fp16 caches.  The library splits q into fp16 parts hi = fp16(q) and
 * lo = fp16(q - hi) (in the decode kernel itself for up to 16 query rows
 * per KV head, otherwise staged at the start of the workspace by a launch
 * of their own) and multiplies both by K; P multiplies V as hi + lo parts
 * too.  The parts hold q to
 * about 22 significant bits: |q| < 65504, error at most
 * 2^-25 + 2^-22 |q|.  q and out: [tokens][q_heads][head_dim] float32;
 * shapes, limits and kernels otherwise as qv_attention. */
int qv_attention_precise(float *out, const float *q, const void *k_pages, const void *v_pages,
                         int q_heads, int kv_heads, int head_dim, int tokens, int position,
                         int capacity, float scale, void *workspace, uint64_t workspace_bytes,
                         void *stream);

/* Workspace bytes of qv_attention_fused for this batch/position. */
int qv_attention_fused_workspace(uint64_t *bytes, int batch, int position);
/* Device-side drop-in for the reference's k_attention (src/kernels.cu:575-580)
 * on the paged fp16 cache: RMSNorm + RoPE of q/k, fp16 append of k/v at
 * position..position+batch-1, causal GQA attention (scale 1/16), times
 * sigmoid(gate). Shapes as qv_test_attention, all float32 device buffers;
 * the caches are fp16 pages with 24/4/256 geometry. batch is 1..8 as in the
 * reference, or a prefill chunk of up to 8192 tokens (the reference's server
 * prefills in 8-token steps, qvelox/server.py:177-192): more than 8 tokens
 * run the chunked-prefill kernel with the same fp32-query precision.  Up to
 * 8 tokens prepare q and k inside the attention kernels (one launch on at
 * most 256 keys, else the split kernel and the combine); a prefill chunk
 * runs a prepare launch first. */
int qv_attention_fused(float *out, void *k_pages, void *v_pages,
                       const float *q_gate, const float *key, const float *value,
                       const float *q_norm, const float *k_norm,
                       int batch, int position, int capacity, float epsilon,
                       void *workspace, uint64_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif
