// extern "C" entry points of libredshift_hip (declared in include/runtime.h).
//
// Error convention of the reference (src/runtime.cu:10-18,51-63): every entry
// point runs inside call(), which turns any C++ exception into -1 and a
// thread-local message; qv_error() returns "" after a success.
#include "runtime.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <mutex>
#include <vector>

#include "kernels.hpp"

namespace {

thread_local char last_error[512] = {};

template <class Function>
int call(Function function) noexcept {
    last_error[0] = '\0';
    try {
        function();
        return 0;
    } catch (const std::exception &error) {
        std::snprintf(last_error, sizeof(last_error), "%s", error.what());
    } catch (...) {
        std::snprintf(last_error, sizeof(last_error), "unknown native error");
    }
    return -1;
}

using rs::check;
using rs::require;

// Owns one device allocation; frees it on every exit path.
class DeviceBuffer {
    void *data_ = nullptr;
public:
    explicit DeviceBuffer(size_t size) {
        if (size) check(hipMalloc(&data_, size));
    }
    ~DeviceBuffer() {
        if (data_) (void)hipFree(data_);
    }
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    void *data() const { return data_; }
    float *floats() const { return static_cast<float *>(data_); }
};

void upload(void *device, const void *host, size_t size) {
    if (size) check(hipMemcpy(device, host, size, hipMemcpyHostToDevice));
}
void download(void *host, const void *device, size_t size) {
    if (size) check(hipMemcpy(host, device, size, hipMemcpyDeviceToHost));
}

// Same checks and messages as src/runtime.cu:65-71.
void batch_size(int batch) {
    require(batch >= 1 && batch <= 8, "batch must be between 1 and 8");
}
// The device fused entry also takes prefill chunks of up to kMaxFusedTokens.
constexpr int kMaxFusedTokens = 8192;
void fused_batch_size(int batch) {
    require(batch >= 1 && batch <= kMaxFusedTokens, "batch must be between 1 and 8192");
}
void epsilon_value(float epsilon) {
    require(std::isfinite(epsilon) && epsilon > 0, "epsilon must be finite and positive");
}

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

rs::Dtype dtype_of(int dtype) {
    require(dtype == QV_F16 || dtype == QV_BF16, "dtype must be QV_F16 or QV_BF16");
    return dtype == QV_BF16 ? rs::Dtype::BF16 : rs::Dtype::F16;
}

// True for fp32 output; otherwise the output type must equal the input's.
bool out_f32_of(int dtype, int out_dtype) {
    require(out_dtype == dtype || out_dtype == QV_F32, "out_dtype must be dtype or QV_F32");
    return out_dtype == QV_F32;
}

void geometry(int kv_heads, int head_dim, int capacity) {
    require(kv_heads >= 1 && kv_heads <= 256, "kv_heads must be in 1..256");
    require(head_dim == 128 || head_dim == 256, "head_dim must be 128 or 256");
    require(capacity >= rs::kPageTokens && capacity % rs::kPageTokens == 0,
            "capacity must be a positive multiple of 32 tokens");
}

rs::Shape attention_shape(int q_heads, int kv_heads, int head_dim, int tokens,
                          int position, int capacity) {
    require(kv_heads >= 1 && q_heads >= kv_heads && q_heads % kv_heads == 0,
            "q_heads must be a positive multiple of kv_heads");
    require(q_heads / kv_heads <= rs::kMaxRows, "at most 48 query heads per KV head");
    require(head_dim == 128 || head_dim == 256, "head_dim must be 128 or 256");
    require(tokens >= 1, "tokens must be positive");
    require(position >= 0, "position must be non-negative");
    // Row counts (q_heads * tokens) and the prefill launch's work-items
    // (about 4 per row) stay within 32 bits.
    require((long long)q_heads * tokens <= rs::kMaxQueryRows, "q_heads*tokens exceeds 2^28 query rows");
    return rs::Shape{q_heads, kv_heads, head_dim, tokens, position, capacity};
}

void fits_cache(const rs::Shape &s) {
    geometry(s.kv_heads, s.head_dim, s.capacity);
    require((long long)s.position + s.tokens <= s.capacity, "position+tokens exceeds the cache capacity");
}

// More than kMaxRows query rows per KV head: the prefill kernel.  Otherwise
// split + combine over token chunks of at most kMaxRows query rows per KV
// head; every chunk reuses the workspace in stream order.  q (and q_lo,
// the lo part of a precise query) are 16-bit [tokens][q_heads][D].
void run_attention(const rs::Shape &s, rs::Dtype dtype, bool precise, float scale,
                   const void *q, const void *q_lo, const void *k_pages, const void *v_pages,
                   void *workspace, void *out, bool out_f32, const float *gate,
                   hipStream_t stream) {
    if (s.group() * s.tokens > rs::kMaxRows) {
        // Long token runs (chunked prefill): the prefill kernel, after a V
        // conversion pass for bf16 pages and before a combine when the call
        // splits its keys (the workspace holds the V copy and the partials).
        rs::launch_prefill(s, dtype, precise, scale, q, q_lo, k_pages, v_pages, out, out_f32, gate, workspace,
                           stream);
        return;
    }
    const size_t out_elem = out_f32 ? sizeof(float) : sizeof(uint16_t);
    const int ct = rs::chunk_tokens(s);
    const size_t row = (size_t)s.q_heads * s.head_dim;
    for (int t0 = 0; t0 < s.tokens; t0 += ct) {
        rs::Shape c = s;
        c.position = s.position + t0;
        c.tokens = std::min(ct, s.tokens - t0);
        const rs::SplitPlan plan = rs::plan_split(c, c.tokens, dtype, precise, gate == nullptr);
        const size_t q_offset = t0 * row * sizeof(uint16_t);
        void *out_chunk = static_cast<char *>(out) + t0 * row * out_elem;
        const float *gate_chunk = gate ? gate + (size_t)t0 * 2 * row : nullptr;
        // A short context without a gate: one split per KV head writes the
        // rows itself.
        rs::launch_split(c, plan, dtype, precise, scale, static_cast<const char *>(q) + q_offset,
                         q_lo ? static_cast<const char *>(q_lo) + q_offset : nullptr,
                         k_pages, v_pages, workspace, stream, out_chunk, out_f32);
        if (!plan.direct)
            rs::launch_combine(c, plan, dtype, workspace, out_chunk, out_f32, gate_chunk, stream);
    }
}

// Partials bytes of a fused call: those of the prepared path (attention over
// keys 0 .. position+batch-1) or of the fused split (the cached keys only),
// whichever is larger.  The ring kernel's split count is not monotonic in
// the page count (65 pages take 33 splits of two pages, 64 pages 64 splits
// of one), so neither bounds the other.
size_t fused_partials_bytes(int batch, int position) {
    constexpr int H = rs::kModelQHeads, HKV = rs::kModelKvHeads, D = rs::kModelHeadDim;
    const rs::Shape s{H, HKV, D, batch, position, 0};
    size_t parts = rs::attention_workspace_bytes(s, rs::Dtype::F16, true);
    if (batch <= rs::kMaxFusedSplitTokens && position >= 1)
        parts = std::max(parts, rs::fused_tokens_workspace_bytes(batch, position));
    return std::max(parts, rs::prefill_prep_workspace_bytes(batch, position));
}

// The reference's k_attention on device buffers of the 24/4/256 model.  A
// short context (up to 8 tokens, position + batch <= 256): one launch that
// does everything.  Up to 8 tokens after at least one cached key (decode,
// verification): two launches, the split kernel preparing the query and
// appending the new keys and values, the combine merging (and, for one or
// two tokens, adding the new keys).  A short prefill chunk (more than 8
// tokens whose keys fit four pages from the one holding key `position`):
// the prepared prefill, whose workgroups prepare their query rows, its
// cached runs attend to keys 0 .. position-1 and one split per row
// workgroup prepares, appends and attends to the chunk's keys, then the
// gated combine.  A longer chunk: the prepare kernel appends the new K/V to
// the pages (keys only; q_hilo is not written), then the precise prefill,
// which prepares its query rows from q_gate itself (RMSNorm, RoPE, hi + lo
// parts, the prepare kernel's functions) and applies the sigmoid gate: its
// workgroups read new keys that other workgroups would append, so the append
// stays a launch of its own there.
void fused_attention(float *out, void *k_pages, void *v_pages, const float *q_gate, const float *key,
                     const float *value, const float *q_norm, const float *k_norm, int batch,
                     int position, int capacity, float epsilon, uint16_t *q_hilo, void *partials,
                     size_t partials_bytes, hipStream_t stream) {
    require(partials_bytes >= fused_partials_bytes(batch, position), "workspace too small");
    constexpr int H = rs::kModelQHeads, HKV = rs::kModelKvHeads, D = rs::kModelHeadDim;
    const bool short_context = batch <= rs::kShortMaxTokens && position + batch <= rs::kShortFusedKeys;
    auto fused_token = [&] {
        rs::FusedToken tok = {};
        tok.q_gate = q_gate;
        tok.key = key;
        tok.value = value;
        tok.q_norm = q_norm;
        tok.k_norm = k_norm;
        tok.k_pages = k_pages;
        tok.v_pages = v_pages;
        tok.head_stride = (size_t)capacity * D;
        tok.epsilon = epsilon;
        tok.position = position;
        tok.tokens = batch;
        return tok;
    };
    if (short_context) {
        rs::launch_fused_short(fused_token(), out, stream);
        return;
    }
    if (batch <= rs::kMaxFusedSplitTokens && position >= 1) {
        rs::launch_fused_tokens(fused_token(), capacity, partials, out, stream);
        return;
    }
    if (rs::prefill_prep_fits(batch, position)) {
        rs::launch_prefill_prep(fused_token(), out, partials, stream);
        return;
    }
    // Longer chunks: the keys and values appended first (every workgroup
    // reads keys that others would append), then the prefill, which
    // prepares its query rows from q_gate itself.
    rs::launch_prepare(q_hilo, k_pages, v_pages, q_gate, key, value, q_norm, k_norm, batch, position,
                       capacity, epsilon, stream, true);
    rs::launch_prefill_fused(fused_token(), out, partials, stream);
}

[[noreturn]] void not_in_library(const char *name) {
    char message[200];
    std::snprintf(message, sizeof(message),
                  "%s is not part of libredshift_hip, which implements the attention path only", name);
    throw std::runtime_error(message);
}

}  // namespace

extern "C" const char *qv_error(void) { return last_error; }

extern "C" int qv_test_mm(float *, const void *, const float *, int, int, int, int) {
    return call([] { not_in_library("qv_test_mm"); });
}
extern "C" int qv_test_mm_fast(float *, const void *, const float *, int, int, int, int) {
    return call([] { not_in_library("qv_test_mm_fast"); });
}
extern "C" int qv_test_norm(float *, const float *, const float *, int, int, float) {
    return call([] { not_in_library("qv_test_norm"); });
}
extern "C" int qv_test_delta(float *, float *, float *, const float *, const float *,
                             const float *, const float *, const float *, const float *,
                             const float *, const float *, int, int, int, int, float) {
    return call([] { not_in_library("qv_test_delta"); });
}

extern "C" int qv_test_attention(float *out, void *key_cache, void *value_cache,
                                 const float *q_gate, const float *key, const float *value,
                                 const float *q_norm, const float *k_norm,
                                 int batch, int position, float epsilon) {
    return call([&] {
        // Validation order of src/runtime.cu:172-176; nothing is read before it.
        batch_size(batch);
        epsilon_value(epsilon);
        require(position >= 0 && position <= rs::kModelCapacity - batch,
                "attention context exceeds 139264");
        require(out && key_cache && value_cache && q_gate && key && value && q_norm && k_norm,
                "null attention buffer");
        constexpr int H = rs::kModelQHeads, HKV = rs::kModelKvHeads, D = rs::kModelHeadDim;
        const int n = position + batch;
        const int capacity = (n + rs::kPageTokens - 1) / rs::kPageTokens * rs::kPageTokens;
        const size_t out_bytes = (size_t)batch * H * D * sizeof(float);
        const size_t kv_bytes = (size_t)batch * HKV * D * sizeof(float);
        const size_t row_bytes = (size_t)HKV * D * sizeof(uint16_t);
        const size_t page_bytes = (size_t)HKV * capacity * D * sizeof(uint16_t);
        DeviceBuffer k_pages(page_bytes), v_pages(page_bytes);
        DeviceBuffer k_rows((size_t)n * row_bytes), v_rows((size_t)n * row_bytes);
        DeviceBuffer qg(2 * out_bytes), k(kv_bytes), v(kv_bytes);
        DeviceBuffer qn(D * sizeof(float)), kn(D * sizeof(float));
        DeviceBuffer q(out_bytes), output(out_bytes);   // q: hi and lo fp16 parts
        const size_t partials_bytes = fused_partials_bytes(batch, position);
        DeviceBuffer workspace(partials_bytes);
        hipStream_t stream = nullptr;
        // Host -> device: only the prefix [0, position) of each cache.
        upload(k_rows.data(), key_cache, (size_t)position * row_bytes);
        upload(v_rows.data(), value_cache, (size_t)position * row_bytes);
        upload(qg.data(), q_gate, 2 * out_bytes);
        upload(k.data(), key, kv_bytes);
        upload(v.data(), value, kv_bytes);
        upload(qn.data(), q_norm, D * sizeof(float));
        upload(kn.data(), k_norm, D * sizeof(float));
        rs::launch_pack(k_pages.data(), v_pages.data(), k_rows.data(), v_rows.data(), HKV, D,
                        capacity, 0, position, stream);
        fused_attention(output.floats(), k_pages.data(), v_pages.data(), qg.floats(), k.floats(),
                        v.floats(), qn.floats(), kn.floats(), batch, position, capacity, epsilon,
                        static_cast<uint16_t *>(q.data()), workspace.data(), partials_bytes, stream);
        rs::launch_unpack(k_rows.data(), v_rows.data(), k_pages.data(), v_pages.data(), HKV, D,
                          capacity, 0, n, stream);
        check(hipGetLastError());
        check(hipDeviceSynchronize());
        // Device -> host: out and both whole caches [0, position+batch).
        download(out, output.data(), out_bytes);
        download(key_cache, k_rows.data(), (size_t)n * row_bytes);
        download(value_cache, v_rows.data(), (size_t)n * row_bytes);
    });
}

// ---- model session ABI: not part of this library ---------------------------
extern "C" int qv_create(void **handle, const char *, int, float) {
    return call([&] {
        if (handle) *handle = nullptr;
        not_in_library("qv_create (model session)");
    });
}
extern "C" int qv_upload(void *, int, uint64_t, uint64_t) {
    return call([] { not_in_library("qv_upload (model session)"); });
}
extern "C" int qv_evaluate(void *, const int *, int, float *) {
    return call([] { not_in_library("qv_evaluate (model session)"); });
}
extern "C" int qv_verify(void *, const int *, int, float *) {
    return call([] { not_in_library("qv_verify (model session)"); });
}
extern "C" int qv_commit(void *, int) {
    return call([] { not_in_library("qv_commit (model session)"); });
}
extern "C" int qv_advance(void *, const int *, int, int *) {
    return call([] { not_in_library("qv_advance (model session)"); });
}
extern "C" int qv_reset(void *) { return call([] { not_in_library("qv_reset (model session)"); }); }
extern "C" int qv_checkpoint(void *) {
    return call([] { not_in_library("qv_checkpoint (model session)"); });
}
extern "C" int qv_restore(void *) { return call([] { not_in_library("qv_restore (model session)"); }); }
extern "C" int qv_position(void *, int *) {
    return call([] { not_in_library("qv_position (model session)"); });
}
extern "C" void qv_destroy(void *) {}

// ---- device ABI -----------------------------------------------------------
extern "C" int qv_kv_bytes(uint64_t *bytes, int kv_heads, int head_dim, int capacity) {
    return call([&] {
        require(bytes != nullptr, "null bytes output");
        geometry(kv_heads, head_dim, capacity);
        *bytes = (uint64_t)kv_heads * capacity * head_dim * sizeof(uint16_t);
    });
}

static void kv_convert_args(const void *k_pages, const void *v_pages, const void *k_rows,
                            const void *v_rows, int kv_heads, int head_dim, int capacity,
                            int first, int count) {
    geometry(kv_heads, head_dim, capacity);
    require(first >= 0 && count >= 0 && (long long)first + count <= capacity,
            "token range outside the cache capacity");
    require((k_pages && k_rows) || (v_pages && v_rows), "null KV buffer");
    require(!k_pages == !k_rows && !v_pages == !v_rows, "each side needs both pages and rows");
}

extern "C" int qv_kv_pack(void *k_pages, void *v_pages, const void *k_rows, const void *v_rows,
                          int kv_heads, int head_dim, int capacity, int first, int count,
                          void *stream) {
    return call([&] {
        kv_convert_args(k_pages, v_pages, k_rows, v_rows, kv_heads, head_dim, capacity, first, count);
        rs::launch_pack(k_pages, v_pages, k_rows, v_rows, kv_heads, head_dim, capacity, first,
                        count, static_cast<hipStream_t>(stream));
    });
}

extern "C" int qv_kv_unpack(void *k_rows, void *v_rows, const void *k_pages, const void *v_pages,
                            int kv_heads, int head_dim, int capacity, int first, int count,
                            void *stream) {
    return call([&] {
        kv_convert_args(k_pages, v_pages, k_rows, v_rows, kv_heads, head_dim, capacity, first, count);
        rs::launch_unpack(k_rows, v_rows, k_pages, v_pages, kv_heads, head_dim, capacity, first,
                          count, static_cast<hipStream_t>(stream));
    });
}

extern "C" int qv_kv_copy(void *dst_k, void *dst_v, const void *src_k, const void *src_v,
                          int kv_heads, int head_dim, int dst_capacity, int src_capacity, int tokens,
                          void *stream) {
    return call([&] {
        geometry(kv_heads, head_dim, dst_capacity);
        geometry(kv_heads, head_dim, src_capacity);
        require(tokens >= 0, "tokens must be non-negative");
        const long long pages = ((long long)tokens + rs::kPageTokens - 1) / rs::kPageTokens;
        require(pages * rs::kPageTokens <= std::min(dst_capacity, src_capacity),
                "the pages of tokens exceed a cache capacity");
        require(dst_k && dst_v && src_k && src_v, "null KV cache");
        require(aligned16(dst_k) && aligned16(dst_v) && aligned16(src_k) && aligned16(src_v),
                "KV caches must be 16-byte aligned");
        rs::launch_copy(dst_k, dst_v, src_k, src_v, kv_heads, head_dim, dst_capacity, src_capacity, (int)pages,
                        static_cast<hipStream_t>(stream));
    });
}

extern "C" int qv_attention_workspace(uint64_t *bytes, int q_heads, int kv_heads, int head_dim,
                                      int tokens, int position) {
    return call([&] {
        require(bytes != nullptr, "null bytes output");
        const rs::Shape s = attention_shape(q_heads, kv_heads, head_dim, tokens, position, 0);
        // The bf16 kernels use the same partial layout and the same split count.
        *bytes = std::max(rs::attention_workspace_bytes(s, rs::Dtype::F16, false),
                          rs::attention_workspace_bytes(s, rs::Dtype::BF16, false));
    });
}

static void raw_buffers(const void *out, const void *q, const void *k_pages, const void *v_pages,
                        const void *workspace) {
    require(q && k_pages && v_pages && out, "null attention buffer");
    require(aligned16(q) && aligned16(k_pages) && aligned16(v_pages) && aligned16(workspace) &&
            aligned16(out), "attention buffers must be 16-byte aligned");
}

// The workspace may be NULL only where the shape needs none.
static void workspace_fits(const void *workspace, uint64_t bytes, size_t needed) {
    require(workspace || !needed, "null attention buffer");
    require(bytes >= needed, "workspace too small");
}

extern "C" int qv_attention(void *out, const void *q, const void *k_pages, const void *v_pages,
                            int dtype, int out_dtype, int q_heads, int kv_heads, int head_dim,
                            int tokens, int position, int capacity, float scale,
                            void *workspace, uint64_t workspace_bytes, void *stream) {
    return call([&] {
        const rs::Dtype dt = dtype_of(dtype);
        const bool out_f32 = out_f32_of(dtype, out_dtype);
        const rs::Shape s = attention_shape(q_heads, kv_heads, head_dim, tokens, position, capacity);
        fits_cache(s);
        require(std::isfinite(scale), "scale must be finite");
        raw_buffers(out, q, k_pages, v_pages, workspace);
        workspace_fits(workspace, workspace_bytes, rs::attention_workspace_bytes(s, dt, false));
        run_attention(s, dt, false, scale, q, nullptr, k_pages, v_pages, workspace, out, out_f32,
                      nullptr, static_cast<hipStream_t>(stream));
    });
}

// ---- qv_attention_noalloc: the workspace in a static device array --------
// One array per GPU, loaded with the library's code object and held until the
// process ends.  The largest split-K plan on a 256-CU part is 256 workgroups
// x 48 rows x (256 + 2) floats = 12.1 MiB (split counts are capped by the
// resident workgroups, and a KV head never has fewer than one split); a bf16
// prefill keeps an fp16 copy of its V pages there, kv_heads x keys x
// head_dim x 2 bytes (32 MiB for 4 x 256 at 16,384 keys), and a prefill that
// splits its keys its partial rows (at most about 51 MB at head_dim 256 on
// 256 CUs: one 192-row workgroup per CU).
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
// Device address of `scratch` on the current device.  In host code the
// array's name is only a stand-in for the symbol, so the address is looked
// up once per device (with that device current) and kept.
void *scratch_address() {
    static std::mutex mutex;
    static std::vector<void *> addresses;
    int device = 0;
    check(hipGetDevice(&device));
    std::lock_guard<std::mutex> lock(mutex);
    if ((int)addresses.size() <= device) addresses.resize(device + 1, nullptr);
    if (!addresses[device]) {
        void *ptr = nullptr;
        check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        require(ptr != nullptr, "no device address for the attention scratch array");
        addresses[device] = ptr;
    }
    return addresses[device];
}
}  // namespace

extern "C" int qv_attention_noalloc(void *out, const void *q, const void *k_pages, const void *v_pages,
                                    int dtype, int out_dtype, int q_heads, int kv_heads, int head_dim,
                                    int tokens, int position, int capacity, float scale, void *stream) {
    return call([&] {
        const rs::Dtype dt = dtype_of(dtype);
        const bool out_f32 = out_f32_of(dtype, out_dtype);
        const rs::Shape s = attention_shape(q_heads, kv_heads, head_dim, tokens, position, capacity);
        fits_cache(s);
        require(std::isfinite(scale), "scale must be finite");
        void *workspace = scratch_address();
        raw_buffers(out, q, k_pages, v_pages, workspace);
        require(rs::attention_workspace_bytes(s, dt, false) <= kScratchBytes,
                "the shape needs more than the 64 MiB of workspace of qv_attention_noalloc");
        run_attention(s, dt, false, scale, q, nullptr, k_pages, v_pages, workspace, out, out_f32,
                      nullptr, static_cast<hipStream_t>(stream));
    });
}

extern "C" int qv_attention_split(const void *q, const void *k_pages, const void *v_pages,
                                  int dtype, int q_heads, int kv_heads, int head_dim,
                                  int tokens, int position, int capacity, float scale,
                                  void *workspace, uint64_t workspace_bytes, void *stream) {
    return call([&] {
        const rs::Dtype dt = dtype_of(dtype);
        const rs::Shape s = attention_shape(q_heads, kv_heads, head_dim, tokens, position, capacity);
        fits_cache(s);
        require(tokens <= rs::chunk_tokens(s), "qv_attention_split takes one chunk: group*tokens <= 48");
        require(std::isfinite(scale), "scale must be finite");
        raw_buffers(workspace, q, k_pages, v_pages, workspace);
        const rs::SplitPlan plan = rs::plan_split(s, tokens, dt, false);
        require(workspace_bytes >= rs::plan_bytes(s, plan), "workspace too small");
        rs::launch_split(s, plan, dt, false, scale, q, nullptr, k_pages, v_pages, workspace,
                         static_cast<hipStream_t>(stream));
    });
}

extern "C" int qv_attention_combine(void *out, int dtype, int out_dtype, int q_heads, int kv_heads,
                                    int head_dim, int tokens, int position, const void *workspace,
                                    uint64_t workspace_bytes, void *stream) {
    return call([&] {
        const rs::Dtype dt = dtype_of(dtype);
        const bool out_f32 = out_f32_of(dtype, out_dtype);
        const rs::Shape s = attention_shape(q_heads, kv_heads, head_dim, tokens, position, 0);
        require(tokens <= rs::chunk_tokens(s), "qv_attention_combine takes one chunk: group*tokens <= 48");
        require(out && workspace, "null attention buffer");
        require(aligned16(out) && aligned16(workspace), "attention buffers must be 16-byte aligned");
        const rs::SplitPlan plan = rs::plan_split(s, tokens, dt, false);
        require(workspace_bytes >= rs::plan_bytes(s, plan), "workspace too small");
        rs::launch_combine(s, plan, dt, workspace, out, out_f32, nullptr, static_cast<hipStream_t>(stream));
    });
}

// qv_attention_precise: the query's fp16 hi and lo parts (2 * tokens *
// q_heads * head_dim halves, rounded up to 256 bytes), then the partials of
// the precise kernel instances.
static size_t precise_query_bytes(const rs::Shape &s) {
    return align256((size_t)2 * s.tokens * s.q_heads * s.head_dim * sizeof(uint16_t));
}
static size_t precise_workspace(const rs::Shape &s) {
    return precise_query_bytes(s) + rs::attention_workspace_bytes(s, rs::Dtype::F16, true);
}

extern "C" int qv_attention_precise_workspace(uint64_t *bytes, int q_heads, int kv_heads, int head_dim,
                                              int tokens, int position) {
    return call([&] {
        require(bytes != nullptr, "null bytes output");
        *bytes = precise_workspace(attention_shape(q_heads, kv_heads, head_dim, tokens, position, 0));
    });
}

extern "C" int qv_attention_precise(float *out, const float *q, const void *k_pages, const void *v_pages,
                                    int q_heads, int kv_heads, int head_dim, int tokens, int position,
                                    int capacity, float scale, void *workspace, uint64_t workspace_bytes,
                                    void *stream) {
    return call([&] {
        const rs::Shape s = attention_shape(q_heads, kv_heads, head_dim, tokens, position, capacity);
        fits_cache(s);
        require(std::isfinite(scale), "scale must be finite");
        require(workspace != nullptr, "null attention buffer");
        raw_buffers(out, q, k_pages, v_pages, workspace);
        require(workspace_bytes >= precise_workspace(s), "workspace too small");
        hipStream_t st = static_cast<hipStream_t>(stream);
        void *partials = static_cast<char *>(workspace) + precise_query_bytes(s);
        if (s.group() * s.tokens <= 16) {
            // One query tile: the stream kernel splits the fp32 query into
            // its hi + lo parts itself.
            run_attention(s, rs::Dtype::F16, true, scale, q, nullptr, k_pages, v_pages, partials, out, true, nullptr,
                          st);
            return;
        }
        const size_t n = (size_t)s.tokens * s.q_heads * s.head_dim;
        uint16_t *q_hilo = static_cast<uint16_t *>(workspace);
        rs::launch_split_query(q_hilo, q, n, st);
        run_attention(s, rs::Dtype::F16, true, scale, q_hilo, q_hilo + n, k_pages, v_pages, partials, out, true,
                      nullptr, st);
    });
}

// The query's hi + lo parts, then the partials.
static size_t fused_query_bytes(int batch) {
    return align256((size_t)batch * rs::kModelQHeads * rs::kModelHeadDim * sizeof(float));
}
static size_t fused_workspace(int batch, int position) {
    return fused_query_bytes(batch) + fused_partials_bytes(batch, position);
}

extern "C" int qv_attention_fused_workspace(uint64_t *bytes, int batch, int position) {
    return call([&] {
        require(bytes != nullptr, "null bytes output");
        fused_batch_size(batch);
        require(position >= 0 && position <= rs::kModelCapacity - batch,
                "attention context exceeds 139264");
        *bytes = fused_workspace(batch, position);
    });
}

extern "C" int qv_attention_fused(float *out, void *k_pages, void *v_pages,
                                  const float *q_gate, const float *key, const float *value,
                                  const float *q_norm, const float *k_norm,
                                  int batch, int position, int capacity, float epsilon,
                                  void *workspace, uint64_t workspace_bytes, void *stream) {
    return call([&] {
        fused_batch_size(batch);
        epsilon_value(epsilon);
        require(position >= 0 && position <= rs::kModelCapacity - batch,
                "attention context exceeds 139264");
        require(out && k_pages && v_pages && q_gate && key && value && q_norm && k_norm && workspace,
                "null attention buffer");
        constexpr int H = rs::kModelQHeads, HKV = rs::kModelKvHeads, D = rs::kModelHeadDim;
        const rs::Shape s{H, HKV, D, batch, position, capacity};
        fits_cache(s);
        require(aligned16(out) && aligned16(q_gate) && aligned16(key) && aligned16(value) && aligned16(q_norm) &&
                aligned16(k_norm) && aligned16(workspace) && aligned16(k_pages) && aligned16(v_pages),
                "attention buffers must be 16-byte aligned");
        require(workspace_bytes >= fused_workspace(batch, position), "workspace too small");
        hipStream_t st = static_cast<hipStream_t>(stream);
        uint16_t *q = static_cast<uint16_t *>(workspace);   // hi then lo fp16 parts
        void *partials = static_cast<char *>(workspace) + fused_query_bytes(batch);
        fused_attention(out, k_pages, v_pages, q_gate, key, value, q_norm, k_norm, batch, position,
                        capacity, epsilon, q, partials, workspace_bytes - fused_query_bytes(batch), st);
    });
}
