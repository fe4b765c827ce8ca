// Host-side AddressSanitizer + UndefinedBehaviorSanitizer gate for
// libredshift_hip's C ABI.
//
// The reference runs its kernel tests under compute-sanitizer memcheck and
// racecheck (Makefile:23-26).  Device code has no sanitizer on this platform,
// so this program covers the host half of the library: it is linked from the
// library's sources compiled with -fsanitize=address,undefined on the host
// side only (the device code is the ordinary gfx950 build), and it drives
// every entry point of include/runtime.h:
//   * host mode (always): the stubs, the validation of every entry point
//     with its messages (invalid inputs only, each rejected before any device
//     work, with heap buffers of one element where a buffer is passed, so a
//     read before validation is an ASan report), qv_kv_bytes over a sweep
//     including int32 extremes, and the split-K and prefill planners
//     (plan_split_for, plan_prefill_for; no device query) over sweeps of
//     shapes with their invariants;
//   * device mode (a GPU is present): the same plus small real calls of
//     every entry point on device buffers, the workspace queries against the
//     planner, the error paths that need a device, and qv_test_attention on
//     host buffers of exactly the documented sizes, so that any host access
//     outside them is an ASan report.
// Exit status 0 when every check passed; a sanitizer report aborts with a
// non-zero status.  Usage: abi_sanitize [--host-only]
#include "runtime.h"
#include "kernels.hpp"

#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <random>
#include <vector>

// Leak checking would report the HIP runtime's own process-lifetime objects.
extern "C" const char *__asan_default_options() { return "detect_leaks=0"; }

namespace {

int checks = 0, failures = 0;

void expect(bool ok, const char *what, int line) {
    ++checks;
    if (!ok) {
        ++failures;
        std::fprintf(stderr, "FAIL line %d: %s (qv_error: \"%s\")\n", line, what, qv_error());
    }
}
#define EXPECT(cond) expect((cond), #cond, __LINE__)

bool failed_with(int rc, const char *needle) { return rc == -1 && std::strstr(qv_error(), needle) != nullptr; }

constexpr int H = 24, HKV = 4, D = 256;

// ---- host mode ---------------------------------------------------------------

void stubs() {
    float f = 0.f;
    const char *msg = "not part of libredshift_hip";
    EXPECT(failed_with(qv_test_mm(&f, nullptr, nullptr, 0, 1, 1, 1), msg));
    EXPECT(failed_with(qv_test_mm_fast(&f, nullptr, nullptr, 0, 1, 1, 1), msg));
    EXPECT(failed_with(qv_test_norm(&f, nullptr, nullptr, 1, 1, 1e-6f), msg));
    EXPECT(failed_with(qv_test_delta(&f, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                     nullptr, nullptr, 1, 1, 1, 1, 1e-6f), msg));
    void *handle = &f;
    EXPECT(failed_with(qv_create(&handle, "model", 1, 1e-6f), msg) && handle == nullptr);
    EXPECT(failed_with(qv_create(nullptr, nullptr, 1, 1e-6f), msg));
    int tokens[8] = {}, next = 0, position = 0;
    EXPECT(failed_with(qv_upload(nullptr, 0, 0, 0), msg));
    EXPECT(failed_with(qv_evaluate(nullptr, tokens, 1, &f), msg));
    EXPECT(failed_with(qv_verify(nullptr, tokens, 1, &f), msg));
    EXPECT(failed_with(qv_commit(nullptr, 0), msg));
    EXPECT(failed_with(qv_advance(nullptr, tokens, 1, &next), msg));
    EXPECT(failed_with(qv_reset(nullptr), msg));
    EXPECT(failed_with(qv_checkpoint(nullptr), msg));
    EXPECT(failed_with(qv_restore(nullptr), msg));
    EXPECT(failed_with(qv_position(nullptr, &position), msg));
    qv_destroy(nullptr);
}

// qv_test_attention's validation order (batch, epsilon, position, null
// buffers); every buffer is a one-element heap array, so a read before the
// validation is an ASan report.
void test_attention_validation() {
    std::vector<float> one(1);
    std::vector<uint16_t> half(1);
    float *o = one.data();
    void *kc = half.data(), *vc = half.data();
    const float *x = one.data();
    const char *batch = "batch must be between 1 and 8", *eps = "epsilon must be finite and positive";
    const char *ctx = "attention context exceeds 139264", *null = "null attention buffer";
    for (int b : {INT_MIN, -1, 0, 9, 100, INT_MAX})
        EXPECT(failed_with(qv_test_attention(o, kc, vc, x, x, x, x, x, b, 0, 1e-6f), batch));
    EXPECT(failed_with(qv_test_attention(o, kc, vc, x, x, x, x, x, 0, -5, NAN), batch));   // batch first
    for (float e : {0.f, -1e-6f, NAN, INFINITY, -INFINITY})
        EXPECT(failed_with(qv_test_attention(o, kc, vc, x, x, x, x, x, 1, 0, e), eps));
    EXPECT(failed_with(qv_test_attention(o, kc, vc, x, x, x, x, x, 1, -1, NAN), eps));     // epsilon second
    for (int b = 1; b <= 8; ++b) {
        for (int p : {INT_MIN, -1, 139264 - b + 1, 139264, INT_MAX - 8, INT_MAX})
            EXPECT(failed_with(qv_test_attention(o, kc, vc, x, x, x, x, x, b, p, 1e-6f), ctx));
    }
    EXPECT(failed_with(qv_test_attention(nullptr, kc, vc, x, x, x, x, x, 1, -1, 1e-6f), ctx));   // position third
    for (int which = 0; which < 8; ++which) {
        void *p[8] = {o, kc, vc, one.data(), one.data(), one.data(), one.data(), one.data()};
        p[which] = nullptr;
        EXPECT(failed_with(qv_test_attention(static_cast<float *>(p[0]), p[1], p[2], static_cast<float *>(p[3]),
                                             static_cast<float *>(p[4]), static_cast<float *>(p[5]),
                                             static_cast<float *>(p[6]), static_cast<float *>(p[7]), 2, 10, 1e-6f),
                           null));
    }
}

// qv_kv_bytes against the product computed in 128 bits.
void kv_bytes_sweep() {
    for (int kv : {INT_MIN, -1, 0, 1, 2, 4, 64, 256, 257, INT_MAX})
        for (int d : {-256, 0, 64, 128, 255, 256, 512})
            for (int cap : {INT_MIN, -32, 0, 1, 31, 32, 33, 4096, 139264, INT_MAX - INT_MAX % 32, INT_MAX}) {
                uint64_t bytes = 12345;
                const int rc = qv_kv_bytes(&bytes, kv, d, cap);
                const bool valid = kv >= 1 && kv <= 256 && (d == 128 || d == 256) && cap >= 32 && cap % 32 == 0;
                if (valid) {
                    const unsigned __int128 want = (unsigned __int128)kv * (unsigned)cap * (unsigned)d * 2;
                    EXPECT(rc == 0 && bytes == (uint64_t)want && qv_error()[0] == '\0');
                } else {
                    EXPECT(rc == -1 && bytes == 12345 && qv_error()[0] != '\0');
                }
            }
    EXPECT(failed_with(qv_kv_bytes(nullptr, 4, 256, 32), "null bytes output"));
}

// Validation of the device entry points on inputs that each break one rule
// checked before any device work.  The pointers point at a small host array:
// nothing may dereference them.
alignas(16) uint16_t cell[8];

void device_entry_validation() {
    void *p = cell;
    void *odd = reinterpret_cast<char *>(cell) + 2;
    float *f = reinterpret_cast<float *>(cell);
    // qv_kv_pack / qv_kv_unpack / qv_kv_copy
    const char *range = "token range outside the cache capacity";
    EXPECT(failed_with(qv_kv_pack(p, p, p, p, 4, 256, 64, -1, 1, nullptr), range));
    EXPECT(failed_with(qv_kv_pack(p, p, p, p, 4, 256, 64, 0, -1, nullptr), range));
    EXPECT(failed_with(qv_kv_pack(p, p, p, p, 4, 256, 64, 60, 5, nullptr), range));
    EXPECT(failed_with(qv_kv_pack(p, p, p, p, 4, 256, 64, INT_MAX, INT_MAX, nullptr), range));
    EXPECT(failed_with(qv_kv_unpack(p, p, p, p, 4, 256, INT_MAX - INT_MAX % 32, INT_MAX - 40, 100, nullptr), range));
    EXPECT(failed_with(qv_kv_pack(nullptr, nullptr, p, p, 4, 256, 64, 0, 1, nullptr), "null KV buffer"));
    EXPECT(failed_with(qv_kv_pack(p, p, p, nullptr, 4, 256, 64, 0, 1, nullptr), "each side needs both"));
    EXPECT(failed_with(qv_kv_pack(p, p, p, p, 0, 256, 64, 0, 1, nullptr), "kv_heads must be in 1..256"));
    EXPECT(failed_with(qv_kv_pack(p, p, p, p, 4, 96, 64, 0, 1, nullptr), "head_dim must be 128 or 256"));
    EXPECT(failed_with(qv_kv_unpack(p, p, p, p, 4, 256, 48, 0, 1, nullptr), "capacity must be a positive multiple"));
    const char *pages = "the pages of tokens exceed a cache capacity";
    EXPECT(failed_with(qv_kv_copy(p, p, p, p, 4, 256, 64, 64, -1, nullptr), "tokens must be non-negative"));
    EXPECT(failed_with(qv_kv_copy(p, p, p, p, 4, 256, 64, 128, 65, nullptr), pages));
    EXPECT(failed_with(qv_kv_copy(p, p, p, p, 4, 256, 64, 64, INT_MAX, nullptr), pages));
    EXPECT(failed_with(qv_kv_copy(p, p, p, p, 4, 256, INT_MAX - INT_MAX % 32, 64, INT_MAX - 3, nullptr), pages));
    EXPECT(failed_with(qv_kv_copy(p, nullptr, p, p, 4, 256, 64, 64, 1, nullptr), "null KV cache"));
    EXPECT(failed_with(qv_kv_copy(odd, p, p, p, 4, 256, 64, 64, 1, nullptr), "16-byte aligned"));

    // qv_attention (and the variants sharing its shape rules)
    auto raw = [&](int dtype, int out_dtype, int qh, int kvh, int d, int t, int pos, int cap, float scale,
                   void *out = cell, const void *q = cell, const void *kp = cell, const void *vp = cell) {
        return qv_attention(out, q, kp, vp, dtype, out_dtype, qh, kvh, d, t, pos, cap, scale, cell, 1 << 30,
                            nullptr);
    };
    EXPECT(failed_with(raw(0, 0, 24, 4, 256, 1, 0, 64, 1.f), "dtype must be QV_F16 or QV_BF16"));
    EXPECT(failed_with(raw(QV_F32, QV_F32, 24, 4, 256, 1, 0, 64, 1.f), "dtype must be QV_F16 or QV_BF16"));
    EXPECT(failed_with(raw(QV_F16, QV_BF16, 24, 4, 256, 1, 0, 64, 1.f), "out_dtype must be dtype or QV_F32"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 24, 5, 256, 1, 0, 64, 1.f), "q_heads must be a positive multiple"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 0, 0, 256, 1, 0, 64, 1.f), "q_heads must be a positive multiple"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, INT_MIN, 1, 256, 1, 0, 64, 1.f), "q_heads must be a positive multiple"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 49, 1, 256, 1, 0, 64, 1.f), "at most 48 query heads per KV head"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 24, 4, 64, 1, 0, 64, 1.f), "head_dim must be 128 or 256"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 24, 4, 256, 0, 0, 64, 1.f), "tokens must be positive"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 24, 4, 256, 1, -1, 64, 1.f), "position must be non-negative"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 48, 1, 256, INT_MAX, 0, 64, 1.f), "exceeds 2^28 query rows"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 48, 48, 256, (1 << 28) / 48 + 1, 0, 64, 1.f), "exceeds 2^28 query rows"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 24, 4, 256, 1, 0, 100, 1.f), "capacity must be a positive multiple"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 24, 4, 256, 1, 64, 64, 1.f), "position+tokens exceeds the cache capacity"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 24, 4, 256, 100, INT_MAX - 50, INT_MAX - INT_MAX % 32, 1.f),
                       "position+tokens exceeds the cache capacity"));
    for (float s : {NAN, INFINITY, -INFINITY})
        EXPECT(failed_with(raw(QV_F16, QV_F16, 24, 4, 256, 1, 0, 64, s), "scale must be finite"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 24, 4, 256, 1, 0, 64, 1.f, nullptr), "null attention buffer"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 24, 4, 256, 1, 0, 64, 1.f, cell, nullptr), "null attention buffer"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 24, 4, 256, 1, 0, 64, 1.f, odd), "16-byte aligned"));
    EXPECT(failed_with(raw(QV_F16, QV_F16, 24, 4, 256, 1, 0, 64, 1.f, cell, cell, odd), "16-byte aligned"));
    EXPECT(failed_with(qv_attention_noalloc(p, p, p, p, QV_F16, QV_F16, 24, 4, 256, 1, 70, 64, 1.f, nullptr),
                       "position+tokens exceeds the cache capacity"));
    EXPECT(failed_with(qv_attention_split(p, p, p, QV_F16, 24, 4, 256, 9, 0, 64, 1.f, p, 1 << 30, nullptr),
                       "qv_attention_split takes one chunk"));
    EXPECT(failed_with(qv_attention_combine(p, QV_F16, QV_F16, 24, 4, 256, 9, 0, p, 1 << 30, nullptr),
                       "qv_attention_combine takes one chunk"));
    EXPECT(failed_with(qv_attention_combine(nullptr, QV_F16, QV_F16, 24, 4, 256, 1, 0, p, 1 << 30, nullptr),
                       "null attention buffer"));
    EXPECT(failed_with(qv_attention_precise(f, f, p, p, 24, 4, 256, 1, 0, 64, 1.f, nullptr, 1 << 30, nullptr),
                       "null attention buffer"));
    EXPECT(failed_with(qv_attention_precise(f, f, p, p, 24, 4, 256, 1, 0, 64, NAN, p, 1 << 30, nullptr),
                       "scale must be finite"));
    uint64_t bytes = 0;
    EXPECT(failed_with(qv_attention_workspace(nullptr, 24, 4, 256, 1, 0), "null bytes output"));
    EXPECT(failed_with(qv_attention_workspace(&bytes, 24, 4, 256, 0, 0), "tokens must be positive"));
    EXPECT(failed_with(qv_attention_precise_workspace(&bytes, 24, 7, 256, 1, 0), "q_heads must be a positive multiple"));

    // qv_attention_fused: batch, epsilon, position, buffers, capacity, alignment
    auto fused = [&](int batch, int pos, int cap, float eps, void *out = cell, void *ws = cell) {
        return qv_attention_fused(static_cast<float *>(out), p, p, f, f, f, f, f, batch, pos, cap, eps, ws, 1 << 30,
                                  nullptr);
    };
    for (int b : {INT_MIN, 0, 8193, INT_MAX})
        EXPECT(failed_with(fused(b, 0, 64, 1e-6f), "batch must be between 1 and 8192"));
    EXPECT(failed_with(fused(1, 0, 64, NAN), "epsilon must be finite and positive"));
    for (int pos : {INT_MIN, -1, 139264, INT_MAX})
        EXPECT(failed_with(fused(1, pos, 64, 1e-6f), "attention context exceeds 139264"));
    EXPECT(failed_with(fused(1, 0, 64, 1e-6f, nullptr), "null attention buffer"));
    EXPECT(failed_with(fused(1, 0, 64, 1e-6f, cell, nullptr), "null attention buffer"));
    EXPECT(failed_with(fused(8, 60, 64, 1e-6f), "position+tokens exceeds the cache capacity"));
    EXPECT(failed_with(fused(1, 0, 40, 1e-6f), "capacity must be a positive multiple"));
    EXPECT(failed_with(fused(1, 0, 64, 1e-6f, odd), "16-byte aligned"));
    EXPECT(failed_with(qv_attention_fused_workspace(nullptr, 1, 0), "null bytes output"));
    EXPECT(failed_with(qv_attention_fused_workspace(&bytes, 0, 0), "batch must be between 1 and 8192"));
    EXPECT(failed_with(qv_attention_fused_workspace(&bytes, 8, 139257), "attention context exceeds 139264"));
}

// The split planner on a sweep of shapes and devices (no device query):
// every plan fits the shape, every split holds pages, and the partial bytes
// are the documented product without overflow.
int resident_one(const rs::SplitPlan &, int, rs::Dtype, bool) { return 1; }
int resident_two(const rs::SplitPlan &p, int, rs::Dtype, bool) { return p.kind == rs::SplitKind::Stream ? 2 : 1; }

void planner_sweep() {
    const int heads[][2] = {{24, 4}, {8, 2}, {16, 2}, {24, 1}, {48, 1}, {64, 8}, {1, 1}, {256, 256}};
    const int positions[] = {0, 1, 31, 32, 33, 255, 1000, 4095, 16384, 139263, 1 << 20, (1 << 30) - 1,
                             INT_MAX - 64};
    int plans = 0;
    for (const auto &hk : heads)
        for (int d : {128, 256})
            for (int cus : {1, 8, 80, 256, 304})
                for (auto resident : {resident_one, resident_two})
                    for (int pos : positions)
                        for (int dt = 0; dt < 2; ++dt)
                            for (int precise = 0; precise < 2; ++precise)
                                for (int direct = 0; direct < 2; ++direct) {
                                    const rs::Shape s0{hk[0], hk[1], d, 1, pos, 0};
                                    const int ct = rs::chunk_tokens(s0);
                                    for (int t : {1, 2, ct}) {
                                        if (t > ct || (long long)pos + t > INT_MAX) continue;
                                        const rs::Shape s{hk[0], hk[1], d, t, pos, 0};
                                        const rs::Dtype dtype = dt ? rs::Dtype::BF16 : rs::Dtype::F16;
                                        const rs::SplitPlan p =
                                            rs::plan_split_for(s, t, dtype, precise, direct, cus, resident);
                                        ++plans;
                                        const long long n_keys = (long long)pos + t;
                                        EXPECT(p.rows == s.group() * t && p.rows <= rs::kMaxRows);
                                        EXPECT(p.nqt == (p.rows + 15) / 16 && p.nqt >= 1 && p.nqt <= 3);
                                        EXPECT((long long)p.n_pages == (n_keys + 31) / 32);
                                        EXPECT(p.splits >= 1 && p.splits <= p.n_pages);
                                        EXPECT(!p.direct || (direct && p.splits == 1 && p.n_pages <= 8));
                                        EXPECT(!p.half_parts || (p.kind == rs::SplitKind::Ring && !dt && !precise));
                                        if (p.kind == rs::SplitKind::Ring) {
                                            // Contiguous runs, none empty: p0(split) strictly increases.
                                            const long long longest = (p.n_pages + p.splits - 1) / p.splits;
                                            EXPECT((p.splits - 1) * longest < p.n_pages);
                                        }
                                        const size_t bytes = rs::plan_bytes(s, p);
                                        const unsigned __int128 want =
                                            p.direct ? 0
                                                     : (unsigned __int128)s.kv_heads * p.splits * p.rows *
                                                           ((unsigned)d + 2) * 4;
                                        EXPECT(bytes == (size_t)want);
                                    }
                                }
    std::printf("abi_sanitize: %d split plans checked\n", plans);
}

// The prefill planner on a sweep of shapes and devices (no device query):
// rows per workgroup, key splits only for calls of at least
// kPrefillMinSplitKeyPages pages whose row workgroups leave CUs idle, then at
// most one workgroup per CU in runs of at least kPrefillMinSplitPages pages,
// as many as those bounds allow; the workspace is the documented sum without
// overflow, and the launch stays within 2^32 work-items.
void prefill_planner_sweep() {
    const int heads[][2] = {{24, 4}, {8, 2}, {16, 2}, {24, 1}, {48, 1}, {64, 8}, {256, 256}};
    const int positions[] = {0, 31, 32, 1000, 6144, 16384, 139263, 1 << 20, (1 << 30) - 1};
    int plans = 0;
    for (const auto &hk : heads)
        for (int d : {128, 256})
            for (int cus : {1, 8, 80, 256, 304})
                for (int pos : positions)
                    for (long long t : {0LL, 64LL, 300LL, 2048LL, 8192LL, 1LL << 28})
                        for (int dt = 0; dt < 2; ++dt)
                            for (int precise = 0; precise < 2; ++precise) {
                                const int group = hk[0] / hk[1];
                                long long tokens = t ? t : 48 / group + 1;   // 0: the fewest prefill tokens
                                tokens = std::min(tokens, (1LL << 28) / hk[0]);
                                if (tokens < 1 || (long long)group * tokens <= rs::kMaxRows ||
                                    (long long)pos + tokens > 2147483616LL)
                                    continue;
                                const rs::Shape s{hk[0], hk[1], d, (int)tokens, pos, 0};
                                const rs::Dtype dtype = dt ? rs::Dtype::BF16 : rs::Dtype::F16;
                                const rs::PrefillPlan p = rs::plan_prefill_for(s, dtype, precise, cus);
                                ++plans;
                                const long long R = (long long)group * tokens;
                                const long long pages = ((long long)pos + tokens + 31) / 32;
                                // A precise call without key splits takes two passes over 192-row
                                // workgroups when 128-row ones need more than 1.5 times their rounds.
                                const long long one = (R + rs::kPreciseRows - 1) / rs::kPreciseRows * hk[1];
                                const long long two = (R + rs::kPreciseTwoPassRows - 1) / rs::kPreciseTwoPassRows * hk[1];
                                const bool two_pass = precise && p.splits == 1 &&
                                                      3 * ((two + cus - 1) / cus) < 2 * ((one + cus - 1) / cus);
                                EXPECT(p.passes == (two_pass ? 2 : 1));
                                EXPECT(p.rows == (!precise ? rs::kPrefillRows
                                                  : p.passes == 2 ? rs::kPreciseTwoPassRows : rs::kPreciseRows));
                                EXPECT(p.row_wgs == (R + p.rows - 1) / p.rows);
                                const long long base = (long long)(p.passes == 2 ? one / hk[1] : p.row_wgs) * hk[1];
                                EXPECT(p.splits >= 1 && p.splits <= rs::kPrefillMaxSplits);
                                if (pages < rs::kPrefillMinSplitKeyPages || base >= cus) {
                                    EXPECT(p.splits == 1);
                                } else {
                                    // Within every bound, and one more split would break one.
                                    EXPECT(base * p.splits <= cus && p.splits * rs::kPrefillMinSplitPages <= pages);
                                    EXPECT(p.splits == rs::kPrefillMaxSplits || base * (p.splits + 1) > cus ||
                                           (p.splits + 1) * rs::kPrefillMinSplitPages > pages);
                                }
                                const auto r256 = [](unsigned __int128 x) { return (x + 255) / 256 * 256; };
                                const unsigned __int128 conv =
                                    dt && !precise ? r256((unsigned __int128)hk[1] * pages * 32 * d * 2) +
                                                         r256((unsigned __int128)hk[1] * pages * 4)
                                                   : 0;
                                const unsigned __int128 parts =
                                    p.splits > 1 ? r256((unsigned __int128)hk[1] * p.splits * R * (d + 2) * 4) : 0;
                                EXPECT((unsigned __int128)p.part_offset == conv);
                                EXPECT((unsigned __int128)p.bytes == conv + parts);
                                EXPECT((unsigned __int128)p.row_wgs * hk[1] * p.splits *
                                           (p.passes == 2 ? 8 : p.rows / 16) * 64 < ((unsigned __int128)1 << 32));
                            }
    std::printf("abi_sanitize: %d prefill plans checked\n", plans);
}

// The prepared prefill of a fused chunk (plan_prefill_prep_for): chunks of
// 9 .. 128 - position % 32 tokens fit; 128-row workgroups; runs over the
// cached pages as plan_prefill_for splits a call's pages (one below
// kPrefillMinSplitKeyPages cached pages or with no idle CU, else as many as
// the CUs, kPrefillMinSplitPages pages per run and kPrefillMaxSplits
// allow); the chunk's keys span at most four pages; the workspace is the
// documented partials.
void prefill_prep_planner_sweep() {
    int plans = 0;
    for (int cus : {1, 8, 80, 256, 304})
        for (int pos : {0, 1, 8, 31, 32, 33, 255, 1000, 6000, 16000, 16384, 139135})
            for (int tokens = 1; tokens <= 200; ++tokens) {
                const bool fits = rs::prefill_prep_fits(tokens, pos);
                EXPECT(fits == (tokens > rs::kMaxFusedSplitTokens && tokens + pos % 32 <= 128));
                if (!fits) continue;
                const rs::PrefillPlan p = rs::plan_prefill_prep_for(tokens, pos, cus);
                ++plans;
                const long long R = 6LL * tokens, cached = (pos + 31LL) / 32;
                const long long base = (R + 127) / 128 * 4;
                EXPECT(p.rows == rs::kPreciseRows && p.passes == 1 && p.row_wgs == (R + 127) / 128);
                EXPECT(p.splits >= 1 && p.splits <= rs::kPrefillMaxSplits);
                if (cached < rs::kPrefillMinSplitKeyPages || base >= cus) {
                    EXPECT(p.splits == 1);
                } else {
                    EXPECT(base * p.splits <= cus && p.splits * rs::kPrefillMinSplitPages <= cached);
                    EXPECT(p.splits == rs::kPrefillMaxSplits || base * (p.splits + 1) > cus ||
                           (p.splits + 1) * rs::kPrefillMinSplitPages > cached);
                }
                // The chunk's pages: from the one holding key pos to the last key's.
                EXPECT((pos + tokens - 1) / 32 - pos / 32 + 1 <= rs::kPrepNewKeyPages);
                const unsigned long long parts =
                    p.splits > 1 ? (4ULL * p.splits * R * (256 + 2) * 4 + 255) / 256 * 256 : 0;
                EXPECT(p.bytes == parts && p.part_offset == 0);
            }
    std::printf("abi_sanitize: %d prepared prefill plans checked\n", plans);
}

// ---- device mode -------------------------------------------------------------

#define HIP_OK(call) EXPECT((call) == hipSuccess)

template <class T>
struct Dev {
    T *p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) { HIP_OK(hipMalloc(&p, count * sizeof(T) + 256)); }
    ~Dev() { (void)hipFree(p); }
    Dev(const Dev &) = delete;
    Dev &operator=(const Dev &) = delete;
};

bool all_finite(const std::vector<float> &v) {
    for (float x : v)
        if (!std::isfinite(x)) return false;
    return true;
}

uint16_t half_bits(float x) {
    const _Float16 h = (_Float16)x;
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

// count values of a device buffer of type QV_F16, QV_BF16 or QV_F32, as floats.
std::vector<float> fetch(const void *dev, size_t count, int dtype) {
    std::vector<float> f(count);
    if (dtype == QV_F32) {
        EXPECT(hipMemcpy(f.data(), dev, count * 4, hipMemcpyDeviceToHost) == hipSuccess);
        return f;
    }
    std::vector<uint16_t> h(count);
    EXPECT(hipMemcpy(h.data(), dev, count * 2, hipMemcpyDeviceToHost) == hipSuccess);
    for (size_t i = 0; i < count; ++i) {
        if (dtype == QV_BF16) {
            const uint32_t bits = (uint32_t)h[i] << 16;
            std::memcpy(&f[i], &bits, 4);
        } else {
            _Float16 x;
            std::memcpy(&x, &h[i], 2);
            f[i] = (float)x;
        }
    }
    return f;
}

void device_calls(hipStream_t stream) {
    std::mt19937 rng(7);
    std::normal_distribution<float> normal(0.f, 1.f);
    const int cap = 2048;
    uint64_t kv_bytes = 0;
    EXPECT(qv_kv_bytes(&kv_bytes, HKV, D, cap) == 0);
    Dev<uint16_t> kp(kv_bytes / 2), vp(kv_bytes / 2), kp2(kv_bytes / 2), vp2(kv_bytes / 2);
    // Token-major fp16 rows of the whole capacity, packed into pages.
    {
        std::vector<uint16_t> rows((size_t)cap * HKV * D);
        for (auto &r : rows) r = half_bits(0.5f * normal(rng));
        Dev<uint16_t> krows(rows.size()), vrows(rows.size());
        HIP_OK(hipMemcpy(krows.p, rows.data(), rows.size() * 2, hipMemcpyHostToDevice));
        for (auto &r : rows) r = half_bits(normal(rng));
        HIP_OK(hipMemcpy(vrows.p, rows.data(), rows.size() * 2, hipMemcpyHostToDevice));
        EXPECT(qv_kv_pack(kp.p, vp.p, krows.p, vrows.p, HKV, D, cap, 0, cap, stream) == 0);
        Dev<uint16_t> back(rows.size());
        EXPECT(qv_kv_unpack(back.p, nullptr, kp.p, nullptr, HKV, D, cap, 100, 200, stream) == 0);
        EXPECT(qv_kv_copy(kp2.p, vp2.p, kp.p, vp.p, HKV, D, cap, cap, 1500, stream) == 0);
        HIP_OK(hipStreamSynchronize(stream));
    }
    // Raw attention on every kernel family: decode, short direct, verify,
    // prefill; fp16 and bf16 pages (the same bits read as bf16 are finite
    // too); 16-bit and fp32 outputs.
    struct Case { int tokens, position, dtype, out_dtype; };
    const Case cases[] = {{1, 1000, QV_F16, QV_F16}, {1, 40, QV_F16, QV_F32}, {8, 1000, QV_F16, QV_F16},
                          {8, 50, QV_F16, QV_F32},   {3, 700, QV_BF16, QV_BF16}, {100, 500, QV_F16, QV_F32},
                          {64, 1900, QV_BF16, QV_F32}};
    for (const Case &c : cases) {
        const size_t n = (size_t)c.tokens * H * D;
        std::vector<uint16_t> q(n);
        for (auto &x : q) x = half_bits(normal(rng));
        Dev<uint16_t> dq(n);
        Dev<float> dout(n);
        HIP_OK(hipMemcpy(dq.p, q.data(), n * 2, hipMemcpyHostToDevice));
        uint64_t ws_bytes = 0;
        EXPECT(qv_attention_workspace(&ws_bytes, H, HKV, D, c.tokens, c.position) == 0);
        Dev<char> ws(ws_bytes + 16);
        EXPECT(qv_attention(dout.p, dq.p, kp.p, vp.p, c.dtype, c.out_dtype, H, HKV, D, c.tokens, c.position, cap,
                            1.f / 16, ws.p, ws_bytes, stream) == 0);
        HIP_OK(hipStreamSynchronize(stream));
        EXPECT(all_finite(fetch(dout.p, n, c.out_dtype)));
        // qv_attention_workspace covers both page types; an fp16 prefill
        // (more than 48 rows per KV head) needs less of it (no V copy).
        const bool f16_prefill = c.dtype == QV_F16 && c.tokens * (H / HKV) > 48;
        if (ws_bytes > 0 && !f16_prefill) {
            EXPECT(failed_with(qv_attention(dout.p, dq.p, kp.p, vp.p, c.dtype, c.out_dtype, H, HKV, D, c.tokens,
                                            c.position, cap, 1.f / 16, ws.p, ws_bytes - 1, stream),
                               "workspace too small"));
        }
        if (c.tokens <= 2 && c.dtype == QV_F16) {
            // The two phases, and the entry without a workspace.
            EXPECT(qv_attention_split(dq.p, kp.p, vp.p, c.dtype, H, HKV, D, c.tokens, c.position, cap, 1.f / 16,
                                      ws.p, ws_bytes, stream) == 0);
            EXPECT(qv_attention_combine(dout.p, c.dtype, QV_F32, H, HKV, D, c.tokens, c.position, ws.p, ws_bytes,
                                        stream) == 0);
            EXPECT(qv_attention_noalloc(dout.p, dq.p, kp.p, vp.p, c.dtype, QV_F32, H, HKV, D, c.tokens, c.position,
                                        cap, 1.f / 16, stream) == 0);
            HIP_OK(hipStreamSynchronize(stream));
            EXPECT(all_finite(fetch(dout.p, n, QV_F32)));
        }
        // The precise entry on the same shape (fp32 query).
        if (c.dtype == QV_F16) {
            std::vector<float> q32(n);
            for (auto &x : q32) x = normal(rng);
            Dev<float> dq32(n);
            HIP_OK(hipMemcpy(dq32.p, q32.data(), n * 4, hipMemcpyHostToDevice));
            uint64_t pb = 0;
            EXPECT(qv_attention_precise_workspace(&pb, H, HKV, D, c.tokens, c.position) == 0);
            Dev<char> pws(pb + 16);
            EXPECT(qv_attention_precise(dout.p, dq32.p, kp.p, vp.p, H, HKV, D, c.tokens, c.position, cap, 1.f / 16,
                                        pws.p, pb, stream) == 0);
            EXPECT(failed_with(qv_attention_precise(dout.p, dq32.p, kp.p, vp.p, H, HKV, D, c.tokens, c.position, cap,
                                                    1.f / 16, pws.p, pb - 1, stream),
                               "workspace too small"));
            HIP_OK(hipStreamSynchronize(stream));
            EXPECT(all_finite(fetch(dout.p, n, QV_F32)));
        }
    }
    // The fused entry: short context, decode, verification (two tokens on
    // the stream kernel, 3-8 on the ring kernel), prefill chunk.
    const int fused_cases[][2] = {{3, 10}, {1, 500}, {2, 700}, {5, 300}, {8, 1000}, {20, 64}};
    std::vector<float> qn(D), kn(D);
    for (int i = 0; i < D; ++i) qn[i] = 1.f + 0.01f * i, kn[i] = 1.f - 0.001f * i;
    Dev<float> dqn(D), dkn(D);
    HIP_OK(hipMemcpy(dqn.p, qn.data(), D * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dkn.p, kn.data(), D * 4, hipMemcpyHostToDevice));
    for (const auto &fc : fused_cases) {
        const int b = fc[0], pos = fc[1];
        std::vector<float> qg((size_t)b * H * 2 * D), kv((size_t)b * HKV * D);
        for (auto &x : qg) x = normal(rng);
        Dev<float> dqg(qg.size()), dk(kv.size()), dv(kv.size()), dout((size_t)b * H * D);
        HIP_OK(hipMemcpy(dqg.p, qg.data(), qg.size() * 4, hipMemcpyHostToDevice));
        for (auto &x : kv) x = normal(rng);
        HIP_OK(hipMemcpy(dk.p, kv.data(), kv.size() * 4, hipMemcpyHostToDevice));
        for (auto &x : kv) x = normal(rng);
        HIP_OK(hipMemcpy(dv.p, kv.data(), kv.size() * 4, hipMemcpyHostToDevice));
        uint64_t fb = 0;
        EXPECT(qv_attention_fused_workspace(&fb, b, pos) == 0);
        Dev<char> fws(fb + 16);
        EXPECT(failed_with(qv_attention_fused(dout.p, kp2.p, vp2.p, dqg.p, dk.p, dv.p, dqn.p, dkn.p, b, pos, cap,
                                              1e-6f, fws.p, fb - 1, stream),
                           "workspace too small"));
        EXPECT(qv_attention_fused(dout.p, kp2.p, vp2.p, dqg.p, dk.p, dv.p, dqn.p, dkn.p, b, pos, cap, 1e-6f, fws.p,
                                  fb, stream) == 0);
        HIP_OK(hipStreamSynchronize(stream));
        EXPECT(all_finite(fetch(dout.p, (size_t)b * H * D, QV_F32)));
    }
}

// qv_test_attention on host buffers of exactly the documented sizes: the
// caches hold position + batch rows, of which only [0, position) are read.
void test_attention_exact_buffers() {
    std::mt19937 rng(11);
    std::normal_distribution<float> normal(0.f, 1.f);
    for (const auto &bp : {std::pair<int, int>{2, 40}, {1, 0}, {8, 300}, {3, 2047}}) {
        const int b = bp.first, pos = bp.second, n = pos + b;
        std::vector<float> out((size_t)b * H * D), qg((size_t)b * H * 2 * D), key((size_t)b * HKV * D),
            value((size_t)b * HKV * D), qn(D), kn(D);
        std::vector<uint16_t> kc((size_t)n * HKV * D), vc((size_t)n * HKV * D);
        for (auto &x : qg) x = normal(rng);
        for (auto &x : key) x = normal(rng);
        for (auto &x : value) x = normal(rng);
        for (int i = 0; i < D; ++i) qn[i] = kn[i] = 1.f;
        for (size_t i = 0; i < (size_t)pos * HKV * D; ++i) kc[i] = half_bits(0.5f * normal(rng)), vc[i] = half_bits(normal(rng));
        EXPECT(qv_test_attention(out.data(), kc.data(), vc.data(), qg.data(), key.data(), value.data(), qn.data(),
                                 kn.data(), b, pos, 1e-6f) == 0);
        EXPECT(all_finite(out));
        EXPECT(qv_error()[0] == '\0');
    }
}

}  // namespace

int main(int argc, char **argv) {
    std::setvbuf(stdout, nullptr, _IOLBF, 0);
    const bool host_only = argc > 1 && std::strcmp(argv[1], "--host-only") == 0;
    stubs();
    test_attention_validation();
    kv_bytes_sweep();
    device_entry_validation();
    planner_sweep();
    prefill_planner_sweep();
    prefill_prep_planner_sweep();
    int devices = 0;
    const bool gpu = hipGetDeviceCount(&devices) == hipSuccess && devices > 0;
    std::printf("abi_sanitize: host checks done (%d checks, %d failed); %s\n", checks, failures,
                host_only ? "device checks skipped (--host-only)"
                          : gpu ? "running device checks" : "no GPU: device checks skipped");
    if (gpu && !host_only) {
        HIP_OK(hipSetDevice(0));
        device_calls(nullptr);
        hipStream_t stream = nullptr;
        HIP_OK(hipStreamCreate(&stream));
        device_calls(stream);
        HIP_OK(hipStreamDestroy(stream));
        test_attention_exact_buffers();
        HIP_OK(hipDeviceSynchronize());
    }
    std::printf("abi_sanitize: %d checks, %d failed\n", checks, failures);
    std::fflush(stdout);
    std::fflush(stderr);
    // Leave without running the HIP runtime's static destructors: with the
    // ASan runtime linked in, its teardown frees runtime objects after ASan's
    // device-memory allocator has shut down, and ASan's own consistency check
    // then aborts the process.  Nothing of this program needs the teardown.
    std::_Exit(failures == 0 ? 0 : 1);
}
