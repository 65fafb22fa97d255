// capi.cpp — the extern "C" boundary (include/ei_attn.h): argument validation, error
// reporting and dispatch to the gfx950 launchers.  No exception leaves this file; every
// entry point returns an EI_* status and records a message for ei_last_error().
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <string>

#include "../../include/ei_attn.h"
#include "../../include/ei_gguf.h"
#include "../host/gguf_index.h"
#include "launch.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int ok() {
    g_err.clear();
    return EI_OK;
}

int hip_status(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(EI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

#define REQUIRE(cond, ...)                           \
    do {                                             \
        if (!(cond)) return fail(EI_ERR_ARG, __VA_ARGS__); \
    } while (0)

// Shape limits that keep every size and index computation in range: KV heads per layer, and the
// rows of one prefill chunk (B * n_head query rows, B <= 2^20 tokens).
constexpr int kMaxKvHeads = 1024;
constexpr long kMaxPrefillB = 1L << 20, kMaxPrefillRows = 1L << 28;

bool prefill_rows_ok(int B, int n_head) { return B <= kMaxPrefillB && (long)B * n_head <= kMaxPrefillRows; }

int check_heads(int n_head, int n_head_kv, int head_dim) {
    if (head_dim != 128)
        return fail(EI_ERR_UNSUPPORTED, "head_dim %d: only 128 is built (the reference GPU path requires it too)",
                    head_dim);
    REQUIRE(n_head > 0 && n_head_kv > 0, "n_head (%d) and n_head_kv (%d) must be positive", n_head, n_head_kv);
    REQUIRE(n_head_kv <= kMaxKvHeads, "n_head_kv %d above %d", n_head_kv, kMaxKvHeads);
    REQUIRE(n_head % n_head_kv == 0, "n_head %d is not a multiple of n_head_kv %d", n_head, n_head_kv);
    const int g = n_head / n_head_kv;
    if (g > 8) return fail(EI_ERR_UNSUPPORTED, "GQA group %d: built for groups of 1 to 8 query heads", g);
    return EI_OK;
}

int check_rope(int rope_dim, int head_dim) {
    REQUIRE(rope_dim > 0 && rope_dim % 2 == 0 && rope_dim <= head_dim, "rope_dim %d must be even and in (0, %d]",
            rope_dim, head_dim);
    return EI_OK;
}

// the fused decode steps copy the RoPE row (rope_dim/2 float pairs) in whole 16-byte pieces
int check_rope_fused_decode(int rope_dim, int head_dim) {
    if (int e = check_rope(rope_dim, head_dim)) return e;
    if (rope_dim % 4 != 0)
        return fail(EI_ERR_UNSUPPORTED, "rope_dim %d: the fused decode step needs a multiple of 4", rope_dim);
    return EI_OK;
}

}  // namespace

#define EI_API extern "C" __attribute__((visibility("default")))

EI_API const char* ei_last_error(void) { return g_err.c_str(); }

EI_API int ei_abi_version(void) { return EI_ABI_VERSION; }

EI_API int ei_rope_table_fill(float* cs_host, int n_ctx, int rope_dim, double theta) {
    REQUIRE(cs_host != nullptr, "cs_host is null");
    REQUIRE(n_ctx > 0, "n_ctx %d must be positive", n_ctx);
    REQUIRE(rope_dim > 0 && rope_dim % 2 == 0, "rope_dim %d must be even and positive", rope_dim);
    REQUIRE(theta > 0.0, "theta must be positive");
    const int half = rope_dim / 2;
    for (int i = 0; i < half; ++i) {
        const double inv = std::pow(theta, -2.0 * i / rope_dim);
        for (int p = 0; p < n_ctx; ++p) {
            const double th = double(p) * inv;
            cs_host[(size_t(p) * half + i) * 2 + 0] = float(std::cos(th));
            cs_host[(size_t(p) * half + i) * 2 + 1] = float(std::sin(th));
        }
    }
    return ok();
}

EI_API int ei_headnorm_rope(ei_stream_t stream, float* buf, int rows, long row_stride, int n_heads, int head_dim,
                            const float* gamma, const float* cs, const int* pos_dev, int rope_dim, float eps) {
    if (head_dim != 128) return fail(EI_ERR_UNSUPPORTED, "head_dim %d: only 128 is built", head_dim);
    if (int e = check_rope(rope_dim, head_dim)) return e;
    REQUIRE(buf && gamma && cs && pos_dev, "null pointer argument");
    REQUIRE(rows >= 0 && n_heads > 0, "rows %d / n_heads %d", rows, n_heads);
    REQUIRE(row_stride >= (long)n_heads * head_dim, "row_stride %ld < n_heads*head_dim", row_stride);
    if (rows == 0) return ok();
    return hip_status(ei::launch_headnorm_rope(static_cast<hipStream_t>(stream), buf, rows, row_stride, n_heads,
                                               gamma, cs, pos_dev, rope_dim, eps),
                      "ei_headnorm_rope launch");
}

EI_API int ei_kv_append(ei_stream_t stream, const float* k_src, const float* v_src, long src_stride, int rows,
                        float* kc, float* vc, int kd, const int* pos_dev) {
    REQUIRE(k_src && v_src && kc && vc && pos_dev, "null pointer argument");
    REQUIRE(rows >= 0, "rows %d", rows);
    REQUIRE(kd > 0 && kd % 4 == 0, "kd %d must be a positive multiple of 4", kd);
    REQUIRE(src_stride % 4 == 0 && src_stride >= kd, "src_stride %ld must be a multiple of 4 and >= kd", src_stride);
    REQUIRE(aligned16(k_src) && aligned16(v_src) && aligned16(kc) && aligned16(vc), "pointers must be 16-byte aligned");
    if (rows == 0) return ok();
    return hip_status(ei::launch_kv_append(static_cast<hipStream_t>(stream), k_src, v_src, src_stride, rows, kc, vc,
                                           kd, pos_dev),
                      "ei_kv_append launch");
}

EI_API int ei_qkv_prepare(ei_stream_t stream, float* qkv, int rows, long row_stride, int n_head, int n_head_kv,
                          int head_dim, const float* q_gamma, const float* k_gamma, const float* cs,
                          const int* pos_dev, int rope_dim, float eps, float* kc, float* vc) {
    if (int e = check_heads(n_head, n_head_kv, head_dim)) return e;
    if (int e = check_rope(rope_dim, head_dim)) return e;
    REQUIRE(qkv && q_gamma && k_gamma && cs && pos_dev && kc && vc, "null pointer argument");
    REQUIRE(rows >= 0, "rows %d", rows);
    REQUIRE(row_stride >= (long)(n_head + 2 * n_head_kv) * head_dim, "row_stride %ld < (H+2*HKV)*head_dim",
            row_stride);
    if (rows == 0) return ok();
    return hip_status(ei::launch_qkv_prepare(static_cast<hipStream_t>(stream), qkv, rows, row_stride, n_head,
                                             n_head_kv, q_gamma, k_gamma, cs, pos_dev, rope_dim, eps, kc, vc),
                      "ei_qkv_prepare launch");
}

EI_API size_t ei_attn_decode_ws_bytes(int n_seq, int n_head, int n_head_kv, int max_kv) {
    if (n_seq <= 0 || n_seq > 65535 || n_head <= 0 || n_head_kv <= 0 || n_head_kv > kMaxKvHeads || n_head % n_head_kv ||
        max_kv <= 0)
        return 0;
    return ei::decode_ws_bytes(n_seq, n_head, n_head_kv, max_kv);
}

EI_API int ei_attn_workspace_init(ei_stream_t stream, void* ws, size_t ws_bytes) {
    REQUIRE(ws != nullptr, "workspace is null");
    REQUIRE(aligned16(ws), "workspace must be 16-byte aligned");
    return hip_status(ei::launch_ws_clear(static_cast<hipStream_t>(stream), ws, ws_bytes), "workspace clear");
}

EI_API int ei_attn_workspace_status(ei_stream_t stream, const void* ws, size_t ws_bytes, uint32_t* status) {
    REQUIRE(ws != nullptr && status != nullptr, "null pointer argument");
    REQUIRE(ws_bytes >= 256, "workspace of %zu bytes holds no status word", ws_bytes);
    const char* word = static_cast<const char*>(ws) + ei::ws_status_offset(ws_bytes);
    uint32_t v = 0;
    if (int e = hip_status(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "stream sync")) return e;
    if (int e = hip_status(hipMemcpy(&v, word, sizeof v, hipMemcpyDeviceToHost), "status read")) return e;
    *status = v;
    return ok();
}

EI_API int ei_decode_status_check(uint32_t status) {
    if (status == 0) return ok();
    if (status & 1u)
        return fail(EI_ERR_MERGE,
                    "decode workspace status 0x%x: the splits of one (sequence, kv head) ran on different XCDs, so "
                    "the in-kernel split merge may have read stale partials and outputs since the workspace was "
                    "initialised may be wrong (EI_DECODE_MERGE=launch merges in a second launch)",
                    status);
    return fail(EI_ERR_MERGE, "decode workspace status 0x%x: unknown status bits set", status);
}

namespace {

int decode_common(hipStream_t st, ei::DecodeArgs& a, int n_seq, int max_kv, void* ws, size_t ws_bytes, bool fused,
                  bool launch_combine = false, bool capped = true) {
    REQUIRE(max_kv > 0, "max_kv %d must be positive", max_kv);
    REQUIRE(ws != nullptr && aligned16(ws), "workspace missing or not 16-byte aligned");
    const ei::DecodePlan p = ei::decode_plan(n_seq, a.HKV, max_kv, a.block_table != nullptr, capped);
    const ei::DecodeWsLayout lay = ei::decode_ws_layout(n_seq, a.H, a.HKV, max_kv, capped);
    REQUIRE(ei::ws_fits(ws_bytes, lay.partials, lay.units),
            "workspace of %zu bytes too small for n_seq %d, max_kv %d (ei_attn_decode_ws_bytes gives %zu)", ws_bytes,
            n_seq, max_kv, ei::decode_ws_bytes(n_seq, a.H, a.HKV, max_kv));
    char* base = static_cast<char*>(ws);
    a.part_acc = reinterpret_cast<float*>(base);  // partials are laid out with the kernel's head slots
    a.rec = reinterpret_cast<uint32_t*>(base + lay.rec);
    // the status word and the arrival counters below it sit where the workspace's size puts them,
    // so every call on it finds them at the same addresses whatever its plan
    a.status = reinterpret_cast<uint32_t*>(base + ei::ws_status_offset(ws_bytes));
    a.ctr_top = a.status;
    a.chunk = p.chunk;
    a.nsplit = p.nsplit;
    a.units = n_seq * a.HKV;
    a.n_xcc = ei::device_xccs();
    REQUIRE(((long)a.units + a.n_xcc) * a.nsplit <= 0x7FFFFFFFL,
            "n_seq %d x n_head_kv %d x %d key splits: more workgroups than one launch takes", n_seq, a.HKV, a.nsplit);
    a.merge_in_kernel = !launch_combine && ei::decode_merge_in_kernel(p.chunk, a.n_xcc);
    return hip_status(ei::launch_decode(st, a, n_seq, fused), "decode launch");
}

}  // namespace

EI_API int ei_attn_decode(ei_stream_t stream, const float* q, float* out, const float* kc, const float* vc,
                          const int* pos_dev, int n_head, int n_head_kv, int head_dim, float scale, int max_kv,
                          void* ws, size_t ws_bytes) {
    if (int e = check_heads(n_head, n_head_kv, head_dim)) return e;
    REQUIRE(q && out && kc && vc && pos_dev, "null pointer argument");
    REQUIRE(aligned16(q) && aligned16(out) && aligned16(kc) && aligned16(vc), "pointers must be 16-byte aligned");
    ei::DecodeArgs a{};
    a.q = q;
    a.q_stride = (long)n_head * head_dim;
    a.kc = const_cast<float*>(kc);
    a.vc = const_cast<float*>(vc);
    a.pos_dev = pos_dev;
    a.out = out;
    a.H = n_head;
    a.HKV = n_head_kv;
    a.scale = scale;
    return decode_common(static_cast<hipStream_t>(stream), a, 1, max_kv, ws, ws_bytes, false);
}

EI_API int ei_attn_decode_batched(ei_stream_t stream, const float* q, long q_stride, float* out, const float* kc,
                                  const float* vc, const int64_t* kv_offset, const int* kv_len, int n_seq,
                                  int n_head, int n_head_kv, int head_dim, float scale, int max_kv, void* ws,
                                  size_t ws_bytes) {
    if (int e = check_heads(n_head, n_head_kv, head_dim)) return e;
    REQUIRE(q && out && kc && vc && kv_offset && kv_len, "null pointer argument");
    REQUIRE(n_seq > 0 && n_seq <= 65535, "n_seq %d out of range [1, 65535]", n_seq);
    REQUIRE(q_stride >= (long)n_head * head_dim && q_stride % 4 == 0, "q_stride %ld", q_stride);
    REQUIRE(aligned16(q) && aligned16(out) && aligned16(kc) && aligned16(vc), "pointers must be 16-byte aligned");
    ei::DecodeArgs a{};
    a.q = q;
    a.q_stride = q_stride;
    a.kc = const_cast<float*>(kc);
    a.vc = const_cast<float*>(vc);
    a.kv_offset = kv_offset;
    a.kv_len = kv_len;
    a.out = out;
    a.H = n_head;
    a.HKV = n_head_kv;
    a.scale = scale;
    return decode_common(static_cast<hipStream_t>(stream), a, n_seq, max_kv, ws, ws_bytes, false);
}

namespace {

int decode_step_impl(ei_stream_t stream, const float* qkv, long row_stride, float* out, float* kc, float* vc,
                     const int64_t* kv_offset, const int* kv_len, const int* pos_dev, int n_seq, int n_head,
                     int n_head_kv, int head_dim, const float* q_gamma, const float* k_gamma, const float* cs,
                     int rope_dim, float eps, float scale, int max_kv, void* ws, size_t ws_bytes, bool no_alloc) {
    if (int e = check_heads(n_head, n_head_kv, head_dim)) return e;
    if (int e = check_rope_fused_decode(rope_dim, head_dim)) return e;
    REQUIRE(qkv && out && kc && vc && q_gamma && k_gamma && cs, "null pointer argument");
    REQUIRE(n_seq > 0 && n_seq <= 65535, "n_seq %d out of range [1, 65535]", n_seq);
    REQUIRE(kv_len != nullptr || (pos_dev != nullptr && n_seq == 1),
            "either kv_len, or pos_dev with n_seq == 1, must be given");
    REQUIRE(n_seq == 1 || kv_offset != nullptr, "kv_offset is required when n_seq > 1");
    REQUIRE(row_stride >= (long)(n_head + 2 * n_head_kv) * head_dim, "row_stride %ld < (H+2*HKV)*head_dim",
            row_stride);
    REQUIRE(aligned16(qkv) && aligned16(out) && aligned16(kc) && aligned16(vc) && row_stride % 4 == 0,
            "pointers and row_stride must be 16-byte aligned");
    ei::DecodeArgs a{};
    a.q = qkv;
    a.q_stride = row_stride;
    a.kc = kc;
    a.vc = vc;
    a.kv_offset = kv_offset;
    a.kv_len = kv_len;
    a.pos_dev = pos_dev;
    a.out = out;
    a.H = n_head;
    a.HKV = n_head_kv;
    a.scale = scale;
    a.q_gamma = q_gamma;
    a.k_gamma = k_gamma;
    a.cs = reinterpret_cast<const float2*>(cs);
    a.rope_dim = rope_dim;
    a.eps = eps;
    bool capped = true;
    if (no_alloc) {
        // the capped plan (1024-key chunks) if its partials fit the static array, else the plan
        // without the cap (fewer splits of longer sequences: a ragged batch balances less well)
        REQUIRE(max_kv > 0, "max_kv %d must be positive", max_kv);
        const ei::DecodeWsLayout lay = ei::decode_ws_layout(n_seq, n_head, n_head_kv, max_kv, true);
        if (!ei::ws_fits(ei::kDecodeScratchBytes, lay.partials, lay.units)) {
            capped = false;
            const ei::DecodeWsLayout lay2 = ei::decode_ws_layout(n_seq, n_head, n_head_kv, max_kv, false);
            REQUIRE(ei::ws_fits(ei::kDecodeScratchBytes, lay2.partials, lay2.units),
                    "n_seq %d, n_head %d, n_head_kv %d, max_kv %d need %zu bytes of scratch; the allocation-free step "
                    "has %zu (use ei_decode_step with a workspace)",
                    n_seq, n_head, n_head_kv, max_kv, ei::ws_bytes_for(lay2.partials, lay2.units),
                    ei::kDecodeScratchBytes);
        }
        if (int e = hip_status(ei::decode_scratch(&ws), "scratch address lookup")) return e;
        ws_bytes = ei::kDecodeScratchBytes;
    }
    // the allocation-free step always merges the splits in the second launch: its partials are
    // fully rewritten by every call, so nothing in the shared scratch has to start at zero
    return decode_common(static_cast<hipStream_t>(stream), a, n_seq, max_kv, ws, ws_bytes, true, no_alloc, capped);
}

}  // namespace

EI_API int ei_decode_step(ei_stream_t stream, const float* qkv, long row_stride, float* out, float* kc, float* vc,
                          const int64_t* kv_offset, const int* kv_len, const int* pos_dev, int n_seq, int n_head,
                          int n_head_kv, int head_dim, const float* q_gamma, const float* k_gamma, const float* cs,
                          int rope_dim, float eps, float scale, int max_kv, void* ws, size_t ws_bytes) {
    return decode_step_impl(stream, qkv, row_stride, out, kc, vc, kv_offset, kv_len, pos_dev, n_seq, n_head,
                            n_head_kv, head_dim, q_gamma, k_gamma, cs, rope_dim, eps, scale, max_kv, ws, ws_bytes,
                            false);
}

EI_API int ei_decode_step_noalloc(ei_stream_t stream, const float* qkv, long row_stride, float* out, float* kc,
                                  float* vc, const int64_t* kv_offset, const int* kv_len, const int* pos_dev, int n_seq,
                                  int n_head, int n_head_kv, int head_dim, const float* q_gamma, const float* k_gamma,
                                  const float* cs, int rope_dim, float eps, float scale, int max_kv) {
    // Every call on one GPU shares that GPU's static array.  A call issued while another host
    // thread is still issuing one on the same GPU is refused; calls issued one after another on
    // different streams can still overlap on the GPU, which the caller must not do.
    int dev = 0;
    if (int e = hip_status(hipGetDevice(&dev), "device query")) return e;
    REQUIRE(dev >= 0 && dev < 64, "device %d out of range", dev);
    static std::atomic<int> issuing[64];
    if (issuing[dev].exchange(1, std::memory_order_acquire))
        return fail(EI_ERR_ARG,
                    "another ei_decode_step_noalloc call on device %d is being issued by another thread: calls on "
                    "one GPU share one scratch array and must not overlap",
                    dev);
    const int rc = decode_step_impl(stream, qkv, row_stride, out, kc, vc, kv_offset, kv_len, pos_dev, n_seq, n_head,
                                    n_head_kv, head_dim, q_gamma, k_gamma, cs, rope_dim, eps, scale, max_kv, nullptr,
                                    0, true);
    issuing[dev].store(0, std::memory_order_release);
    return rc;
}

namespace {

int check_paged(const int* block_table, int max_blocks, int block_size, const int* kv_len, int max_kv, int* shift) {
    REQUIRE(block_table && kv_len, "block_table and kv_len are required");
    REQUIRE(block_size >= 16 && (block_size & (block_size - 1)) == 0,
            "block_size %d must be a power of two >= 16 (whole 16-key tiles per block)", block_size);
    REQUIRE(max_blocks > 0 && (long)max_blocks * block_size >= max_kv,
            "max_blocks %d x block_size %d does not cover max_kv %d", max_blocks, block_size, max_kv);
    // the kernels index a sequence's keys and the table's span with 32-bit ints
    REQUIRE((long)max_blocks * block_size <= 0x7FFFFFFFL, "max_blocks %d x block_size %d exceeds 2^31 - 1 keys",
            max_blocks, block_size);
    REQUIRE(max_kv > 0 && (long)max_kv <= (long)ei::kDecodeMaxSplits * ei::kDecodePagedMaxChunk,
            "max_kv %d out of range for paged decode", max_kv);
    int sh = 0;
    while ((1 << sh) < block_size) ++sh;
    *shift = sh;
    return EI_OK;
}

}  // namespace

EI_API int ei_attn_decode_paged(ei_stream_t stream, const float* q, long q_stride, float* out, const float* kc,
                                const float* vc, const int* block_table, int max_blocks, int block_size,
                                const int* kv_len, int n_seq, int n_head, int n_head_kv, int head_dim, float scale,
                                int max_kv, void* ws, size_t ws_bytes) {
    if (int e = check_heads(n_head, n_head_kv, head_dim)) return e;
    REQUIRE(q && out && kc && vc, "null pointer argument");
    REQUIRE(n_seq > 0 && n_seq <= 65535, "n_seq %d out of range [1, 65535]", n_seq);
    REQUIRE(q_stride >= (long)n_head * head_dim && q_stride % 4 == 0, "q_stride %ld", q_stride);
    REQUIRE(aligned16(q) && aligned16(out) && aligned16(kc) && aligned16(vc), "pointers must be 16-byte aligned");
    int shift = 0;
    if (int e = check_paged(block_table, max_blocks, block_size, kv_len, max_kv, &shift)) return e;
    ei::DecodeArgs a{};
    a.q = q;
    a.q_stride = q_stride;
    a.kc = const_cast<float*>(kc);
    a.vc = const_cast<float*>(vc);
    a.block_table = block_table;
    a.max_blocks = max_blocks;
    a.block_shift = shift;
    a.kv_len = kv_len;
    a.out = out;
    a.H = n_head;
    a.HKV = n_head_kv;
    a.scale = scale;
    return decode_common(static_cast<hipStream_t>(stream), a, n_seq, max_kv, ws, ws_bytes, false);
}

EI_API int ei_decode_step_paged(ei_stream_t stream, const float* qkv, long row_stride, float* out, float* kc, float* vc,
                                const int* block_table, int max_blocks, int block_size, const int* kv_len, int n_seq,
                                int n_head, int n_head_kv, int head_dim, const float* q_gamma, const float* k_gamma,
                                const float* cs, int rope_dim, float eps, float scale, int max_kv, void* ws,
                                size_t ws_bytes) {
    if (int e = check_heads(n_head, n_head_kv, head_dim)) return e;
    if (int e = check_rope_fused_decode(rope_dim, head_dim)) return e;
    REQUIRE(qkv && out && kc && vc && q_gamma && k_gamma && cs, "null pointer argument");
    REQUIRE(n_seq > 0 && n_seq <= 65535, "n_seq %d out of range [1, 65535]", n_seq);
    REQUIRE(row_stride >= (long)(n_head + 2 * n_head_kv) * head_dim, "row_stride %ld < (H+2*HKV)*head_dim",
            row_stride);
    REQUIRE(aligned16(qkv) && aligned16(out) && aligned16(kc) && aligned16(vc) && row_stride % 4 == 0,
            "pointers and row_stride must be 16-byte aligned");
    int shift = 0;
    if (int e = check_paged(block_table, max_blocks, block_size, kv_len, max_kv, &shift)) return e;
    ei::DecodeArgs a{};
    a.q = qkv;
    a.q_stride = row_stride;
    a.kc = kc;
    a.vc = vc;
    a.block_table = block_table;
    a.max_blocks = max_blocks;
    a.block_shift = shift;
    a.kv_len = kv_len;
    a.out = out;
    a.H = n_head;
    a.HKV = n_head_kv;
    a.scale = scale;
    a.q_gamma = q_gamma;
    a.k_gamma = k_gamma;
    a.cs = reinterpret_cast<const float2*>(cs);
    a.rope_dim = rope_dim;
    a.eps = eps;
    return decode_common(static_cast<hipStream_t>(stream), a, n_seq, max_kv, ws, ws_bytes, true);
}

EI_API int ei_attn_prefill(ei_stream_t stream, const float* q, long q_stride, float* out, const float* kc,
                           const float* vc, const int* pos_dev, int B, int n_head, int n_head_kv, int head_dim,
                           float scale) {
    if (int e = check_heads(n_head, n_head_kv, head_dim)) return e;
    REQUIRE(q && out && kc && vc && pos_dev, "null pointer argument");
    REQUIRE(B >= 0, "B %d", B);
    REQUIRE(prefill_rows_ok(B, n_head), "B %d x n_head %d: at most 2^20 tokens and 2^28 query rows per launch", B,
            n_head);
    REQUIRE(q_stride >= (long)n_head * head_dim && q_stride % 4 == 0, "q_stride %ld", q_stride);
    REQUIRE(aligned16(q) && aligned16(out) && aligned16(kc) && aligned16(vc), "pointers must be 16-byte aligned");
    if (B == 0) return ok();
    return hip_status(ei::launch_prefill(static_cast<hipStream_t>(stream), q, q_stride, out, kc, vc, pos_dev, B,
                                         n_head, n_head_kv, scale, 1, nullptr),
                      "prefill launch");
}

EI_API size_t ei_attn_prefill_ws_bytes(int max_B, int n_head, int n_head_kv, int max_kv) {
    if (max_B <= 0 || n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv || max_kv < max_B) return 0;
    if (n_head_kv > kMaxKvHeads || !prefill_rows_ok(max_B, n_head)) return 0;
    size_t most = 0;  // the plan varies with B: size for every chunk of up to max_B rows
    for (int b = 1; b <= max_B; ++b) {
        const size_t need = ei::prefill_ws_bytes(b, n_head, n_head_kv, max_kv);
        if (need > most) most = need;
    }
    return most;
}

EI_API int ei_attn_prefill_split(ei_stream_t stream, const float* q, long q_stride, float* out, const float* kc,
                                 const float* vc, const int* pos_dev, int B, int n_head, int n_head_kv, int head_dim,
                                 float scale, int max_kv, void* ws, size_t ws_bytes) {
    if (int e = check_heads(n_head, n_head_kv, head_dim)) return e;
    REQUIRE(q && out && kc && vc && pos_dev, "null pointer argument");
    REQUIRE(B >= 0, "B %d", B);
    REQUIRE(prefill_rows_ok(B, n_head), "B %d x n_head %d: at most 2^20 tokens and 2^28 query rows per launch", B,
            n_head);
    REQUIRE(max_kv >= B, "max_kv %d < B %d", max_kv, B);
    REQUIRE(q_stride >= (long)n_head * head_dim && q_stride % 4 == 0, "q_stride %ld", q_stride);
    REQUIRE(aligned16(q) && aligned16(out) && aligned16(kc) && aligned16(vc), "pointers must be 16-byte aligned");
    if (B == 0) return ok();
    const int ksplit = ei::prefill_split(B, n_head, n_head_kv, max_kv);
    const size_t need = ei::prefill_ws_bytes(B, n_head, n_head_kv, max_kv);
    REQUIRE(ws_bytes >= need, "workspace %zu B < %zu B (ei_attn_prefill_ws_bytes)", ws_bytes, need);
    REQUIRE(need == 0 || (ws && aligned16(ws)), "workspace must be a 16-byte aligned device pointer");
    return hip_status(ei::launch_prefill(static_cast<hipStream_t>(stream), q, q_stride, out, kc, vc, pos_dev, B,
                                         n_head, n_head_kv, scale, ksplit, ws),
                      "prefill launch");
}

namespace {

int prefill_step_impl(ei_stream_t stream, float* qkv, long row_stride, float* out, float* kc, float* vc,
                      const int* pos_dev, int B, int n_head, int n_head_kv, int head_dim, const float* q_gamma,
                      const float* k_gamma, const float* cs, int rope_dim, float eps, float scale, int max_kv, void* ws,
                      size_t ws_bytes, const int* block_table, int block_shift, int max_blocks) {
    if (int e = check_heads(n_head, n_head_kv, head_dim)) return e;
    if (int e = check_rope(rope_dim, head_dim)) return e;
    REQUIRE(qkv && out && kc && vc && pos_dev && q_gamma && k_gamma && cs, "null pointer argument");
    REQUIRE(B >= 0, "B %d", B);
    REQUIRE(prefill_rows_ok(B, n_head), "B %d x n_head %d: at most 2^20 tokens and 2^28 query rows per launch", B,
            n_head);
    REQUIRE(max_kv >= B, "max_kv %d < B %d", max_kv, B);
    REQUIRE(row_stride >= (long)(n_head + 2 * n_head_kv) * head_dim, "row_stride %ld < (H+2*HKV)*head_dim",
            row_stride);
    REQUIRE(aligned16(qkv) && aligned16(out) && aligned16(kc) && aligned16(vc) && row_stride % 4 == 0,
            "pointers and row_stride must be 16-byte aligned");
    if (B == 0) return ok();
    const int ksplit = ei::prefill_split(B, n_head, n_head_kv, max_kv);
    const size_t need = ei::prefill_ws_bytes(B, n_head, n_head_kv, max_kv);
    REQUIRE(ws_bytes >= need, "workspace %zu B < %zu B (ei_attn_prefill_ws_bytes)", ws_bytes, need);
    REQUIRE(need == 0 || (ws && aligned16(ws)), "workspace must be a 16-byte aligned device pointer");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    // the attention kernel norms q itself (full-width RoPE, every Qwen3) when the key range is
    // split over at most four shares: each share norms the q rows of the units it runs (one
    // pass for most shares), which costs less than the q traffic it saves in the prologue
    // (512-token chunks, 4 shares: chunk step 90.7 -> 91.3 TFLOP/s); with more shares the
    // prologue norms every head in place first (the paged variant always takes the full
    // prologue: the in-kernel norm and the block table together exceed the attention kernel's
    // register budget)
    const bool fuse_q = rope_dim == head_dim && ksplit <= 4 && block_table == nullptr;
    if (int e = hip_status(ei::launch_qkv_prepare(st, qkv, B, row_stride, n_head, n_head_kv, q_gamma, k_gamma, cs,
                                                  pos_dev, rope_dim, eps, kc, vc, fuse_q ? n_head : 0, block_table,
                                                  block_shift, max_blocks),
                           "prefill step: prologue launch"))
        return e;
    return hip_status(ei::launch_prefill(st, qkv, row_stride, out, kc, vc, pos_dev, B, n_head, n_head_kv, scale, ksplit,
                                         ws, fuse_q ? q_gamma : nullptr, cs, eps, block_table, block_shift, max_blocks),
                      "prefill step: attention launch");
}

}  // namespace

EI_API int ei_prefill_step(ei_stream_t stream, float* qkv, long row_stride, float* out, float* kc, float* vc,
                           const int* pos_dev, int B, int n_head, int n_head_kv, int head_dim, const float* q_gamma,
                           const float* k_gamma, const float* cs, int rope_dim, float eps, float scale, int max_kv,
                           void* ws, size_t ws_bytes) {
    return prefill_step_impl(stream, qkv, row_stride, out, kc, vc, pos_dev, B, n_head, n_head_kv, head_dim, q_gamma,
                             k_gamma, cs, rope_dim, eps, scale, max_kv, ws, ws_bytes, nullptr, 0, 0);
}

EI_API int ei_prefill_step_paged(ei_stream_t stream, float* qkv, long row_stride, float* out, float* kc, float* vc,
                                 const int* block_table, int max_blocks, int block_size, const int* pos_dev, int B,
                                 int n_head, int n_head_kv, int head_dim, const float* q_gamma, const float* k_gamma,
                                 const float* cs, int rope_dim, float eps, float scale, int max_kv, void* ws,
                                 size_t ws_bytes) {
    REQUIRE(block_table != nullptr, "null block_table");
    REQUIRE(block_size >= 32 && (block_size & (block_size - 1)) == 0,
            "block_size %d must be a power of two >= 32 (whole 32-key prefill tiles per block)", block_size);
    REQUIRE(max_blocks > 0 && (long)max_blocks * block_size >= max_kv,
            "max_blocks %d x block_size %d does not cover max_kv %d", max_blocks, block_size, max_kv);
    // the kernels index a sequence's keys and the table's span with 32-bit ints
    REQUIRE((long)max_blocks * block_size <= 0x7FFFFFFFL, "max_blocks %d x block_size %d exceeds 2^31 - 1 keys",
            max_blocks, block_size);
    int shift = 0;
    while ((1 << shift) < block_size) ++shift;
    return prefill_step_impl(stream, qkv, row_stride, out, kc, vc, pos_dev, B, n_head, n_head_kv, head_dim, q_gamma,
                             k_gamma, cs, rope_dim, eps, scale, max_kv, ws, ws_bytes, block_table, shift, max_blocks);
}

EI_API int ei_qkv_project(ei_stream_t stream, const float* x, long x_stride, int rows, int n_embd,
                          const float* attn_norm, float eps, const void* w, int w_type, int n_out, float* qkv,
                          long qkv_stride) {
    REQUIRE(x && attn_norm && w && qkv, "null pointer argument");
    REQUIRE(w_type == EI_W_F32 || w_type == EI_W_F16 || w_type == EI_W_Q8_0 || w_type == EI_W_Q4_K ||
                w_type == EI_W_Q6_K,
            "w_type %d: EI_W_F32 (0), EI_W_F16 (1), EI_W_Q8_0 (8), EI_W_Q4_K (12) or EI_W_Q6_K (14)", w_type);
    if (!ei::qkv_project_built(n_embd, w_type))
        return fail(EI_ERR_UNSUPPORTED,
                    "n_embd %d, w_type %d: built for 1024, 2048, 2560, 4096 and 5120 (F32); also 8192 and 10240 (F16); "
                    "1024, 2048, 2560, 4096 and 5120 (Q8_0, Q4_K, Q6_K)",
                    n_embd, w_type);
    REQUIRE(rows >= 0 && rows <= ei::qkv_project_max_rows(n_embd), "rows %d: at most %d rows per launch at n_embd %d",
            rows, ei::qkv_project_max_rows(n_embd), n_embd);
    REQUIRE(n_out > 0, "n_out %d", n_out);
    REQUIRE(x_stride >= n_embd && qkv_stride >= n_out, "x_stride %ld / qkv_stride %ld too small", x_stride,
            qkv_stride);
    REQUIRE(aligned16(x) && aligned16(w) && aligned16(attn_norm) && x_stride % 4 == 0,
            "x, w, attn_norm and x_stride must be 16-byte aligned");
    if (rows == 0) return ok();
    return hip_status(ei::launch_qkv_project(static_cast<hipStream_t>(stream), x, x_stride, rows, n_embd, attn_norm,
                                             eps, w, w_type, n_out, qkv, qkv_stride),
                      "qkv projection launch");
}

EI_API int ei_qkv_project_max_rows(int n_embd) { return n_embd > 0 ? ei::qkv_project_max_rows(n_embd) : 0; }

EI_API int ei_stream_ceiling(ei_stream_t stream, const float* kc, const float* vc, int n_head_kv, int kv_len,
                             float* sink) {
    REQUIRE(kc && vc && sink, "null pointer argument");
    REQUIRE(n_head_kv > 0 && kv_len > 0, "n_head_kv %d / kv_len %d", n_head_kv, kv_len);
    REQUIRE(aligned16(kc) && aligned16(vc), "pointers must be 16-byte aligned");
    return hip_status(ei::launch_stream_ceiling(static_cast<hipStream_t>(stream), kc, vc, n_head_kv, kv_len, sink),
                      "stream ceiling launch");
}

EI_API int ei_read_ceiling(ei_stream_t stream, const void* src, size_t bytes, int n_workgroups, int all_in_flight,
                           void* sink) {
    REQUIRE(src && sink, "null pointer argument");
    REQUIRE(aligned16(src) && aligned16(sink), "pointers must be 16-byte aligned");
    REQUIRE(bytes % 16 == 0 && bytes > 0, "bytes %zu must be a positive multiple of 16", bytes);
    REQUIRE(n_workgroups > 0 && n_workgroups <= 65535, "n_workgroups %d out of range", n_workgroups);
    REQUIRE(bytes <= (size_t)n_workgroups * 256 * 64 * 16, "bytes %zu: more than 64 loads per thread", bytes);
    return hip_status(ei::launch_read_ceiling(static_cast<hipStream_t>(stream), src, bytes, n_workgroups,
                                              all_in_flight != 0, sink),
                      "read ceiling launch");
}

EI_API int ei_synth_fill(ei_stream_t stream, float* dst, size_t n, uint64_t seed, uint64_t offset, long row_len,
                         long spike_every, float spike_mult) {
    REQUIRE(dst != nullptr || n == 0, "dst is null");
    REQUIRE(row_len > 0, "row_len %ld must be positive", row_len);
    return hip_status(ei::launch_synth_fill(static_cast<hipStream_t>(stream), dst, n, seed, offset, row_len,
                                            spike_every, spike_mult),
                      "synth fill launch");
}

// ------------------------------------------------------------------ GGUF reader (include/ei_gguf.h)
struct ei_gguf {
    ei::gguf::Index file;
    explicit ei_gguf(const char* path) : file(path) {}
};

EI_API ei_gguf* ei_gguf_open(const char* path) {
    if (!path) {
        fail(EI_ERR_ARG, "path is null");
        return nullptr;
    }
    try {
        ei_gguf* g = new ei_gguf(path);
        ok();
        return g;
    } catch (const std::exception& e) {
        fail(EI_ERR_ARG, "%s", e.what());
    } catch (...) {
        fail(EI_ERR_ARG, "unknown error reading %s", path);
    }
    return nullptr;
}

EI_API void ei_gguf_close(ei_gguf* g) { delete g; }

EI_API int ei_gguf_version(const ei_gguf* g) { return g ? (int)g->file.version() : 0; }

EI_API long ei_gguf_n_tensors(const ei_gguf* g) { return g ? (long)g->file.tensors().size() : 0; }

EI_API int ei_gguf_tensor(const ei_gguf* g, long index, const char** name, int* type, int* n_dims, uint64_t* ne,
                          const void** data, uint64_t* nbytes) {
    REQUIRE(g != nullptr, "file handle is null");
    REQUIRE(index >= 0 && index < (long)g->file.tensors().size(), "tensor index %ld out of range", index);
    const ei::gguf::TensorSlot& t = g->file.tensors()[(size_t)index];
    if (name) *name = t.name.c_str();
    if (type) *type = (int)t.type;
    if (n_dims) *n_dims = (int)t.rank;
    if (ne)
        for (size_t i = 0; i < 4; ++i) ne[i] = t.dims[i];
    if (data) *data = t.data;
    if (nbytes) *nbytes = t.bytes;
    return ok();
}

EI_API long ei_gguf_find_tensor(const ei_gguf* g, const char* name) {
    if (!g || !name) return -1;
    const ei::gguf::TensorSlot* t = g->file.tensor(name);
    return t ? (long)(t - g->file.tensors().data()) : -1;
}

namespace {

template <class F>
int gguf_call(const ei_gguf* g, const char* key, F f) {
    REQUIRE(g != nullptr && key != nullptr, "null argument");
    try {
        f();
        return ok();
    } catch (const std::exception& e) {
        return fail(EI_ERR_ARG, "%s", e.what());
    }
}

}  // namespace

EI_API int ei_gguf_get_int(const ei_gguf* g, const char* key, int64_t* out) {
    return gguf_call(g, key, [&] {
        const int64_t v = g->file.integer(key);
        if (out) *out = v;
    });
}

EI_API int ei_gguf_get_float(const ei_gguf* g, const char* key, double* out) {
    return gguf_call(g, key, [&] {
        const double v = g->file.number(key);
        if (out) *out = v;
    });
}

EI_API int ei_gguf_get_str(const ei_gguf* g, const char* key, const char** out) {
    return gguf_call(g, key, [&] {
        const std::string& v = g->file.text(key);
        if (out) *out = v.c_str();
    });
}

EI_API int ei_gguf_qwen3_config(const ei_gguf* g, ei_qwen3_config* out) {
    REQUIRE(g != nullptr && out != nullptr, "null argument");
    try {
        const ei::gguf::Qwen3Config c = ei::gguf::qwen3_config(g->file);
        out->n_layer = c.n_layer;
        out->n_embd = c.n_embd;
        out->n_ff = c.n_ff;
        out->n_head = c.n_head;
        out->n_head_kv = c.n_head_kv;
        out->head_dim = c.head_dim;
        out->rope_dim = c.rope_dim;
        out->n_ctx_train = c.n_ctx_train;
        out->n_vocab = c.n_vocab;
        out->rope_base = c.rope_base;
        out->eps = c.eps;
        return ok();
    } catch (const std::exception& e) {
        return fail(EI_ERR_ARG, "%s", e.what());
    }
}
