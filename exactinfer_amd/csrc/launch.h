// launch.h — internal launchers behind the C ABI (capi.cpp validates, these launch).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>

namespace ei {

// Workspaces of the decode's split merge are laid out by their size alone, so that
// calls of any plan on one workspace agree: the status word at the top, below it a zone of
// arrival counters (one 256-byte line per unit, unit u at (u + 1) lines below the status word;
// every call leaves them at zero), and the partials of the call's plan from the start.  The
// counter zone is the top sixteenth, so partials and counters never overlap whatever the plan.
inline size_t ws_status_offset(size_t ws_bytes) { return (ws_bytes - 256) & ~(size_t)255; }
inline size_t ws_counter_zone(size_t ws_bytes) { return (ws_bytes / 16) & ~(size_t)255; }
// workspace bytes for partials of up to `partials` bytes and up to `units` counters
inline size_t ws_bytes_for(size_t partials, size_t units) {
    const size_t a = ((partials + 1024) * 16 / 15 + 255) & ~(size_t)255;
    const size_t b = (units * 256 * 16 + 1024 + 255) & ~(size_t)255;
    return a > b ? a : b;
}
// whether a call's partials and counters fit the workspace's zones
inline bool ws_fits(size_t ws_bytes, size_t partials, size_t units) {
    if (ws_bytes < 1024) return false;
    const size_t zone = ws_counter_zone(ws_bytes);
    return units * 256 <= zone && partials + zone + 512 <= ws_bytes;
}

// Opt kernel f into `bytes` of dynamic LDS (> 64 KB needs it) once per process.  Setting the
// attribute is idempotent, so first launches racing from several host threads only repeat it.
inline hipError_t opt_in_lds(std::atomic<bool>& done, const void* f, size_t bytes) {
    if (done.load(std::memory_order_acquire)) return hipSuccess;
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess) done.store(true, std::memory_order_release);
    return e;
}

// ------------------------------------------------------------------ prologue.hip
hipError_t launch_headnorm_rope(hipStream_t st, float* buf, int rows, long row_stride, int n_heads,
                                const float* gamma, const float* cs, const int* pos_dev, int rope_dim, float eps);
hipError_t launch_kv_append(hipStream_t st, const float* k_src, const float* v_src, long src_stride, int rows,
                            float* kc, float* vc, int kd, const int* pos_dev);
// h_begin: first head processed (0: all; H: the key heads and the cache append only)
hipError_t launch_qkv_prepare(hipStream_t st, float* qkv, int rows, long row_stride, int H, int HKV,
                              const float* q_gamma, const float* k_gamma, const float* cs, const int* pos_dev,
                              int rope_dim, float eps, float* kc, float* vc, int h_begin = 0,
                              const int* block_table = nullptr, int block_shift = 0, int max_blocks = 0);
hipError_t launch_synth_fill(hipStream_t st, float* dst, size_t n, uint64_t seed, uint64_t offset, long row_len,
                             long spike_every, float spike_mult);

// ------------------------------------------------------------------ decode.hip
// Split plan: keys of one (sequence, kv head) are cut into `nsplit` chunks of `chunk`
// keys (a multiple of the 64-key sub-tile); fixed by max_kv so graphs replay unchanged.
struct DecodePlan {
    int chunk;
    int nsplit;
};
constexpr int kDecodeMaxSplits = 256;
constexpr int kDecodePagedMaxChunk = 8192;  // 4 waves x 128 tiles of 16 keys
constexpr int kDecodeMaxChunk = 1024;       // longer keys are split (ragged batches balance across CUs)
// capped: chunks of at most kDecodeMaxChunk keys (every workspace call); the allocation-free step
// falls back to the uncapped plan when the capped one does not fit its static array
DecodePlan decode_plan(int n_seq, int HKV, int max_kv, bool paged, bool capped = true);
size_t decode_ws_bytes(int n_seq, int H, int HKV, int max_kv);
// the call's partials: accumulators at 0, then the split records (ending at `partials`)
struct DecodeWsLayout {
    size_t rec, partials, units;
};
DecodeWsLayout decode_ws_layout(int n_seq, int H, int HKV, int max_kv, bool capped = true);
int decode_group_slots(int g);  // heads per KV head the decode kernel is built for (0: unsupported)

struct DecodeArgs {
    const float* q;         // raw [Q|K|V] row (fused) or normed q [H][128], per sequence
    long q_stride;          // floats between sequences
    float* kc;              // cache base (rows of HKV*128 floats)
    float* vc;
    const int64_t* kv_offset;  // per-sequence first cache row, or null (0)
    const int* block_table;    // paged: [n_seq][max_blocks] physical block of each logical block, or null
    int max_blocks;
    int block_shift;           // paged: log2(block size), block size a power of two >= 16
    const int* kv_len;         // per-sequence visible keys, or null (then *pos_dev + 1)
    const int* pos_dev;
    float* out;             // [n_seq][H][128]
    int H, HKV;
    float scale;
    int chunk, nsplit;
    float* part_acc;        // [n_seq*HKV*nsplit][G][128]
    uint32_t* rec;          // [n_seq*HKV*nsplit][32]: split record line, word 1 the XCD it ran on,
                            // words 2+2g, 3+2g the (m, l) of head slot g (float bits)
    uint32_t* ctr_top;      // the workspace's status word; unit u's arrival counter of the in-kernel
                            // merge sits (u+1)*256 bytes below it, wherever the call's plan puts its
                            // partials (zero between launches)
    uint32_t* status;       // sticky word: bit 0 set when a workgroup ran on another XCD than its grid slot says
    int units;              // n_seq * HKV
    int n_xcc;              // XCDs the grid is spread over (workgroup b runs on XCD b % n_xcc)
    bool merge_in_kernel;   // the last workgroup of a unit merges its splits (else k_combine does)
    // fused prologue
    const float* q_gamma;
    const float* k_gamma;
    const float2* cs;
    int rope_dim;
    float eps;
};

hipError_t launch_decode(hipStream_t st, const DecodeArgs& a, int n_seq, bool fused);
int device_xccs();              // XCDs of the current device
// split merge inside the decode launch for this chunk size on a device of n_xcc XCDs (only where
// the placement it relies on was validated: 8 XCDs, or 1)
bool decode_merge_in_kernel(int chunk, int n_xcc);
hipError_t launch_ws_clear(hipStream_t st, void* ws, size_t bytes);
// the decode plan's memory traffic alone, for one sequence of len keys; sink takes one float per workgroup
hipError_t launch_stream_ceiling(hipStream_t st, const float* kc, const float* vc, int HKV, int len, float* sink);
hipError_t launch_read_ceiling(hipStream_t st, const void* src, size_t bytes, int n_wg, bool all_in_flight,
                               void* sink);
// allocation-free decode: this device's address of a static scratch array of kDecodeScratchBytes
constexpr size_t kDecodeScratchBytes = size_t(4) << 20;
hipError_t decode_scratch(void** ptr);

// ------------------------------------------------------------------ project.hip
// attention RMSNorm of B activation rows + the fused QKV product (raw [Q|K|V] rows out)
constexpr int kProjMaxRows = 4;
int qkv_project_max_rows(int E);                // rows per launch at hidden size E
bool qkv_project_built(int E, int w_type);      // a kernel exists for hidden size E and this weight type
hipError_t launch_qkv_project(hipStream_t st, const float* x, long x_stride, int B, int E, const float* gamma,
                              float eps, const void* w, int w_type, int n_out, float* out, long out_stride);

// ------------------------------------------------------------------ prefill.hip
// Key split across workgroups for short chunks: ksplit shares per query block, merged by a
// second launch; fixed by (B, max_kv) so graphs replay unchanged.
constexpr int kPrefillMaxSplit = 8;
int prefill_split(int B, int H, int HKV, int max_kv);
size_t prefill_ws_bytes(int B, int H, int HKV, int max_kv);  // 0 when no split is planned
// q_gamma != nullptr: the q rows are raw projections; the kernel applies QK-norm + full-width
// RoPE (table cs of rope_dim 128, eps) to each row where it stages it, leaving the q buffer
// untouched.  block_table != nullptr: the keys sit in a paged pool (block size 2^block_shift >= 32;
// q normed beforehand: the two together are not built).
hipError_t launch_prefill(hipStream_t st, const float* q, long q_stride, float* out, const float* kc,
                          const float* vc, const int* pos_dev, int B, int H, int HKV, float scale, int ksplit,
                          void* ws, const float* q_gamma = nullptr, const float* cs = nullptr, float eps = 0.f,
                          const int* block_table = nullptr, int block_shift = 0, int max_blocks = 0);

}  // namespace ei
