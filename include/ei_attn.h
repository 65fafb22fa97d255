/*
 * ei_attn.h — C ABI of the MI355X (gfx950) Qwen3 attention hot path.
 *
 * Conventions (mirroring the reference CUDA backend's, src/cuda/model_cuda.cu):
 *  - Every entry point returns an int status: EI_OK (0) or an EI_ERR_* code; the message of
 *    the last failure on the calling thread is returned by ei_last_error().  No C++
 *    exception crosses this boundary (the reference throws std::runtime_error from CK/
 *    CK_LAUNCH, src/cuda/model_cuda.cu:40-44; a C++ caller turns a non-zero status back
 *    into that exception).
 *  - All tensor pointers are device pointers owned by the caller; the library allocates
 *    nothing.  `stream` is a hipStream_t (NULL = the default stream).  Launches are
 *    asynchronous, perform no host synchronisation and are capturable into a hipGraph.
 *  - Positions may live in device memory (`pos_dev`) so a captured graph replays
 *    unchanged while the position advances (src/cuda/model_cuda.cu:1632, :1846).
 *  - fp32 everywhere; head_dim must be 128 (the reference GPU path requires it,
 *    src/cuda/model_cuda.cu:46, :1542); n_head must be a multiple of n_head_kv with a
 *    group size of 1 to 8 (every dense Qwen3: 0.6B-8B and 32B have 2, 4 or 8, 14B has 5);
 *    rope_dim even and <= head_dim.
 *  - Shape limits that keep sizes and indices in range (EI_ERR_ARG past them; the workspace
 *    size queries return 0): n_head_kv <= 1024; decode batches of at most 65535 sequences and
 *    2^31 workgroups; prefill chunks of at most 2^20 tokens and 2^28 (token, query head) rows.
 *  - KV cache layout per layer: [position][n_head_kv][head_dim] fp32 (src/model.cpp:153,
 *    src/cuda/model_cuda.cu:1571), i.e. row p holds kd = n_head_kv*128 floats.
 *  - Base pointers and row strides must be 16-byte aligned (multiples of 4 floats).
 */
#ifndef EI_ATTN_H
#define EI_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ei_stream_t; /* hipStream_t */

enum {
    EI_OK = 0,
    EI_ERR_ARG = 1,         /* invalid argument (shape, alignment, null pointer, size) */
    EI_ERR_UNSUPPORTED = 2, /* valid in the reference but not built here (e.g. head_dim != 128) */
    EI_ERR_HIP = 3,         /* a HIP runtime call or kernel launch failed */
    EI_ERR_MERGE = 4        /* a decode workspace's status word reports a failed split-merge check:
                               outputs of the in-kernel merge on it may be wrong */
};

/* Message of the last failure on this thread ("" if none).  Valid until the next call. */
const char* ei_last_error(void);

/* ABI version, bumped on any signature change: a host checks ei_abi_version() == EI_ABI_VERSION. */
#define EI_ABI_VERSION 3
int ei_abi_version(void);

/* ------------------------------------------------------------------ RoPE table
 * Host-side fill of the (cos, sin) table the kernels read: cs[p][i] =
 * (float(cos th), float(sin th)), th = double(p) * theta^(-2i/rope_dim) computed in double,
 * shape [n_ctx][rope_dim/2][2].  Replaces the table build of src/cuda/model_cuda.cu:1610-1619
 * (angles as in src/model.cpp:23-32 and rope_inv_freq, src/model.cpp:105-109).
 * The caller copies it to device memory once. */
int ei_rope_table_fill(float* cs_host, int n_ctx, int rope_dim, double theta);

/* ------------------------------------------------------------------ QKV projection
 * Weight element types of ei_qkv_project: the GGML type ids of F32, F16 and of the block
 * formats the reference decodes (src/quant.h:21-39): Q8_0 (32 values in 34 bytes), Q4_K and
 * Q6_K (256 values in 144 and 210 bytes). */
enum { EI_W_F32 = 0, EI_W_F16 = 1, EI_W_Q8_0 = 8, EI_W_Q4_K = 12, EI_W_Q6_K = 14 };

/* Attention RMSNorm + fused QKV projection of `rows` activation rows (decode: one token per
 * sequence): h = rmsnorm(x_b, attn_norm, eps) (sum of squares in double, as the CPU rmsnorm),
 * then qkv_b[r] = sum_i W[r][i] h[i] for the n_out = (n_head + 2 n_head_kv) * 128 rows of the
 * fused [Wq | Wk | Wv] weight (row r of n_embd elements in the GGUF row layout of w_type:
 * n_embd floats, binary16 values, or n_embd / 32 Q8_0 blocks, n_embd / 256 Q4_K or Q6_K
 * blocks, rows one after another).  Quantised weights are decoded exactly as the CPU path's
 * convert_row (src/quant.cpp:7-60).  A file whose Wq, Wk and Wv have different types takes one
 * call per segment, qkv offset to the segment's first column.
 * Row b of x at x + b*x_stride, of qkv at qkv + b*qkv_stride, left raw: the decode steps
 * (ei_decode_step, ei_decode_step_paged) apply the QK-norm, RoPE and cache append to it.
 * Replaces k_rmsnorm + linear(h, L.qkv, qkv, ...) of src/cuda/model_cuda.cu:1797-1799 (the
 * B == 1 GEMV, :300-320); arithmetic of the CPU path's rmsnorm + matvec (src/ops.cpp:126-160).
 * Built for n_embd 1024, 2048, 2560, 4096, 5120 (every dense Qwen3; F16 also 8192, 10240);
 * 0 <= rows <= min(4, 24576 / n_embd).
 * w must be 16-byte aligned (GGUF aligns tensor data to 32 bytes). */
int ei_qkv_project(ei_stream_t stream, const float* x, long x_stride, int rows, int n_embd, const float* attn_norm,
                   float eps, const void* w, int w_type, int n_out, float* qkv, long qkv_stride);

/* Rows ei_qkv_project takes per launch at this hidden size: min(4, 24576 / n_embd) (the
 * activations of all rows are staged in LDS); 0 for n_embd <= 0.  Callers with more rows split
 * them into launches of at most this many.  No counterpart in the reference, whose GEMV takes
 * any B (src/cuda/model_cuda.cu:300-320). */
int ei_qkv_project_max_rows(int n_embd);

/* ------------------------------------------------------------------ QK-norm + RoPE
 * In place on `rows` rows of `buf` (row b at buf + b*row_stride, head h at + h*128):
 * per head, RMSNorm with gamma (sum of squares in double, inv = float(1/sqrt(ss/128+eps)),
 * out = x*inv*gamma) then NEOX RoPE at position *pos_dev + b from `cs`.
 * Replaces k_headnorm_rope (src/cuda/model_cuda.cu:87-105); arithmetic follows the CPU
 * reference rmsnorm + rope (src/ops.cpp:155-160, src/model.cpp:23-32). */
int ei_headnorm_rope(ei_stream_t stream, float* buf, int rows, long row_stride, int n_heads, int head_dim,
                     const float* gamma, const float* cs, const int* pos_dev, int rope_dim, float eps);

/* ------------------------------------------------------------------ KV append
 * Bit-exact copy of `rows` K and V rows (kd floats each; row b at k_src + b*src_stride)
 * into cache rows *pos_dev + b.  Rows outside [pos, pos+rows) are not touched.
 * Replaces k_store_kv (src/cuda/model_cuda.cu:108-117) / src/model.cpp:186-189. */
int ei_kv_append(ei_stream_t stream, const float* k_src, const float* v_src, long src_stride, int rows, float* kc,
                 float* vc, int kd, const int* pos_dev);

/* ------------------------------------------------------------------ fused prologue
 * One launch for the per-layer prologue of src/cuda/model_cuda.cu:1800-1806 on a
 * [rows][ (H + 2*HKV) * 128 ] QKV buffer ([Q | K | V] per row, row stride `row_stride`):
 * QK-norm + RoPE of the H query heads and the HKV key heads in place (as
 * ei_headnorm_rope), then K and V rows appended to the cache at *pos_dev + b
 * (as ei_kv_append). */
int ei_qkv_prepare(ei_stream_t stream, float* qkv, int rows, long row_stride, int n_head, int n_head_kv,
                   int head_dim, const float* q_gamma, const float* k_gamma, const float* cs, const int* pos_dev,
                   int rope_dim, float eps, float* kc, float* vc);

/* ------------------------------------------------------------------ decode (split-K)
 * Workspace for the decode entry points: per (sequence, kv head, key split) partial
 * (m, l, acc), one arrival counter per (sequence, kv head) for the in-kernel split merge, and a
 * status word.  Its layout follows from its size alone, so calls of different plans (n_seq,
 * max_kv, paged or not) may share it one after another: partials from the start, the counters in
 * the top sixteenth, the status word (uint32) at ws + ((ws_bytes - 256) & ~255), ws_bytes as passed
 * to the calls.  A call whose plan does not fit is rejected (EI_ERR_ARG).  max_kv sizes the split
 * grid (fixed, so a captured graph stays valid as positions advance); a sequence longer than
 * max_kv is still attended in full (its last split takes the excess keys), only more slowly.
 * The workspace must be zero-filled once before its first use, by ei_attn_workspace_init (a
 * fill kernel, not a memset, so it may be captured) or any other zero fill; every decode call
 * leaves the counters at zero again.  Status bit 0 is set, and stays set, if the splits of one
 * (sequence, kv head) were ever found on different XCDs, against the round-robin placement the
 * in-kernel merge relies on (never seen on MI355X; that merge is then unreliable: set
 * EI_DECODE_MERGE=launch for the two-launch combine).  The in-kernel merge is only chosen on a
 * device whose XCD count is one the placement was validated on (8, an MI355X in SPX mode, or 1,
 * one L2); elsewhere every call merges in the second launch.  Calls that share a workspace must
 * not overlap in time. */
size_t ei_attn_decode_ws_bytes(int n_seq, int n_head, int n_head_kv, int max_kv);
int ei_attn_workspace_init(ei_stream_t stream, void* ws, size_t ws_bytes);

/* Reads a decode workspace's status word into *status once the work queued on `stream` has
 * finished (a host synchronisation: not for use under graph capture).  No counterpart in the
 * reference, whose split combine is always a second launch (src/cuda/model_cuda.cu:1097-1111):
 * it is how a caller learns that the in-kernel merge saw a broken placement. */
int ei_attn_workspace_status(ei_stream_t stream, const void* ws, size_t ws_bytes, uint32_t* status);

/* Host-only: EI_OK for a status word of 0, else EI_ERR_MERGE with a message naming the failed
 * check (ei_last_error).  HipAttention and other callers turn a read status word into an error
 * with it. */
int ei_decode_status_check(uint32_t status);

/* Single-sequence decode attention: q [n_head][128] (already normed + roped), cache rows
 * 0..*pos_dev visible (T = *pos_dev + 1 <= max_kv), out [n_head][128].
 * Replaces k_attn_split + k_attn_combine (src/cuda/model_cuda.cu:1043-1111); the math is
 * the CPU reference's softmax attention (src/model.cpp:191-214). */
int ei_attn_decode(ei_stream_t stream, const float* q, float* out, const float* kc, const float* vc,
                   const int* pos_dev, int n_head, int n_head_kv, int head_dim, float scale, int max_kv, void* ws,
                   size_t ws_bytes);

/* Ragged multi-sequence decode: sequence s reads its q at q + s*q_stride ([n_head][128]),
 * attends to cache rows kv_offset[s] .. kv_offset[s]+kv_len[s]-1 (kv_offset and kv_len
 * are device arrays; 0 <= kv_len[s] <= max_kv, a sequence with kv_len 0 gets zeros) and writes
 * out + s*n_head*128.
 * No reference counterpart (the reference decodes one sequence); per sequence the
 * result is that of ei_attn_decode. */
int ei_attn_decode_batched(ei_stream_t stream, const float* q, long q_stride, float* out, const float* kc,
                           const float* vc, const int64_t* kv_offset, const int* kv_len, int n_seq, int n_head,
                           int n_head_kv, int head_dim, float scale, int max_kv, void* ws, size_t ws_bytes);

/* Fused decode step: ei_qkv_prepare + ei_attn_decode for one token per sequence in one
 * decode launch (the splits of chunks over 128 keys merge inside it, shorter ones in a second
 * small launch; rope_dim must be a multiple of 4).  qkv row s (at qkv + s*row_stride, [Q|K|V] raw projections) is read only;
 * the normed+roped K row and the V row are written to cache row kv_offset[s] + pos_s,
 * pos_s = kv_len[s]-1 (or *pos_dev when kv_len is NULL; then n_seq must be 1 and
 * kv_offset may be NULL).  out [n_seq][n_head][128].  Equivalent to the per-layer
 * sequence k_headnorm_rope(Q), k_headnorm_rope(K), k_store_kv, k_attn_split,
 * k_attn_combine of src/cuda/model_cuda.cu:1800-1814. */
int ei_decode_step(ei_stream_t stream, const float* qkv, long row_stride, float* out, float* kc, float* vc,
                   const int64_t* kv_offset, const int* kv_len, const int* pos_dev, int n_seq, int n_head,
                   int n_head_kv, int head_dim, const float* q_gamma, const float* k_gamma, const float* cs,
                   int rope_dim, float eps, float scale, int max_kv, void* ws, size_t ws_bytes);

/* Allocation-free fused decode step.  No counterpart in the reference: it is for callers that
 * cannot allocate or pass a workspace (code under HIP graph capture set up before any
 * workspace exists, tight serving loops, harnesses that forbid allocation).  Same arguments,
 * semantics as ei_decode_step without (ws, ws_bytes); the split partials live in a static
 * device array of 4 MiB per GPU, held until the process ends, so the call allocates nothing.
 * It runs ei_decode_step's plan (chunks of at most 1024 keys) when that plan's partials fit the
 * array, and otherwise the plan without the chunk cap (fewer, longer splits: results within the
 * parity bar, bits may differ from ei_decode_step's); a shape that fits neither is rejected with
 * EI_ERR_ARG.  One sequence at H32/HKV8 takes 0.57 MiB up to max_kv 32768; 64 sequences at
 * H16/HKV8 and max_kv 8192 take 4.8 MiB capped (too much) and 0.56 MiB uncapped; 256 sequences
 * at H32/HKV8 and max_kv 4096 take 4.25 MiB even uncapped (rejected).  Every call on one GPU shares that array:
 * calls that overlap in time on one GPU (two streams, two threads) race and must not be made; a
 * call made while another thread is still inside one on the same GPU is refused (EI_ERR_ARG).
 * The splits are always merged by the second small launch. */
int ei_decode_step_noalloc(ei_stream_t stream, const float* qkv, long row_stride, float* out, float* kc, float* vc,
                           const int64_t* kv_offset, const int* kv_len, const int* pos_dev, int n_seq, int n_head,
                           int n_head_kv, int head_dim, const float* q_gamma, const float* k_gamma, const float* cs,
                           int rope_dim, float eps, float scale, int max_kv);

/* ------------------------------------------------------------------ paged KV (multi-sequence serving)
 * Sequence s's key t lives in cache row block_table[s*max_blocks + t/block_size]*block_size
 * + t%block_size of the shared pool kc/vc (rows of n_head_kv*128 floats); block_size is a
 * power of two >= 16, max_blocks*block_size >= max_kv and < 2^31, 0 <= kv_len[s] (kv_len 0
 * gives zeros; a kv_len above max_kv is still attended in full, one beyond the table's span
 * max_blocks*block_size, outside the contract, is read only up to that span and appends nothing).  Sequences may share physical blocks (a common prefix cached once).  The
 * reference decodes one contiguous sequence (src/cuda/model_cuda.cu:1043-1111); these are
 * the serve-side extension of ei_attn_decode_batched and ei_decode_step: per sequence the
 * result is that of ei_attn_decode on the gathered rows.  ei_decode_step_paged writes the
 * new K/V row of sequence s (logical position kv_len[s]-1) to its physical row, so that
 * row's block must be private to the sequence. */
int ei_attn_decode_paged(ei_stream_t stream, const float* q, long q_stride, float* out, const float* kc,
                         const float* vc, const int* block_table, int max_blocks, int block_size, const int* kv_len,
                         int n_seq, int n_head, int n_head_kv, int head_dim, float scale, int max_kv, void* ws,
                         size_t ws_bytes);
int ei_decode_step_paged(ei_stream_t stream, const float* qkv, long row_stride, float* out, float* kc, float* vc,
                         const int* block_table, int max_blocks, int block_size, const int* kv_len, int n_seq,
                         int n_head, int n_head_kv, int head_dim, const float* q_gamma, const float* k_gamma,
                         const float* cs, int rope_dim, float eps, float scale, int max_kv, void* ws, size_t ws_bytes);

/* ------------------------------------------------------------------ causal prefill
 * B query rows (row b at q + b*q_stride, heads [n_head][128], already normed + roped) at
 * positions *pos_dev + b; query b attends to cache rows 0 .. *pos_dev + b (the whole
 * chunk's K/V must already be appended).  out [B][n_head][128].  fp32 MFMA contraction
 * with online softmax.  Replaces k_attn_prefill64 (src/cuda/model_cuda.cu:1204-1341);
 * the math is the CPU reference's per-token attention (src/model.cpp:138-140, :191-214). */
int ei_attn_prefill(ei_stream_t stream, const float* q, long q_stride, float* out, const float* kc, const float* vc,
                    const int* pos_dev, int B, int n_head, int n_head_kv, int head_dim, float scale);

/* Key-split prefill for short chunks at long positions.  The reference engine feeds a prompt
 * in chunks of at most 512 tokens (src/cuda/model_cuda.cu:1912) and runs one
 * k_attn_prefill64 per chunk; at 512 tokens (or with GQA groups under 4 heads at any
 * length) one workgroup per query-block pair and KV head leaves CUs idle.  This variant
 * splits every query block's key range over up to 8 workgroups, as many as fill whole
 * rounds of the CUs (planned from B and max_kv, an upper bound of *pos_dev + B) and merges the
 * shares with a second launch, using `ws`: ei_attn_prefill_ws_bytes(max_B, ...) bytes serve
 * every chunk of up to max_B rows (0 bytes when no split is planned; the call then equals
 * ei_attn_prefill).  Same semantics and arguments as ei_attn_prefill otherwise; no
 * counterpart in the reference beyond k_attn_prefill64.  Calls sharing `ws` must not overlap. */
size_t ei_attn_prefill_ws_bytes(int max_B, int n_head, int n_head_kv, int max_kv);
int ei_attn_prefill_split(ei_stream_t stream, const float* q, long q_stride, float* out, const float* kc,
                          const float* vc, const int* pos_dev, int B, int n_head, int n_head_kv, int head_dim,
                          float scale, int max_kv, void* ws, size_t ws_bytes);

/* Fused prefill step for a chunk of B tokens at positions *pos_dev .. *pos_dev+B-1: the
 * per-layer sequence k_headnorm_rope(Q), k_headnorm_rope(K), k_store_kv, k_attn_prefill64 of
 * src/cuda/model_cuda.cu:1800-1820 in two launches (plus the key-split merge when planned).
 * qkv rows [Q|K|V] are raw projections: the K heads are normed + roped in place and appended
 * with the V rows to cache rows *pos_dev + b (as ei_qkv_prepare does).  With rope_dim = 128
 * (every Qwen3) and a plan of at most four key shares, the Q heads are left raw in qkv and
 * normed + roped inside the attention kernel where it stages them; otherwise (a partial
 * rope_dim, or a plan of more shares) they are normed in
 * place by the prologue first.  Same workspace and plan as ei_attn_prefill_split;
 * out [B][n_head][128]. */
int ei_prefill_step(ei_stream_t stream, float* qkv, long row_stride, float* out, float* kc, float* vc,
                    const int* pos_dev, int B, int n_head, int n_head_kv, int head_dim, const float* q_gamma,
                    const float* k_gamma, const float* cs, int rope_dim, float eps, float scale, int max_kv, void* ws,
                    size_t ws_bytes);

/* ei_prefill_step over a paged pool: key t of the sequence (its cache row before) is pool row
 * block_table[t / block_size] * block_size + t % block_size, for the K and V pools kc and vc
 * (rows of n_head_kv * 128 floats).  block_table is a device array of max_blocks int32 entries
 * covering max_kv keys; block_size a power of two >= 32 (a 32-key prefill tile never straddles
 * blocks).  The chunk's K/V rows are appended at the pool rows of positions *pos_dev ..
 * *pos_dev + B - 1 (those blocks must be private to the sequence); blocks before may be shared
 * with other sequences (a cached common prefix).  Results are bit-identical to ei_prefill_step on
 * the same keys held contiguously.  No counterpart in the reference, which keeps one contiguous
 * cache per sequence (src/cuda/model_cuda.cu:1571); it extends the paged decode
 * (ei_decode_step_paged) to prompt chunks. */
int ei_prefill_step_paged(ei_stream_t stream, float* qkv, long row_stride, float* out, float* kc, float* vc,
                          const int* block_table, int max_blocks, int block_size, const int* pos_dev, int B,
                          int n_head, int n_head_kv, int head_dim, const float* q_gamma, const float* k_gamma,
                          const float* cs, int rope_dim, float eps, float scale, int max_kv, void* ws,
                          size_t ws_bytes);

/* ------------------------------------------------------------------ measurement
 * Not part of the reference path: the memory traffic of ei_attn_decode's plan for one sequence
 * of kv_len keys with no arithmetic (same grid, LDS-DMA instructions, tile order and cache
 * policy; each workgroup writes one float of what it read to sink, which must hold
 * n_head_kv * 256 floats).  Its duration is the floor of a decode launch of that plan. */
int ei_stream_ceiling(ei_stream_t stream, const float* kc, const float* vc, int n_head_kv, int kv_len, float* sink);

/* Not part of the reference path: a plain streaming read of `bytes` (a multiple of 16, src
 * 16-byte aligned) with non-temporal 16-byte global loads by n_workgroups workgroups of 256
 * threads (1..65535, at most 64 loads per thread: bytes <= n_workgroups * 256 KiB; sink holds
 * n_workgroups * 16 bytes and is written only by chance).  all_in_flight != 0 issues every load of
 * a thread before any is used; 0 lets the compiler interleave loads and uses (fewer registers,
 * more waves).  Its duration bounds any kernel that reads that many bytes per launch: the read
 * ceiling a decode launch of the same bytes is measured against. */
int ei_read_ceiling(ei_stream_t stream, const void* src, size_t bytes, int n_workgroups, int all_in_flight,
                    void* sink);

/* ------------------------------------------------------------------ synthetic inputs
 * Not part of the reference path: fills n floats with the counter-based N(0,1)
 * generator (element e = stream element offset+e of `seed`), multiplying by spike_mult
 * every element whose row index ((offset+e) / row_len) is a multiple of spike_every
 * (spike_every <= 0: no spikes).  Bit-identical to the CPU generator used by the tests. */
int ei_synth_fill(ei_stream_t stream, float* dst, size_t n, uint64_t seed, uint64_t offset, long row_len,
                  long spike_every, float spike_mult);

#ifdef __cplusplus
}
#endif

#endif /* EI_ATTN_H */
