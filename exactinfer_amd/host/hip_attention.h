// hip_attention.h — engine-side C++ interface of the gfx950 attention path.
//
// The reference engine keeps attention inside its backends: CpuModel::forward
// (src/model.cpp:171-214) and CudaModel::body (src/cuda/model_cuda.cu:1797-1822), behind
// `class Backend` (src/model.h:42-51).  HipAttention is the attention part of such a backend
// for one MI355X: it owns what CudaModel's constructor allocates for attention (the fp32 KV
// cache of every layer, the RoPE table, the split-K workspace and the device-resident
// position; src/cuda/model_cuda.cu:1571, :1610-1631) and runs the per-layer attention sub-step
// in the reference's order (QK-norm + RoPE of Q and K, KV append, attention) through the C ABI
// of include/ei_attn.h.  Errors are thrown as std::runtime_error / std::out_of_range, the
// reference engine's convention (src/cuda/model_cuda.cu:40-44, :1649-1652).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#define EI_ENGINE_API __attribute__((visibility("default")))

namespace ei {

// The el::Config fields the attention path reads (src/model.h:17-23).
struct AttnConfig {
    int n_layer = 0;
    int n_head = 0;
    int n_head_kv = 0;
    int head_dim = 128;
    int rope_dim = 128;
    double rope_base = 1e6;
    float eps = 1e-6f;
};

class EI_ENGINE_API HipAttention {
public:
    // n_ctx: KV capacity per layer; max_batch: largest chunk passed to begin_chunk
    // (the reference chunks prompts by 512, src/cuda/model_cuda.cu:1653-1657, :1912).
    HipAttention(const AttnConfig& cfg, int n_ctx, int max_batch, hipStream_t stream);
    ~HipAttention();
    HipAttention(const HipAttention&) = delete;
    HipAttention& operator=(const HipAttention&) = delete;

    const AttnConfig& cfg() const { return c_; }
    int n_ctx() const { return n_ctx_; }
    hipStream_t stream() const { return stream_; }

    // Start a chunk of B tokens at positions pos0..pos0+B-1 (bounds-checked like
    // CudaModel::eval, src/cuda/model_cuda.cu:1649-1652); uploads pos0 to the device-resident
    // position read by every kernel (src/cuda/model_cuda.cu:1845-1846).
    void begin_chunk(int pos0, int B);

    // One layer's attention sub-step for the current chunk (src/cuda/model_cuda.cu:1797-1822):
    //   qkv [B][(H + 2*HKV)*128] raw projections, row stride qkv_stride floats;
    //   q_norm / k_norm: the layer's attn_q_norm / attn_k_norm weights [128] (device);
    //   att [B][H*128] output (device).
    // B == 1 runs the fused decode step (qkv is read only); B > 1 runs the fused prefill step:
    // K normalised in place and appended with V, causal fp32-MFMA prefill with Q normalised
    // inside the kernel (key range split over workgroups when the chunk alone would not fill
    // the GPU).
    void layer(int l, float* qkv, long qkv_stride, const float* q_norm, const float* k_norm, float* att);

    // Attention RMSNorm + QKV projection of the current chunk's B rows, the step before layer()
    // (k_rmsnorm + linear(h, L.qkv, ...), src/cuda/model_cuda.cu:1797-1799; the CPU path's
    // rmsnorm + matvec, src/model.cpp:176-179):
    //   x [B][n_embd] residual rows (row stride x_stride), attn_norm [n_embd] (device);
    //   w: n_out rows of n_embd weights in the GGUF row layout of w_type (EI_W_F32, EI_W_F16,
    //   EI_W_Q8_0, EI_W_Q4_K, EI_W_Q6_K); the fused [Wq | Wk | Wv] with n_out = (H + 2 HKV) * 128,
    //   or one segment of it (qkv then points at the segment's first column);
    //   qkv [B][...] output rows (row stride qkv_stride), left raw for layer().
    // Runs ei_qkv_project over groups of rows (at most ei_qkv_project_max_rows(n_embd) per launch).
    void project(const float* x, long x_stride, int n_embd, const float* attn_norm, const void* w, int w_type,
                 int n_out, float* qkv, long qkv_stride);

    // Waits for the queued work and throws std::runtime_error if the decode workspace's status
    // word reports a failed split-merge check (attention outputs may then be wrong).  begin_chunk
    // does the same check at its own synchronisation, so an engine that starts every chunk or
    // token with begin_chunk learns of a failure no later than the next token.
    void check_status();
    // Throws std::runtime_error for a non-zero status word (ei_decode_status_check's message).
    static void raise_on_status(uint32_t status);

    // Device views of layer l's cache, [n_ctx][n_head_kv][128] fp32.
    float* kcache(int l) const;
    float* vcache(int l) const;

private:
    void check(int status) const;
    void allocate();
    void release() noexcept;

    AttnConfig c_;
    int n_ctx_, max_batch_;
    hipStream_t stream_;
    int B_ = 0;
    float* kv_ = nullptr;    // K caches of all layers, then V caches
    float* rope_ = nullptr;  // [n_ctx][rope_dim/2][2]
    void* ws_ = nullptr;  // decode split partials
    size_t ws_bytes_ = 0;
    void* pws_ = nullptr;  // prefill key-split shares (chunks of up to max_batch rows)
    size_t pws_bytes_ = 0;
    int* pos_dev_ = nullptr;
    int* pos_host_ = nullptr;  // pinned
    uint32_t* status_host_ = nullptr;  // pinned copy of the decode workspace's status word
    float scale_;
};

}  // namespace ei
