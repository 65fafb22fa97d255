// hip_attention.cpp — HipAttention: the attention part of a HIP backend (see the header).
#include "hip_attention.h"

#include <cmath>
#include <stdexcept>
#include <string>

#include "../../include/ei_attn.h"

namespace ei {

namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string("HIP error (") + what + "): " + hipGetErrorString(e));
}

}  // namespace

void HipAttention::check(int status) const {
    if (status != EI_OK) throw std::runtime_error(std::string("attention kernel call failed: ") + ei_last_error());
}

HipAttention::HipAttention(const AttnConfig& cfg, int n_ctx, int max_batch, hipStream_t stream)
    : c_(cfg), n_ctx_(n_ctx), max_batch_(max_batch), stream_(stream) {
    if (n_ctx_ <= 0) throw std::runtime_error("n_ctx must be positive");
    if (max_batch_ <= 0) throw std::runtime_error("max_batch must be positive");
    if (c_.n_layer <= 0 || c_.n_head <= 0 || c_.n_head_kv <= 0 || c_.n_head % c_.n_head_kv)
        throw std::runtime_error("invalid attention configuration");
    if (c_.head_dim != 128) throw std::runtime_error("the HIP path supports head_dim = 128 only");
    // scale as the reference computes it (src/model.cpp:163, src/cuda/model_cuda.cu:1786)
    scale_ = 1.0f / std::sqrt(float(c_.head_dim));

    try {
        allocate();
    } catch (...) {
        release();  // the destructor does not run for a constructor that throws
        throw;
    }
}

void HipAttention::allocate() {
    const size_t kd = size_t(c_.n_head_kv) * c_.head_dim;
    const size_t per_cache = size_t(c_.n_layer) * size_t(n_ctx_) * kd * sizeof(float);
    hip_check(hipMalloc(&kv_, 2 * per_cache), "KV cache");
    hip_check(hipMemsetAsync(kv_, 0, 2 * per_cache, stream_), "KV cache clear");

    std::vector<float> cs(size_t(n_ctx_) * size_t(c_.rope_dim));
    check(ei_rope_table_fill(cs.data(), n_ctx_, c_.rope_dim, c_.rope_base));
    hip_check(hipMalloc(&rope_, cs.size() * sizeof(float)), "RoPE table");
    hip_check(hipMemcpy(rope_, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice), "RoPE upload");

    ws_bytes_ = ei_attn_decode_ws_bytes(1, c_.n_head, c_.n_head_kv, n_ctx_);
    if (ws_bytes_ == 0) throw std::runtime_error("decode workspace size");
    hip_check(hipMalloc(&ws_, ws_bytes_), "decode workspace");
    check(ei_attn_workspace_init(stream_, ws_, ws_bytes_));

    pws_bytes_ = ei_attn_prefill_ws_bytes(max_batch_ < n_ctx_ ? max_batch_ : n_ctx_, c_.n_head, c_.n_head_kv, n_ctx_);
    if (pws_bytes_) hip_check(hipMalloc(&pws_, pws_bytes_), "prefill workspace");

    hip_check(hipMalloc(&pos_dev_, sizeof(int)), "position");
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&pos_host_), sizeof(int), hipHostMallocDefault), "pinned position");
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&status_host_), sizeof(uint32_t), hipHostMallocDefault),
              "pinned status");
    hip_check(hipStreamSynchronize(stream_), "init");
}

HipAttention::~HipAttention() { release(); }

void HipAttention::release() noexcept {
    if (stream_) (void)hipStreamSynchronize(stream_);
    if (pos_host_) (void)hipHostFree(pos_host_);
    if (status_host_) (void)hipHostFree(status_host_);
    if (pos_dev_) (void)hipFree(pos_dev_);
    if (ws_) (void)hipFree(ws_);
    if (pws_) (void)hipFree(pws_);
    if (rope_) (void)hipFree(rope_);
    if (kv_) (void)hipFree(kv_);
    pos_host_ = nullptr;
    status_host_ = nullptr;
    pos_dev_ = nullptr;
    ws_ = pws_ = nullptr;
    rope_ = kv_ = nullptr;
}

void HipAttention::begin_chunk(int pos0, int B) {
    if (B <= 0) throw std::invalid_argument("empty chunk");
    if (B > max_batch_) throw std::invalid_argument("chunk larger than max_batch");
    if (pos0 < 0 || pos0 + B > n_ctx_) throw std::out_of_range("context window full");
    // the pinned host word is reused: wait until the previous chunk's upload has been consumed;
    // the wait also brings the decode workspace's status word, checked here
    check_status();
    *pos_host_ = pos0;
    hip_check(hipMemcpyAsync(pos_dev_, pos_host_, sizeof(int), hipMemcpyHostToDevice, stream_), "position upload");
    B_ = B;
}

void HipAttention::raise_on_status(uint32_t status) {
    if (ei_decode_status_check(status) != EI_OK) throw std::runtime_error(ei_last_error());
}

void HipAttention::check_status() {
    // the status word sits where the workspace's size puts it (include/ei_attn.h)
    const char* word = static_cast<const char*>(ws_) + ((ws_bytes_ - 256) & ~size_t(255));
    hip_check(hipMemcpyAsync(status_host_, word, sizeof(uint32_t), hipMemcpyDeviceToHost, stream_), "status read");
    hip_check(hipStreamSynchronize(stream_), "chunk sync");
    raise_on_status(*status_host_);
}

float* HipAttention::kcache(int l) const {
    const size_t kd = size_t(c_.n_head_kv) * c_.head_dim;
    return kv_ + size_t(l) * size_t(n_ctx_) * kd;
}

float* HipAttention::vcache(int l) const {
    const size_t kd = size_t(c_.n_head_kv) * c_.head_dim;
    return kv_ + (size_t(c_.n_layer) + size_t(l)) * size_t(n_ctx_) * kd;
}

void HipAttention::project(const float* x, long x_stride, int n_embd, const float* attn_norm, const void* w,
                           int w_type, int n_out, float* qkv, long qkv_stride) {
    if (B_ <= 0) throw std::logic_error("project() before begin_chunk()");
    if (n_embd <= 0) throw std::invalid_argument("n_embd");
    const int per = ei_qkv_project_max_rows(n_embd);  // rows per launch (staged in LDS)
    if (per < 1) throw std::invalid_argument("n_embd too large for the projection");
    for (int b = 0; b < B_; b += per) {
        const int rows = B_ - b < per ? B_ - b : per;
        check(ei_qkv_project(stream_, x + size_t(b) * x_stride, x_stride, rows, n_embd, attn_norm, c_.eps, w, w_type,
                             n_out, qkv + size_t(b) * qkv_stride, qkv_stride));
    }
}

void HipAttention::layer(int l, float* qkv, long qkv_stride, const float* q_norm, const float* k_norm, float* att) {
    if (l < 0 || l >= c_.n_layer) throw std::out_of_range("layer index");
    if (B_ <= 0) throw std::logic_error("layer() before begin_chunk()");
    const int H = c_.n_head, HKV = c_.n_head_kv, D = c_.head_dim;
    if (B_ == 1) {
        // decode: one fused launch (+ split merge), cache row *pos written in place
        check(ei_decode_step(stream_, qkv, qkv_stride, att, kcache(l), vcache(l), nullptr, nullptr, pos_dev_, 1, H,
                             HKV, D, q_norm, k_norm, rope_, c_.rope_dim, c_.eps, scale_, n_ctx_, ws_, ws_bytes_));
    } else {
        // prompt chunk: QK-norm + RoPE + append of the K rows, then causal attention over cache
        // rows 0..pos0+b (earlier chunks included) with q normed inside the attention kernel
        check(ei_prefill_step(stream_, qkv, qkv_stride, att, kcache(l), vcache(l), pos_dev_, B_, H, HKV, D, q_norm,
                              k_norm, rope_, c_.rope_dim, c_.eps, scale_, n_ctx_, pws_, pws_bytes_));
    }
}

}  // namespace ei
