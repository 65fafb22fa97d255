// prologue.hip — per-layer attention prologue on gfx950: per-head QK-norm + RoPE, KV-cache
// append, the fused [Q|K|V] prepare, and the synthetic-input fill.
//
// All of these are HBM-bound byte movers (a few hundred bytes per head); one wave handles
// one 128-float head (lane l owns elements l and l+64), 4 waves per workgroup.
#include "common.h"
#include "launch.h"

namespace ei {

// grid (rows, ceil(n_heads/4)), block 256.  In place; src/cuda/model_cuda.cu:87-105.
__global__ __launch_bounds__(256) void k_headnorm_rope(float* __restrict__ buf, long row_stride, int n_heads,
                                                       const float* __restrict__ gamma,
                                                       const float2* __restrict__ cs, const int* __restrict__ pos_dev,
                                                       int rope_dim, float eps) {
    __shared__ float scratch[4][kHeadDim];
    const int b = blockIdx.x, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = blockIdx.y * 4 + w;
    if (h >= n_heads) return;  // wave-uniform; this kernel has no block barrier
    float* v = buf + (size_t)b * row_stride + (size_t)h * kHeadDim;
    const int pos = *pos_dev + b;
    float o0, o1;
    norm_rope_head(v, gamma, cs + (size_t)pos * (rope_dim >> 1), rope_dim, eps, scratch[w], lane, &o0, &o1);
    v[lane] = o0;
    v[lane + 64] = o1;
}

// grid rows, block 256: bit-exact float4 copies of one K row and one V row (kd floats).
// src/cuda/model_cuda.cu:108-117.
__global__ __launch_bounds__(256) void k_kv_append(const float* __restrict__ k_src, const float* __restrict__ v_src,
                                                   long src_stride, float* __restrict__ kc, float* __restrict__ vc,
                                                   int kd, const int* __restrict__ pos_dev) {
    const int b = blockIdx.x;
    const size_t dst = (size_t)(*pos_dev + b) * kd;
    const float* ks = k_src + (size_t)b * src_stride;
    const float* vs = v_src + (size_t)b * src_stride;
    for (int i = threadIdx.x * 4; i < kd; i += 1024) {
        *reinterpret_cast<float4*>(kc + dst + i) = *reinterpret_cast<const float4*>(ks + i);
        *reinterpret_cast<float4*>(vc + dst + i) = *reinterpret_cast<const float4*>(vs + i);
    }
}

// grid (rows, ceil((H+HKV)/16)), block 256: each wave takes 4 consecutive heads of the
// row (2 KB) and issues all their loads (and the V rows of its key heads) before any
// arithmetic, so a wave keeps 8-16 loads in flight.  Head index hh < H: query head
// (q_gamma); otherwise key head hh-H (k_gamma), whose normed row also goes to the cache
// together with the raw V row of the same kv head.  Heads below h_begin are skipped (h_begin = H:
// the keys and the append only, when the prefill normalises q itself).  src/cuda/model_cuda.cu:1800-1806.
template <int kPrepHeads>  // heads per wave: 4 for all heads, 2 for the key heads alone (every wave busy)
__global__ __launch_bounds__(256) void k_qkv_prepare(float* __restrict__ qkv, long row_stride, int H, int HKV,
                                                     const float* __restrict__ q_gamma,
                                                     const float* __restrict__ k_gamma,
                                                     const float2* __restrict__ cs, const int* __restrict__ pos_dev,
                                                     int rope_dim, float eps, float* __restrict__ kc,
                                                     float* __restrict__ vc, int h_begin,
                                                     const int* __restrict__ btab, int bshift, int max_blocks) {
    __shared__ float scratch[4][kHeadDim];
    const int b = blockIdx.x, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int NH = H + HKV;
    const int h0 = h_begin + (blockIdx.y * 4 + w) * kPrepHeads;
    if (h0 >= NH) return;  // wave-uniform; this kernel has no block barrier
    float* row = qkv + (size_t)b * row_stride;
    const int pos = *pos_dev + b;
    const float2* cs_row = cs + (size_t)pos * (rope_dim >> 1);
    float x0[kPrepHeads], x1[kPrepHeads], v0[kPrepHeads], v1[kPrepHeads];
#pragma unroll
    for (int j = 0; j < kPrepHeads; ++j) {
        const int hh = min(h0 + j, NH - 1);  // clamped: heads past NH are loaded, not used
        const float* v = row + (size_t)hh * kHeadDim;
        x0[j] = v[lane];
        x1[j] = v[lane + 64];
        const float* vs = row + (size_t)(H + HKV + max(hh - H, 0)) * kHeadDim;  // V of a key head
        v0[j] = vs[lane];
        v1[j] = vs[lane + 64];
    }
    const float qg0 = q_gamma[lane], qg1 = q_gamma[lane + 64];
    const float kg0 = k_gamma[lane], kg1 = k_gamma[lane + 64];
    const size_t kd = (size_t)HKV * kHeadDim;
    float inv[kPrepHeads];  // the wave's heads normalised together (one double 1/sqrt)
    head_inv<kPrepHeads>(x0, x1, eps, inv, lane);
#pragma unroll
    for (int j = 0; j < kPrepHeads; ++j) {
        const int hh = h0 + j;
        if (hh >= NH) break;
        const bool is_k = hh >= H;
        float o0, o1;
        scale_rope_vals(x0[j], x1[j], inv[j], is_k ? kg0 : qg0, is_k ? kg1 : qg1, cs_row, rope_dim, scratch[w], lane,
                        &o0, &o1);
        float* v = row + (size_t)hh * kHeadDim;
        v[lane] = o0;
        v[lane + 64] = o1;
        // (paged: a position past the table's blocks, outside the contract, appends nothing)
        if (is_k && (!btab || (pos >> bshift) < max_blocks)) {
            const int kvh = hh - H;
            // cache row of the position: itself, or through the block table of a paged pool
            const size_t crow = btab ? ((size_t)btab[pos >> bshift] << bshift) | (size_t)(pos & ((1 << bshift) - 1))
                                     : (size_t)pos;
            float* kd_row = kc + crow * kd + (size_t)kvh * kHeadDim;
            float* vd_row = vc + crow * kd + (size_t)kvh * kHeadDim;
            kd_row[lane] = o0;
            kd_row[lane + 64] = o1;
            vd_row[lane] = v0[j];
            vd_row[lane + 64] = v1[j];
        }
    }
}

// grid-stride fill with the counter-based generator.
__global__ __launch_bounds__(256) void k_synth_fill(float* __restrict__ dst, size_t n, uint64_t seed, uint64_t offset,
                                                    long row_len, long spike_every, float spike_mult) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t e = offset + i;
        float v = synth_normal(seed, e);
        if (spike_every > 0 && ((e / (uint64_t)row_len) % (uint64_t)spike_every) == 0) v = v * spike_mult;
        dst[i] = v;
    }
}

// ------------------------------------------------------------------ launchers
hipError_t launch_headnorm_rope(hipStream_t st, float* buf, int rows, long row_stride, int n_heads,
                                const float* gamma, const float* cs, const int* pos_dev, int rope_dim, float eps) {
    k_headnorm_rope<<<dim3(rows, (n_heads + 3) / 4), 256, 0, st>>>(
        buf, row_stride, n_heads, gamma, reinterpret_cast<const float2*>(cs), pos_dev, rope_dim, eps);
    return hipGetLastError();
}

hipError_t launch_kv_append(hipStream_t st, const float* k_src, const float* v_src, long src_stride, int rows,
                            float* kc, float* vc, int kd, const int* pos_dev) {
    k_kv_append<<<rows, 256, 0, st>>>(k_src, v_src, src_stride, kc, vc, kd, pos_dev);
    return hipGetLastError();
}

hipError_t launch_qkv_prepare(hipStream_t st, float* qkv, int rows, long row_stride, int H, int HKV,
                              const float* q_gamma, const float* k_gamma, const float* cs, const int* pos_dev,
                              int rope_dim, float eps, float* kc, float* vc, int h_begin, const int* block_table,
                              int block_shift, int max_blocks) {
    const int nh = H + HKV - h_begin;
    const float2* cs2 = reinterpret_cast<const float2*>(cs);
    if (nh <= 8) {  // 4 waves x 2 heads
        k_qkv_prepare<2><<<dim3(rows, (nh + 7) / 8), 256, 0, st>>>(qkv, row_stride, H, HKV, q_gamma, k_gamma, cs2,
                                                                     pos_dev, rope_dim, eps, kc, vc, h_begin,
                                                                     block_table, block_shift, max_blocks);
    } else {  // 4 waves x 4 heads
        k_qkv_prepare<4><<<dim3(rows, (nh + 15) / 16), 256, 0, st>>>(qkv, row_stride, H, HKV, q_gamma, k_gamma, cs2,
                                                                       pos_dev, rope_dim, eps, kc, vc, h_begin,
                                                                     block_table, block_shift, max_blocks);
    }
    return hipGetLastError();
}

hipError_t launch_synth_fill(hipStream_t st, float* dst, size_t n, uint64_t seed, uint64_t offset, long row_len,
                             long spike_every, float spike_mult) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) return hipSuccess;
    k_synth_fill<<<(unsigned)blocks, 256, 0, st>>>(dst, n, seed, offset, row_len, spike_every, spike_mult);
    return hipGetLastError();
}

}  // namespace ei
