// project.hip — the QKV projection of a decode step on gfx950: attention RMSNorm of the
// residual rows and the fused [Wq | Wk | Wv] product, one HBM-streaming launch.
//
// Reference: CudaModel::body runs k_rmsnorm (x -> h) and linear(h, L.qkv, qkv, B, QKV, E), a
// GEMV per weight segment for B == 1 (src/cuda/model_cuda.cu:1797-1799, GEMV :300-320); the CPU
// path runs rmsnorm then matvec with wq, wk, wv (src/model.cpp:176-179, src/ops.cpp:126-160).
// The rows come out raw, in the [Q | K | V] layout the decode step reads: the per-head QK-norm,
// RoPE and the cache append that the reference launches next (three more kernels) are the
// epilogue that ei_decode_step / ei_decode_step_paged apply inside the attention launch.
//
// A decode step's projection is bound by the weight stream (E x (H + 2 HKV) x 128 weights read
// once per token: 63 MB in fp32, 31 MB in fp16 at Qwen3-4B), so the kernel is a streaming
// GEMV: wave w of a workgroup owns kRowsPerWave consecutive output rows; lane l reads 16-byte
// pieces l, l + 64, ... of each row (whole 1 KB per instruction, non-temporal: read once),
// issues every piece of its rows before any arithmetic, and only then stages the normed
// activations: the x rows are read (L2-resident after the first workgroups), their sum of
// squares is taken in double as the CPU rmsnorm does, and h = (x * inv) * gamma goes to LDS,
// read back as broadcast 16-byte pieces.  Dot products accumulate per lane with FMAs and end
// in a wave butterfly; up to kMaxRows activation rows share each weight load.
#include <hip/hip_fp16.h>

#include "common.h"
#include "launch.h"

namespace ei {

constexpr int kProjWaves = 4;
constexpr int kRowsPerWave = 2;
constexpr int kProjMaxLdsFloats = 24576;  // B * E activations staged in LDS (96 KB)

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void f16x8(const u32x4_t u, float* f) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const __half2 h = *reinterpret_cast<const __half2*>(&w[i]);
        f[2 * i] = __low2float(h);
        f[2 * i + 1] = __high2float(h);
    }
}

// WF16: weights are binary16; NB activation rows (B <= NB); P 16-byte pieces per lane per row,
// E = 64 * P * (4 fp32 or 8 fp16 weights per piece), fixed at compile time so the weights stay
// in registers
template <bool WF16, int NB, int P>
__global__ __launch_bounds__(64 * kProjWaves) void k_qkv_project(const float* __restrict__ x, long x_stride, int B,
                                                                 int E, const float* __restrict__ gamma, float eps,
                                                                 const void* __restrict__ w, int n_out,
                                                                 float* __restrict__ out, long out_stride) {
    constexpr int kPer = WF16 ? 8 : 4;  // weights per 16-byte piece
    extern __shared__ __align__(16) float hs[];  // [NB][E] normed activations
    __shared__ double ssum[kProjWaves][NB];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r0 = (blockIdx.x * kProjWaves + wv) * kRowsPerWave;

    // ---- this thread's activation and gamma elements first (L2-resident after the first
    // workgroups), then every weight piece of the wave's rows: loads return in order, so the
    // norm below waits for the activations only and overlaps the weight stream
    constexpr int kEl = 64 * P * kPer / (64 * kProjWaves);  // elements per thread per row
    float xv[NB][kEl], gv[kEl];
#pragma unroll
    for (int i = 0; i < kEl; ++i) gv[i] = gamma[tid + i * 64 * kProjWaves];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < kEl; ++i) xv[b][i] = b < B ? x[(size_t)b * x_stride + tid + i * 64 * kProjWaves] : 0.f;
    u32x4_t wr[kRowsPerWave][P];
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const int r = min(r0 + rr, n_out - 1);
        const char* row = static_cast<const char*>(w) + (size_t)r * E * (WF16 ? 2 : 4);
#pragma unroll
        for (int p = 0; p < P; ++p)
            wr[rr][p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(row) + p * 64 + lane);
    }

    // ---- attention RMSNorm of the B rows into LDS (src/ops.cpp:155-160: sum of squares in
    // double, inv = float(1 / sqrt(ss / E + eps)), h = (x * inv) * gamma)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < kEl; ++i) ss += (double)xv[b][i] * (double)xv[b][i];
        ss = wave_sum_f64(ss);
        if (lane == 0) ssum[wv][b] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (b >= B) break;
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < kProjWaves; ++k) ss += ssum[k][b];
        const float inv = (float)(1.0 / sqrt(ss / (double)E + (double)eps));
#pragma unroll
        for (int i = 0; i < kEl; ++i) {
#pragma clang fp contract(off)
            hs[b * E + tid + i * 64 * kProjWaves] = (xv[b][i] * inv) * gv[i];
        }
    }
    __syncthreads();

    // ---- dot products: lane l covers pieces p*64 + l of each row
    float acc[kRowsPerWave][NB];
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[rr][b] = 0.f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int e0 = (p * 64 + lane) * kPer;
#pragma unroll
        for (int rr = 0; rr < kRowsPerWave; ++rr) {
            float wf[kPer];
            if constexpr (WF16) {
                f16x8(wr[rr][p], wf);
            } else {
                wf[0] = __uint_as_float(wr[rr][p].x);
                wf[1] = __uint_as_float(wr[rr][p].y);
                wf[2] = __uint_as_float(wr[rr][p].z);
                wf[3] = __uint_as_float(wr[rr][p].w);
            }
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b >= B) break;
#pragma unroll
                for (int k = 0; k < kPer; k += 4) {
                    const float4 h4 = *reinterpret_cast<const float4*>(hs + b * E + e0 + k);
                    acc[rr][b] = fmaf(wf[k], h4.x, acc[rr][b]);
                    acc[rr][b] = fmaf(wf[k + 1], h4.y, acc[rr][b]);
                    acc[rr][b] = fmaf(wf[k + 2], h4.z, acc[rr][b]);
                    acc[rr][b] = fmaf(wf[k + 3], h4.w, acc[rr][b]);
                }
            }
        }
    }
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b >= B) break;
            const float s = wave_sum(acc[rr][b]);
            if (lane == 0 && r0 + rr < n_out) out[(size_t)b * out_stride + r0 + rr] = s;
        }
}

int qkv_project_max_rows(int E) {
    const int r = E > 0 ? kProjMaxLdsFloats / E : 0;
    return r < kProjMaxRows ? r : kProjMaxRows;
}

// 16-byte pieces per lane per row for the supported hidden sizes (0: not built)
int qkv_project_pieces(int E, bool w_f16) {
    const int per = 64 * (w_f16 ? 8 : 4);
    if (E <= 0 || E % per) return 0;
    const int p = E / per;
    if (w_f16) return (p == 2 || p == 4 || p == 5 || p == 8 || p == 10 || p == 16 || p == 20) ? p : 0;
    return (p == 4 || p == 8 || p == 10 || p == 16 || p == 20) ? p : 0;
}

template <bool WF16, int NB, int P>
static hipError_t launch_nbp(hipStream_t st, const float* x, long x_stride, int B, int E, const float* gamma,
                             float eps, const void* w, int n_out, float* out, long out_stride) {
    const size_t lds = (size_t)B * E * sizeof(float);
    static std::atomic<bool> opted;
    if (const hipError_t e = opt_in_lds(opted, (const void*)k_qkv_project<WF16, NB, P>, kProjMaxLdsFloats * 4);
        e != hipSuccess)
        return e;
    const int per_block = kProjWaves * kRowsPerWave;
    k_qkv_project<WF16, NB, P><<<(n_out + per_block - 1) / per_block, 64 * kProjWaves, lds, st>>>(
        x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
    return hipGetLastError();
}

template <bool WF16, int NB>
static hipError_t launch_nb(hipStream_t st, const float* x, long x_stride, int B, int E, const float* gamma, float eps,
                            const void* w, int n_out, float* out, long out_stride) {
#define EI_PROJ_P(PP) \
    case PP: return launch_nbp<WF16, NB, PP>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
    if constexpr (WF16) {
        switch (qkv_project_pieces(E, true)) {
            EI_PROJ_P(2) EI_PROJ_P(4) EI_PROJ_P(5) EI_PROJ_P(8) EI_PROJ_P(10) EI_PROJ_P(16) EI_PROJ_P(20)
            default: return hipErrorInvalidValue;
        }
    } else {
        switch (qkv_project_pieces(E, false)) {
            EI_PROJ_P(4) EI_PROJ_P(8) EI_PROJ_P(10) EI_PROJ_P(16) EI_PROJ_P(20)
            default: return hipErrorInvalidValue;
        }
    }
#undef EI_PROJ_P
}

template <bool WF16>
static hipError_t launch_w(hipStream_t st, const float* x, long x_stride, int B, int E, const float* gamma, float eps,
                           const void* w, int n_out, float* out, long out_stride) {
    if (B <= 1) return launch_nb<WF16, 1>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
    if (B <= 2) return launch_nb<WF16, 2>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
    return launch_nb<WF16, 4>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
}

hipError_t launch_qkv_project(hipStream_t st, const float* x, long x_stride, int B, int E, const float* gamma,
                              float eps, const void* w, bool w_f16, int n_out, float* out, long out_stride) {
    return w_f16 ? launch_w<true>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride)
                 : launch_w<false>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
}

}  // namespace ei
