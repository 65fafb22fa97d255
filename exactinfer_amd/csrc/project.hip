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
//
// Quantised weights (Q8_0, Q4_K, Q6_K: the block formats the reference computes with,
// src/quant.h:21-39) stay in their GGUF block layout.  Each lane decodes items of 16
// consecutive values (half a Q8_0 block, half a 32-value Q4_K sub-block, a 16-value Q6_K group)
// of one of its wave's two rows, with the reference's values (src/quant.cpp:7-60), so every
// weight is the float the CPU path's convert_row gives, before the same FMA dot as the float
// kernels.  Q4_K blocks are whole 16-byte pieces, so each lane loads the two pieces an item needs
// straight into registers; Q8_0 and Q6_K rows are loaded as coalesced pieces (16-byte, or 4-byte
// for Q6_K) and parked in a wave-private LDS area first.
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

// ------------------------------------------------------------------ quantised weights
constexpr int kQWaves = 4;     // waves per workgroup
constexpr int kQRowsPerWave = 2;

template <int T>
struct QFormat;
template <>
struct QFormat<8> {  // Q8_0
    static constexpr int kValues = 32, kBytes = 34;
};
template <>
struct QFormat<12> {  // Q4_K
    static constexpr int kValues = 256, kBytes = 144;
};
template <>
struct QFormat<14> {  // Q6_K
    static constexpr int kValues = 256, kBytes = 210;
};

__device__ __forceinline__ float f16_bits(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)(h & 0xFFFFu)));
}
__device__ __forceinline__ uint32_t lds_u16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }
// 16 bytes from an LDS address that may be only 2-byte aligned (gfx950 LDS reads need no
// natural alignment; memcpy lets the compiler pick the widest reads)
__device__ __forceinline__ u32x4_t lds_16bytes(const uint8_t* p) {
    u32x4_t v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
// byte k of a word as a float (one v_cvt_f32_ubyte)
__device__ __forceinline__ float ubyte_f(uint32_t u, int k) { return (float)((u >> (8 * k)) & 0xFFu); }
// the word as computed, hidden from the optimizer: otherwise it folds a per-word mask into
// every byte's extraction (a bit-field extract per value before the byte conversion; Q4_K
// measured 4% faster with the mask kept, Q8_0 and Q6_K no faster)
__device__ __forceinline__ uint32_t opaque(uint32_t u) {
    asm volatile("" : "+v"(u));
    return u;
}

// Item k (values 16 k .. 16 k + 15) of a row whose bytes start at `row` (LDS) -> wv[16]: half
// a Q8_0 block, half a 32-value Q4_K sub-block, or a 16-value Q6_K group with one scale.  Every
// value is the float the reference's decode gives; the byte-wise conversions are exact.
template <int T>
__device__ __forceinline__ void decode16(const uint8_t* row, int k, float* wv) {
#pragma clang fp contract(off)
    if constexpr (T == 8) {  // Q8_0: y = q * d (src/quant.cpp:7-13)
        const uint8_t* blk = row + 34 * (k >> 1);
        const float d = f16_bits(lds_u16(blk));
        const float off = -128.f * d;  // exact (a power-of-two scaling)
        const u32x4_t q = lds_16bytes(blk + 2 + 16 * (k & 1));
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t u = qw[i] ^ 0x80808080u;  // int8 q + 128 per byte
            // (q + 128) d - 128 d in one rounding: the exact value is q d, so this is the
            // correctly rounded q * d the reference computes (a zero comes out +0 where the
            // reference may have -0, which changes no sum but an exact zero's sign)
#pragma unroll
            for (int b = 0; b < 4; ++b) wv[4 * i + b] = __builtin_fmaf(ubyte_f(u, b), d, off);
        }
    } else if constexpr (T == 12) {  // Q4_K: y = (d sc) q - dmin m (src/quant.cpp:15-33)
        const uint8_t* blk = row + 144 * (k >> 4);
        const int v = (k & 15) * 16, c = v >> 6, hi4 = (v >> 5) & 1, l = v & 31;
        const uint32_t dd = *reinterpret_cast<const uint32_t*>(blk);  // d, dmin (16-byte aligned block)
        const float d = f16_bits(dd), dmin = f16_bits(dd >> 16);
        const uint32_t* pk = reinterpret_cast<const uint32_t*>(blk + 4);  // 12 packed bytes
        const uint32_t p0 = pk[0], p1 = pk[1], p2 = pk[2];
        auto pb = [&](int n) -> int { return (int)(((n < 4 ? p0 : n < 8 ? p1 : p2) >> (8 * (n & 3))) & 0xFFu); };
        const int j = 2 * c + hi4;  // sub-block: 6-bit scale and min (src/quant.h:43-52)
        int sc, m;
        if (j < 4) {
            sc = pb(j) & 63;
            m = pb(j + 4) & 63;
        } else {
            sc = (pb(j + 4) & 15) | ((pb(j - 4) >> 6) << 4);
            m = (pb(j + 4) >> 4) | ((pb(j) >> 6) << 4);
        }
        const float dl = d * (float)sc, ml = dmin * (float)m;
        const u32x4_t q = *reinterpret_cast<const u32x4_t*>(blk + 16 + 32 * c + l);  // 16-byte aligned
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t nib = opaque((qw[i] >> (4 * hi4)) & 0x0F0F0F0Fu);
            // dl * q is exact (17 x 4 significant bits), so the FMA rounds like dl * q - ml
#pragma unroll
            for (int b = 0; b < 4; ++b) wv[4 * i + b] = __builtin_fmaf(dl, ubyte_f(nib, b), -ml);
        }
    } else {  // Q6_K: y = (d sc) (q - 32) (src/quant.cpp:35-60)
        const uint8_t* blk = row + 210 * (k >> 4);
        const int v = (k & 15) * 16, h = v >> 7, g = (v >> 5) & 3, l = v & 31;
        const float d = f16_bits(lds_u16(blk + 208));
        const float dsc = d * (float)(int8_t)blk[192 + 8 * h + (l >> 4) + 2 * g];
        // dsc q - 32 dsc in one rounding (32 dsc is exact): the correctly rounded dsc (q - 32)
        const float off = -32.f * dsc;
        const u32x4_t ql = lds_16bytes(blk + 64 * h + l + 32 * (g & 1));
        const u32x4_t qh = lds_16bytes(blk + 128 + 32 * h + l);
        const uint32_t lw[4] = {ql.x, ql.y, ql.z, ql.w}, hw[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (lw[i] >> (4 * (g >> 1))) & 0x0F0F0F0Fu;
            const uint32_t q6 = lo | (((hw[i] >> (2 * g)) & 0x03030303u) << 4);  // 0..63 per byte
#pragma unroll
            for (int b = 0; b < 4; ++b) wv[4 * i + b] = __builtin_fmaf(dsc, ubyte_f(q6, b), off);
        }
    }
}

// Q4_K item from registers: hdr = the block's first 16 bytes (d, dmin, 12 scale bytes), q = the
// item's 16 bytes of nibbles; sub-block sbj, nibble hi4.  Same arithmetic as decode16<12>.
__device__ __forceinline__ void decode16_q4k_regs(u32x4_t hdr, u32x4_t q, int sbj, int hi4, float* wv) {
#pragma clang fp contract(off)
    const float d = f16_bits(hdr.x), dmin = f16_bits(hdr.x >> 16);
    const uint32_t p0 = hdr.y, p1 = hdr.z, p2 = hdr.w;
    auto pb = [&](int n) -> int { return (int)(((n < 4 ? p0 : n < 8 ? p1 : p2) >> (8 * (n & 3))) & 0xFFu); };
    int sc, m;
    if (sbj < 4) {
        sc = pb(sbj) & 63;
        m = pb(sbj + 4) & 63;
    } else {
        sc = (pb(sbj + 4) & 15) | ((pb(sbj - 4) >> 6) << 4);
        m = (pb(sbj + 4) >> 4) | ((pb(sbj) >> 6) << 4);
    }
    const float dl = d * (float)sc, ml = dmin * (float)m;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t nib = opaque((qw[i] >> (4 * hi4)) & 0x0F0F0F0Fu);
#pragma unroll
        for (int b = 0; b < 4; ++b) wv[4 * i + b] = __builtin_fmaf(dl, ubyte_f(nib, b), -ml);
    }
}

// Quantised rows: T the GGML type (8, 12, 14), NB activation rows (B <= NB), hidden size E
// (compile time: the activation, gamma and weight loads are all issued before any is used,
// activations first, so the norm waits for them alone and overlaps the weight stream).  Row
// bytes RB; wave w owns rows r0, r0 + 1 (clamped to the last row), their bytes at LDS
// qrow + w * 2 RB.
template <int T, int NB, int E>
__global__ __launch_bounds__(64 * kQWaves) void k_qkv_project_q(const float* __restrict__ x, long x_stride, int B,
                                                                const float* __restrict__ gamma, float eps,
                                                                const uint8_t* __restrict__ w, int n_out,
                                                                float* __restrict__ out, long out_stride) {
    using F = QFormat<T>;
    constexpr int RB = E / F::kValues * F::kBytes;
    // Q8_0 and Q4_K rows of a multiple of 512 values are whole 16-byte pieces; Q6_K rows
    // (210-byte blocks) are read in 4-byte pieces
    constexpr bool wide = RB % 16 == 0;
    constexpr int kPiece = wide ? 16 : 4;
    constexpr int kPer = (RB / kPiece + 63) / 64;  // pieces per lane per row
    constexpr int kEl = E / (64 * kQWaves);        // activation elements per thread per row
    static_assert(E % (64 * kQWaves) == 0 && E % 512 == 0 && RB % 4 == 0, "hidden size");
    extern __shared__ __align__(16) float hs[];  // [B][E] normed activations, then the rows' bytes
    __shared__ double ssum[kQWaves][NB];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r0 = (blockIdx.x * kQWaves + wv) * kQRowsPerWave;

    // ---- activations and gamma, then this wave's row bytes (read once: non-temporal)
    float xv[NB][kEl], gv[kEl];
#pragma unroll
    for (int i = 0; i < kEl; ++i) gv[i] = gamma[tid + i * 64 * kQWaves];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < kEl; ++i) xv[b][i] = b < B ? x[(size_t)b * x_stride + tid + i * 64 * kQWaves] : 0.f;
    // Q4_K blocks (144 bytes) are whole 16-byte pieces: each lane loads the two pieces each of its
    // items needs (the block's header with d, dmin and the scales; the item's 16 bytes of nibbles) and
    // decodes from registers, without staging the row through LDS (5.73-5.75 against 6.07-6.08 us at
    // Qwen3-4B).  Q8_0 (34-byte) and Q6_K (210-byte) blocks are not piece-aligned and stay staged.
    constexpr bool kDirect = T == 12;
    u32x4_t dh[kDirect ? E / 512 : 1], dq[kDirect ? E / 512 : 1];
    if constexpr (kDirect) {
        const uint8_t* row = w + (size_t)min(r0 + (lane & 1), n_out - 1) * RB;
#pragma unroll
        for (int j = 0; j < E / 512; ++j) {
            const int k = (lane >> 1) + 32 * j, v = (k & 15) * 16;
            const uint8_t* blk = row + 144 * (k >> 4);
            dh[j] = *reinterpret_cast<const u32x4_t*>(blk);
            dq[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(blk + 16 + 32 * (v >> 6) + (v & 31)));
        }
    }
    u32x4_t pc[kQRowsPerWave][wide ? kPer : 1];
    uint32_t pd[kQRowsPerWave][wide ? 1 : kPer];
#pragma unroll
    for (int rr = 0; rr < kQRowsPerWave; ++rr) {
        if (kDirect) break;
        const uint8_t* row = w + (size_t)min(r0 + rr, n_out - 1) * RB;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int p = min(lane + 64 * k, RB / kPiece - 1);  // clamped: the tail lanes reload the last piece
            if constexpr (wide) pc[rr][k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(row) + p);
            else pd[rr][k] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(row) + p);
        }
    }

    // ---- attention RMSNorm of the B rows into LDS (src/ops.cpp:155-160), as the float kernels
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
        for (int k = 0; k < kQWaves; ++k) ss += ssum[k][b];
        const float inv = (float)(1.0 / sqrt(ss / (double)E + (double)eps));
#pragma unroll
        for (int i = 0; i < kEl; ++i) {
#pragma clang fp contract(off)
            hs[b * E + tid + i * 64 * kQWaves] = (xv[b][i] * inv) * gv[i];
        }
    }

    // ---- the row bytes into this wave's LDS area (sized for B activation rows)
    uint8_t* qrow = reinterpret_cast<uint8_t*>(hs + B * E) + (size_t)wv * kQRowsPerWave * RB;
#pragma unroll
    for (int rr = 0; rr < kQRowsPerWave; ++rr) {
        if (kDirect) break;
        uint8_t* dst = qrow + rr * RB;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int p = lane + 64 * k;
            if (p < RB / kPiece) {
                if constexpr (wide) reinterpret_cast<u32x4_t*>(dst)[p] = pc[rr][k];
                else reinterpret_cast<uint32_t*>(dst)[p] = pd[rr][k];
            }
        }
    }
    __syncthreads();  // the activations of every wave and this wave's row bytes

    // ---- decode items of 16 values and accumulate: lane l works on row l & 1, items l / 2,
    // l / 2 + 32, ... of it; the lanes of one row are summed at the end
    const int rr = lane & 1;
    const uint8_t* myrow = qrow + rr * RB;
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.f;
#pragma unroll
    for (int j = 0; j < E / 512; ++j) {
        const int k = (lane >> 1) + 32 * j;
        float wf[16];
        if constexpr (kDirect) {
            const int v = (k & 15) * 16;
            decode16_q4k_regs(dh[j], dq[j], 2 * (v >> 6) + ((v >> 5) & 1), (v >> 5) & 1, wf);
        } else {
            decode16<T>(myrow, k, wf);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b >= B) break;
            const float4* hp = reinterpret_cast<const float4*>(hs + b * E + 16 * k);
            float a = acc[b];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 hv = hp[q4];
                a = fmaf(wf[4 * q4], hv.x, a);
                a = fmaf(wf[4 * q4 + 1], hv.y, a);
                a = fmaf(wf[4 * q4 + 2], hv.z, a);
                a = fmaf(wf[4 * q4 + 3], hv.w, a);
            }
            acc[b] = a;
        }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (b >= B) break;
        float sres = acc[b];  // sum over the 32 lanes of this lane's row (xor 2 .. 32 keep the parity)
        sres += lane_xor<2>(sres);
        sres += lane_xor<4>(sres);
        sres += lane_xor<8>(sres);
        sres += lane_xor<16>(sres);
        sres += lane_xor<32>(sres);
        if (lane < 2 && r0 + rr < n_out) out[(size_t)b * out_stride + r0 + rr] = sres;
    }
}

static size_t qkv_project_q_lds(int E, int w_type, int B) {
    const int vals = w_type == 8 ? 32 : 256, bytes = w_type == 8 ? 34 : w_type == 12 ? 144 : 210;
    const size_t rb = (size_t)(E / vals) * bytes;
    return (size_t)B * E * sizeof(float) + (size_t)kQWaves * kQRowsPerWave * rb;
}

template <int T, int NB, int E>
static hipError_t launch_q_nbe(hipStream_t st, const float* x, long x_stride, int B, const float* gamma, float eps,
                               const void* w, int n_out, float* out, long out_stride) {
    static std::atomic<bool> opted;
    if (const hipError_t e = opt_in_lds(opted, (const void*)k_qkv_project_q<T, NB, E>, 150 * 1024); e != hipSuccess)
        return e;
    const int per_block = kQWaves * kQRowsPerWave;
    k_qkv_project_q<T, NB, E><<<(n_out + per_block - 1) / per_block, 64 * kQWaves, qkv_project_q_lds(E, T, B), st>>>(
        x, x_stride, B, gamma, eps, static_cast<const uint8_t*>(w), n_out, out, out_stride);
    return hipGetLastError();
}

template <int T, int NB>
static hipError_t launch_q_nb(hipStream_t st, const float* x, long x_stride, int B, int E, const float* gamma,
                              float eps, const void* w, int n_out, float* out, long out_stride) {
#define EI_PROJ_QE(EE) \
    case EE: return launch_q_nbe<T, NB, EE>(st, x, x_stride, B, gamma, eps, w, n_out, out, out_stride);
    switch (E) {
        EI_PROJ_QE(1024) EI_PROJ_QE(2048) EI_PROJ_QE(2560) EI_PROJ_QE(4096) EI_PROJ_QE(5120)
        default: return hipErrorInvalidValue;
    }
#undef EI_PROJ_QE
}

template <int T>
static hipError_t launch_q(hipStream_t st, const float* x, long x_stride, int B, int E, const float* gamma, float eps,
                           const void* w, int n_out, float* out, long out_stride) {
    if (B <= 1) return launch_q_nb<T, 1>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
    if (B <= 2) return launch_q_nb<T, 2>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
    return launch_q_nb<T, 4>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
}

int qkv_project_max_rows(int E) {
    const int r = E > 0 ? kProjMaxLdsFloats / E : 0;
    return r < kProjMaxRows ? r : kProjMaxRows;
}

// 16-byte pieces per lane per row for the supported hidden sizes (0: not built)
static int qkv_project_pieces(int E, bool w_f16) {
    const int per = 64 * (w_f16 ? 8 : 4);
    if (E <= 0 || E % per) return 0;
    const int p = E / per;
    if (w_f16) return (p == 2 || p == 4 || p == 5 || p == 8 || p == 10 || p == 16 || p == 20) ? p : 0;
    return (p == 4 || p == 8 || p == 10 || p == 16 || p == 20) ? p : 0;
}

bool qkv_project_built(int E, int w_type) {
    if (w_type == 0 || w_type == 1) return qkv_project_pieces(E, w_type == 1) != 0;
    if (w_type != 8 && w_type != 12 && w_type != 14) return false;
    // the dense Qwen3 hidden sizes (whole 256-value super-blocks, 8-value items per lane)
    return E == 1024 || E == 2048 || E == 2560 || E == 4096 || E == 5120;
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
                              float eps, const void* w, int w_type, int n_out, float* out, long out_stride) {
    switch (w_type) {
        case 0: return launch_w<false>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
        case 1: return launch_w<true>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
        case 8: return launch_q<8>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
        case 12: return launch_q<12>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
        case 14: return launch_q<14>(st, x, x_stride, B, E, gamma, eps, w, n_out, out, out_stride);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace ei
