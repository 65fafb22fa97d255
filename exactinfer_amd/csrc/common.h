// common.h — shared device helpers for the gfx950 attention kernels.
//
// Wave64 lane exchanges: DPP for partners inside a row of 16 lanes, ds_swizzle (bit mode,
// no LDS memory access) for partners 4 and 16 lanes away, and a bpermute for the half-wave
// exchange.  All helpers are exact data moves; reductions built from them are
// deterministic for a given launch shape.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ei {

constexpr int kHeadDim = 128;  // Qwen3 head_dim; every kernel is specialised for it

// ------------------------------------------------------------------ lane exchanges
__device__ __forceinline__ float lane_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));  // quad_perm 1,0,3,2
}
__device__ __forceinline__ float lane_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));  // quad_perm 2,3,0,1
}
__device__ __forceinline__ float lane_xor4(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x101F));  // and 0x1F, xor 4
}
__device__ __forceinline__ float lane_xor8(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));  // row_ror:8
}
__device__ __forceinline__ float lane_xor16(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));  // and 0x1F, xor 16
}
__device__ __forceinline__ float lane_xor32(float v) { return __shfl_xor(v, 32); }

// Half-wave reductions with v_permlane32_swap: after the swap each lane holds its own value
// and that of lane ^ 32 (in some order), so a symmetric combine needs no ordering.
__device__ __forceinline__ float half_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int M>
__device__ __forceinline__ float lane_xor(float v) {
    if constexpr (M == 1) return lane_xor1(v);
    else if constexpr (M == 2) return lane_xor2(v);
    else if constexpr (M == 4) return lane_xor4(v);
    else if constexpr (M == 8) return lane_xor8(v);
    else if constexpr (M == 16) return lane_xor16(v);
    else return lane_xor32(v);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, lane_xor1(v));
    v = fmaxf(v, lane_xor2(v));
    v = fmaxf(v, lane_xor4(v));
    v = fmaxf(v, lane_xor8(v));
    v = fmaxf(v, lane_xor16(v));
    return fmaxf(v, lane_xor32(v));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += lane_xor1(v);
    v += lane_xor2(v);
    v += lane_xor4(v);
    v += lane_xor8(v);
    v += lane_xor16(v);
    return v + lane_xor32(v);
}

// Butterfly sum of a double over the wave: both halves of the double move through the same
// DPP / swizzle exchanges as the float helpers (no LDS round trips).  Partners add the same
// two values, so every lane ends with identical bits.
template <int M>
__device__ __forceinline__ double lane_xor_f64(double v) {
    const unsigned long long b = __double_as_longlong(v);
    const float lo = lane_xor<M>(__uint_as_float((unsigned)b));
    const float hi = lane_xor<M>(__uint_as_float((unsigned)(b >> 32)));
    return __longlong_as_double((long long)(((unsigned long long)__float_as_uint(hi) << 32) | __float_as_uint(lo)));
}

__device__ __forceinline__ double wave_sum_f64(double v) {
    v += lane_xor_f64<1>(v);
    v += lane_xor_f64<2>(v);
    v += lane_xor_f64<4>(v);
    v += lane_xor_f64<8>(v);
    v += lane_xor_f64<16>(v);
    return v + lane_xor_f64<32>(v);
}

// ------------------------------------------------------------------ LDS DMA
// LDS byte address of a __shared__ object (the low 32 bits of its flat address).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)reinterpret_cast<uintptr_t>(p);
}

// One LDS-DMA instruction: every active lane copies 16 bytes from its global address to
// LDS byte address m0_base + 16*lane.  Issued through inline asm so the compiler does not
// see a pending LDS write and serialise unrelated LDS accesses behind it; completion is
// tracked by hand with wait_vmcnt (each instruction counts one in vmcnt).
__device__ __forceinline__ void dma16(const float* g, uint32_t m0_base) {
    // m0_base is wave-uniform by construction; readfirstlane keeps it in an SGPR even when
    // the compiler computed it in VGPRs (e.g. inside a divergent branch)
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g),
                 "s"(__builtin_amdgcn_readfirstlane(m0_base))
                 : "memory", "m0");
}

// The same with the non-temporal (streaming) cache policy, for data read once: a decode
// step's KV stream runs ~11% faster with it than with the default policy on MI355X.
__device__ __forceinline__ void dma16_nt(const float* g, uint32_t m0_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g),
                 "s"(__builtin_amdgcn_readfirstlane(m0_base))
                 : "memory", "m0");
}

// Scalar-base form: lane address = sbase (wave-uniform 64-bit byte address in SGPRs) +
// voff (32-bit per-lane byte offset).  With per-lane offsets fixed for a whole loop, each
// instruction costs only scalar arithmetic for its base.
__device__ __forceinline__ void dma16_s(uint64_t sbase, uint32_t voff, uint32_t m0_base) {
    // the operands are uniform by construction; readfirstlane states it to the compiler
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)sbase);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(sbase >> 32));
    const uint64_t sb = ((uint64_t)hi << 32) | lo;
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sb),
                 "s"(__builtin_amdgcn_readfirstlane(m0_base))
                 : "memory", "m0");
}

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] + vmcnt[5:4] at 15:14,
// expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// ------------------------------------------------------------------ QK-norm + RoPE of one head
// One wave normalises and rotates one 128-float head vector; lane l holds elements l
// (x0) and l+64 (x1).
//   ss  = sum of double(x)^2 (tree order; the value in double matches the sequential
//         sum to ~1e-16 relative, so the float `inv` is the reference's except within an
//         ulp-rounding tie)                                   src/ops.cpp:155-160
//   inv = float(1 / sqrt(ss/128 + double(eps)));  y = (x * inv) * gamma
//   NEOX rotation of halves with the table's (cos, sin):      src/model.cpp:23-32
//   y[i] = a*c - b*s,  y[i+half] = a*s + b*c   (no FMA contraction: two products, then +/-)
// With rope_dim = 128 (Qwen3) the partners i and i+64 sit in the same lane and the rotation
// is done in registers; other rope_dims exchange partners through `dst`, 128 floats of
// LDS scratch owned by this wave.  Returns the outputs for elements lane and lane+64.
__device__ __forceinline__ void scale_rope_vals(float x0, float x1, float inv, float g0, float g1,
                                                const float2* __restrict__ cs_row, int rope_dim, float* dst,
                                                int lane, float* o0, float* o1);

__device__ __forceinline__ void norm_rope_vals(float x0, float x1, float g0, float g1,
                                               const float2* __restrict__ cs_row, int rope_dim, float eps,
                                               float* dst, int lane, float* o0, float* o1) {
#pragma clang fp contract(off)
    double ss = (double)x0 * (double)x0 + (double)x1 * (double)x1;
    ss = wave_sum_f64(ss);
    const float inv = (float)(1.0 / sqrt(ss / (double)kHeadDim + (double)eps));
    scale_rope_vals(x0, x1, inv, g0, g1, cs_row, rope_dim, dst, lane, o0, o1);
}

// The norm factors of N heads at once (N a power of two, <= 64; lane l holds elements l and
// l+64 of head j in x0[j], x1[j]).  The N sums of squares share one transposing butterfly: in
// the steps over lane bits 5, 4, ... a lane keeps half of its remaining sums and adds its
// partner's copy of that half (N/2 + N/4 + ... exchanges instead of 6N), then the single
// remaining sum finishes the plain butterfly; lane L ends with the total of head
// 32*b5 + 16*b4 + ... of its high bits (for N = 4: head 2*b5 + b4).  Every lane computes
// 1/sqrt for its own head, so the double square root and division run once for all N heads,
// and head j's factor is read from a lane that holds it.  The sum is a different tree order of
// the same exact squares as norm_rope_vals; both match the sequential double sum to ~1e-16
// relative.
template <int N>
__device__ __forceinline__ void head_inv(const float* x0, const float* x1, float eps, float* inv, int lane) {
#pragma clang fp contract(off)
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "a power of two");
    double v[N];
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = (double)x0[j] * (double)x0[j] + (double)x1[j] * (double)x1[j];
    int n = N;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const bool up = (lane & m) != 0;
        if (n > 1) {
#pragma unroll
            for (int i = 0; i < n / 2; ++i) {
                const double send = up ? v[i] : v[i + n / 2];
                const double keep = up ? v[i + n / 2] : v[i];
                double r;
                if (m == 32) r = lane_xor_f64<32>(send);
                else if (m == 16) r = lane_xor_f64<16>(send);
                else if (m == 8) r = lane_xor_f64<8>(send);
                else if (m == 4) r = lane_xor_f64<4>(send);
                else if (m == 2) r = lane_xor_f64<2>(send);
                else r = lane_xor_f64<1>(send);
                v[i] = keep + r;
            }
            n /= 2;
        } else {
            double r;
            if (m == 32) r = lane_xor_f64<32>(v[0]);
            else if (m == 16) r = lane_xor_f64<16>(v[0]);
            else if (m == 8) r = lane_xor_f64<8>(v[0]);
            else if (m == 4) r = lane_xor_f64<4>(v[0]);
            else if (m == 2) r = lane_xor_f64<2>(v[0]);
            else r = lane_xor_f64<1>(v[0]);
            v[0] += r;
        }
    }
    const float mine = (float)(1.0 / sqrt(v[0] / (double)kHeadDim + (double)eps));
#pragma unroll
    for (int j = 0; j < N; ++j) {
        // the lane whose high bits spell j: bit 5 - k of the lane is bit (log2 N - 1 - k) of j
        int src = 0;
#pragma unroll
        for (int k = 0, b = N / 2; b >= 1; ++k, b >>= 1)
            if (j & b) src |= 32 >> k;
        inv[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), src));
    }
}

// y = (x * inv) * gamma, then the NEOX rotation (see norm_rope_vals).
__device__ __forceinline__ void scale_rope_vals(float x0, float x1, float inv, float g0, float g1,
                                                const float2* __restrict__ cs_row, int rope_dim, float* dst,
                                                int lane, float* o0, float* o1) {
#pragma clang fp contract(off)
    const float y0 = (x0 * inv) * g0;
    const float y1 = (x1 * inv) * g1;
    if (rope_dim == kHeadDim) {
        const float2 t = cs_row[lane];
        const float acs = y0 * t.x, bsn = y1 * t.y;
        const float asn = y0 * t.y, bcs = y1 * t.x;
        *o0 = acs - bsn;
        *o1 = asn + bcs;
        return;
    }
    dst[lane] = y0;
    dst[lane + 64] = y1;
    __builtin_amdgcn_wave_barrier();
    const int half = rope_dim >> 1;
    float r0 = y0, r1 = y1;
    // element e: rotated if e < rope_dim; partner e+half (e < half) or e-half
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int e = lane + 64 * k;
        float r = k == 0 ? y0 : y1;
        if (e < rope_dim) {
            if (e < half) {
                const float2 t = cs_row[e];
                const float a = r, b = dst[e + half];
                const float acs = a * t.x, bsn = b * t.y;
                r = acs - bsn;
            } else {
                const float2 t = cs_row[e - half];
                const float a = dst[e - half], b = r;
                const float asn = a * t.y, bcs = b * t.x;
                r = asn + bcs;
            }
        }
        if (k == 0) r0 = r;
        else r1 = r;
    }
    __builtin_amdgcn_wave_barrier();
    *o0 = r0;
    *o1 = r1;
}

__device__ __forceinline__ void norm_rope_head(const float* __restrict__ src, const float* __restrict__ gamma,
                                               const float2* __restrict__ cs_row, int rope_dim, float eps,
                                               float* dst, int lane, float* o0, float* o1) {
    norm_rope_vals(src[lane], src[lane + 64], gamma[lane], gamma[lane + 64], cs_row, rope_dim, eps, dst, lane, o0,
                   o1);
}

// ------------------------------------------------------------------ synthetic inputs
// Counter-based N(0,1): element e of stream `seed` is one Box-Muller normal
// z = sqrt(-2 ln u1) cos(2 pi u2) from two 53-bit uniforms (two splitmix64 outputs), every step an
// IEEE double addition, subtraction or multiplication in a fixed order (no division, no library
// call, no contraction), so the GPU fill and the CPU checker produce identical bits.
//   ln u1:  u1 = m 2^k, m in [sqrt(1/2), sqrt(2)) from the bits; ln m = 2 atanh t,
//           t = (m - 1) / (m + 1), as t (1 + t^2/3 + ... + t^24/25) (|t| <= 0.172); the
//           reciprocal by six Newton steps from 7/16 (m + 1 lies in [1.7, 2.5]);
//   sqrt y: y (1/sqrt y), six Newton steps x (3/2 - y x^2 / 2) from the integer estimate
//           0x5FE6EB50C7B537A9 - bits(y)/2 (Lomont's constant for doubles);
//   cos:    quarter turn q = floor(4 u2), f = 4 u2 - q (both exact); the angle f pi/2, or
//           (1 - f) pi/2 with sine and cosine swapped, lies in [0, pi/4], where Taylor series
//           to degree 17/18 are exact below 2^-60.
// Rounded to float once; |z| <= 8.6 (u1 >= 2^-53).
__host__ __device__ __forceinline__ uint64_t synth_mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__host__ __device__ __forceinline__ float synth_normal(uint64_t seed, uint64_t e) {
#pragma clang fp contract(off)
    const uint64_t base = seed * 0xD1B54A32D192ED03ull + 2ull * e;
    const uint64_t h1 = synth_mix64(base), h2 = synth_mix64(base + 1ull);
    const double u1 = (double)((h1 >> 11) + 1ull) * 0x1.0p-53;  // (0, 1]
    const double u2 = (double)(h2 >> 11) * 0x1.0p-53;           // [0, 1)
    // ln u1
    const uint64_t ub = (uint64_t)__builtin_bit_cast(unsigned long long, u1);
    int k = (int)((ub >> 52) & 0x7FF) - 1023;
    double m = __builtin_bit_cast(double, (unsigned long long)((ub & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull));
    if (m > 1.4142135623730951) {
        m = m * 0.5;
        k = k + 1;
    }
    const double den = m + 1.0;
    double r = 0.4375;
#pragma unroll
    for (int i = 0; i < 6; ++i) r = r * (2.0 - den * r);
    constexpr double inv_odd[13] = {1.0,        1.0 / 3.0,  1.0 / 5.0,  1.0 / 7.0,  1.0 / 9.0,
                                    1.0 / 11.0, 1.0 / 13.0, 1.0 / 15.0, 1.0 / 17.0, 1.0 / 19.0,
                                    1.0 / 21.0, 1.0 / 23.0, 1.0 / 25.0};
    const double t = (m - 1.0) * r, t2 = t * t;
    double poly = inv_odd[12];
#pragma unroll
    for (int j = 11; j >= 0; --j) poly = poly * t2 + inv_odd[j];
    const double ln_u1 = (double)k * 0.6931471805599453 + 2.0 * t * poly;
    // sqrt(-2 ln u1)
    const double y = -2.0 * ln_u1;
    double rad = 0.0;
    if (y > 0.0) {
        const unsigned long long yb = __builtin_bit_cast(unsigned long long, y);
        double x = __builtin_bit_cast(double, 0x5FE6EB50C7B537A9ull - (yb >> 1));
#pragma unroll
        for (int i = 0; i < 6; ++i) x = x * (1.5 - 0.5 * y * x * x);
        rad = y * x;
    }
    // cos(2 pi u2)
    const double v = 4.0 * u2;
    const int q = (int)v;
    const double f = v - (double)q;
    const bool swap = f > 0.5;
    const double phi = (swap ? 1.0 - f : f) * 1.5707963267948966, p2 = phi * phi;
    constexpr double inv_fact[19] = {1.0,
                                     1.0,
                                     1.0 / 2.0,
                                     1.0 / 6.0,
                                     1.0 / 24.0,
                                     1.0 / 120.0,
                                     1.0 / 720.0,
                                     1.0 / 5040.0,
                                     1.0 / 40320.0,
                                     1.0 / 362880.0,
                                     1.0 / 3628800.0,
                                     1.0 / 39916800.0,
                                     1.0 / 479001600.0,
                                     1.0 / 6227020800.0,
                                     1.0 / 87178291200.0,
                                     1.0 / 1307674368000.0,
                                     1.0 / 20922789888000.0,
                                     1.0 / 355687428096000.0,
                                     1.0 / 6402373705728000.0};
    double sn = inv_fact[17], cs = inv_fact[18];
#pragma unroll
    for (int j = 15; j >= 1; j -= 2) sn = -sn * p2 + inv_fact[j];  // sin(phi) / phi
#pragma unroll
    for (int j = 16; j >= 0; j -= 2) cs = -cs * p2 + inv_fact[j];
    sn = sn * phi;
    const double c0 = swap ? sn : cs, s0 = swap ? cs : sn;
    const double cosv = q == 0 ? c0 : q == 1 ? -s0 : q == 2 ? -c0 : s0;
    return (float)(rad * cosv);
}

}  // namespace ei
