/*
 * oracle.c — CPU oracle for the Qwen3 attention hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * This file is a plain-C restatement of the reference CPU path's arithmetic, used as the
 * parity checker for the HIP kernels.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product path (exactinfer_amd/) never calls it.
 *
 * Build: gcc -O2 -ffp-contract=off (no contraction, no reassociation) so every float
 * operation happens in the order the reference writes it (MSVC /fp:precise semantics of
 * the reference build, CMakeLists.txt:49), with that build's ISA (-mavx2 -mfma -mf16c for
 * its /arch:AVX2), which changes no result under those two rules.  OpenMP only splits independent query heads,
 * exactly like the reference (src/model.cpp:191), so results do not depend on thread count.
 *
 * Pinning of each function (what proves the restatement right, checked in tests/):
 *   orc_rmsnorm          bit-exact vs the reference's own el::rmsnorm compiled from
 *                        src/ops.cpp (oracle/_ref), + float64 closed form.
 *   orc_rope_inv_freq,   bit-exact vs el::rope_inv_freq / el::rope compiled from
 *   orc_rope             src/model.cpp (oracle/_ref), + rotation-norm invariant.
 *   orc_rope_table       bit-exact vs orc_rope applied to unit vectors (the table is what
 *                        src/cuda/model_cuda.cu:1610-1619 precomputes).
 *   orc_kv_append        byte compare, untouched-row invariant.
 *   orc_attn_decode      float64 brute force (orc_attn_f64) on small inputs; closed forms
 *                        (1 key -> v0, identical keys -> mean V, dominant score -> that V);
 *                        GQA == repeated K/V.  The reference attention loop sits inside
 *                        CpuModel::forward, which needs a GGUF reader that does not build
 *                        on Linux (src/gguf.cpp:12 includes <windows.h>), so it cannot be
 *                        run directly.
 *   orc_attn_split_combine  == single-pass orc_attn_decode within fp32 tolerance, and
 *                        float64 brute force; empty-split rule.
 *   orc_attn_f64         textbook softmax attention in double; checked by the closed forms.
 *   orc_f16_to_f32,      bit-exact vs the reference's own f16_to_f32, dot_f32 and dot_f16
 *   orc_dot_f32,         (src/ops.cpp:22-24, :92-118) compiled from source (oracle/_ref),
 *   orc_dot_f16          on every binary16 pattern and on dot lengths with and without
 *                        tails; orc_matvec + float64 bound.
 *   orc_dequant_q8_0,    bit-exact vs the reference's own dequant_q8_0 / _q4_K / _q6_K
 *   orc_dequant_q4_K,    (src/quant.cpp:7-60) compiled from source (oracle/_ref), on random
 *   orc_dequant_q6_K     blocks; committed golden vectors; closed forms (unit scales give
 *                        the stored integers back).
 *   orc_fill_normal      synthetic-input generator (not a reference function): Box-Muller
 *                        from basic double operations, equal bit for bit to float32 of
 *                        numpy's float64 sqrt/log/cos formula, KS-tested, and equal to the
 *                        GPU fill.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ synthetic inputs
 * Counter-based generator shared with the GPU fill kernel (exactinfer_amd/csrc/common.h,
 * synth_normal, the same steps): element e of stream `seed` is one Box-Muller normal,
 * z = sqrt(-2 ln u1) cos(2 pi u2), from two 53-bit uniforms (two splitmix64 outputs).  Every
 * step is an IEEE double addition, subtraction or multiplication in a fixed order (no division,
 * no library call, no contraction), so every platform produces identical bits:
 *   ln u1    u1 = m 2^k with m in [sqrt(1/2), sqrt(2)) (exact, from the bits);
 *            ln m = 2 atanh t, t = (m - 1) / (m + 1), as t (1 + t^2/3 + ... + t^24/25)
 *            (|t| <= 0.172: truncation below 2^-60); the reciprocal by six Newton steps
 *            from 7/16 (m + 1 lies in [1.7, 2.5]);
 *   sqrt y   y (1/sqrt y), 1/sqrt y by six Newton steps x (3/2 - y x^2 / 2) from the
 *            integer estimate 0x5FE6EB50C7B537A9 - bits(y)/2 (Lomont's constant for doubles);
 *   cos      the quarter turn q = floor(4 u2) and f = 4 u2 - q (both exact); the angle
 *            f pi/2, or (1 - f) pi/2 with sine and cosine swapped, lies in [0, pi/4], where
 *            Taylor series to degree 17/18 are exact below 2^-60.
 * The result is rounded to float once.  |z| <= 8.6 (u1 >= 2^-53). */
static inline uint64_t orc_mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline double orc_bits_double(uint64_t u) {
    double d;
    memcpy(&d, &u, 8);
    return d;
}

static inline uint64_t orc_double_bits(double d) {
    uint64_t u;
    memcpy(&u, &d, 8);
    return u;
}

static inline float orc_normal_at(uint64_t seed, uint64_t e) {
    const uint64_t base = seed * 0xD1B54A32D192ED03ull + 2ull * e;
    const uint64_t h1 = orc_mix64(base), h2 = orc_mix64(base + 1ull);
    const double u1 = (double)((h1 >> 11) + 1ull) * 0x1.0p-53; /* (0, 1] */
    const double u2 = (double)(h2 >> 11) * 0x1.0p-53;          /* [0, 1) */
    /* ln u1 */
    const uint64_t ub = orc_double_bits(u1);
    int k = (int)((ub >> 52) & 0x7FF) - 1023;
    double m = orc_bits_double((ub & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull); /* [1, 2) */
    if (m > 1.4142135623730951) {
        m = m * 0.5;
        k = k + 1;
    }
    const double den = m + 1.0;
    double r = 0.4375;
    for (int i = 0; i < 6; ++i) r = r * (2.0 - den * r);
    static const double inv_odd[13] = {1.0,        1.0 / 3.0,  1.0 / 5.0,  1.0 / 7.0,  1.0 / 9.0,
                                       1.0 / 11.0, 1.0 / 13.0, 1.0 / 15.0, 1.0 / 17.0, 1.0 / 19.0,
                                       1.0 / 21.0, 1.0 / 23.0, 1.0 / 25.0};
    const double t = (m - 1.0) * r, t2 = t * t;
    double poly = inv_odd[12];
    for (int j = 11; j >= 0; --j) poly = poly * t2 + inv_odd[j];
    const double ln_u1 = (double)k * 0.6931471805599453 + 2.0 * t * poly;
    /* sqrt(-2 ln u1) */
    const double y = -2.0 * ln_u1;
    double rad = 0.0;
    if (y > 0.0) {
        double x = orc_bits_double(0x5FE6EB50C7B537A9ull - (orc_double_bits(y) >> 1));
        for (int i = 0; i < 6; ++i) x = x * (1.5 - 0.5 * y * x * x);
        rad = y * x;
    }
    /* cos(2 pi u2) */
    const double v = 4.0 * u2;
    const int q = (int)v;
    const double f = v - (double)q;
    const int swap = f > 0.5;
    const double phi = (swap ? 1.0 - f : f) * 1.5707963267948966, p2 = phi * phi;
    static const double inv_fact[19] = {1.0, 1.0, 1.0 / 2.0, 1.0 / 6.0, 1.0 / 24.0, 1.0 / 120.0, 1.0 / 720.0,
                                        1.0 / 5040.0, 1.0 / 40320.0, 1.0 / 362880.0, 1.0 / 3628800.0,
                                        1.0 / 39916800.0, 1.0 / 479001600.0, 1.0 / 6227020800.0,
                                        1.0 / 87178291200.0, 1.0 / 1307674368000.0, 1.0 / 20922789888000.0,
                                        1.0 / 355687428096000.0, 1.0 / 6402373705728000.0};
    double sn = inv_fact[17], cs = inv_fact[18];
    for (int j = 15; j >= 1; j -= 2) sn = -sn * p2 + inv_fact[j]; /* sin/phi: 1 - p2/3! + ... */
    for (int j = 16; j >= 0; j -= 2) cs = -cs * p2 + inv_fact[j];
    sn = sn * phi;
    const double c0 = swap ? sn : cs, s0 = swap ? cs : sn;
    const double cosv = q == 0 ? c0 : q == 1 ? -s0 : q == 2 ? -c0 : s0;
    return (float)(rad * cosv);
}

ORC_API void orc_fill_normal(float* out, size_t n, uint64_t seed, uint64_t offset) {
    /* elements are independent (counter-based), so threads change no bit */
#pragma omp parallel for schedule(static) if (n >= 65536)
    for (long i = 0; i < (long)n; ++i) out[i] = orc_normal_at(seed, offset + (uint64_t)i);
}

/* gamma ~ 1 + 0.1 * N(0,1), rounded step by step in float */
ORC_API void orc_fill_gamma(float* out, size_t n, uint64_t seed) {
    for (size_t i = 0; i < n; ++i) {
        const float z = orc_normal_at(seed, i);
        const float t = 0.1f * z;
        out[i] = 1.0f + t;
    }
}

/* ------------------------------------------------------------------ QK-norm
 * src/ops.cpp:155-160: ss = sum double(x)^2 sequentially; inv = float(1/sqrt(ss/n + eps))
 * (eps promoted to double); out = x * inv * w, two float multiplies left to right. */
ORC_API void orc_rmsnorm(float* out, const float* x, const float* w, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * x[i];
    const float inv = (float)(1.0 / sqrt(ss / n + eps));
    for (int i = 0; i < n; ++i) {
        const float t = x[i] * inv;
        out[i] = t * w[i];
    }
}

/* ------------------------------------------------------------------ RoPE
 * src/model.cpp:105-109: inv_freq[i] = pow(base, -2.0*i/rope_dim) in double. */
ORC_API void orc_rope_inv_freq(double* out, int rope_dim, double base) {
    for (int i = 0; i < rope_dim / 2; ++i) out[i] = pow(base, -2.0 * i / rope_dim);
}

/* src/model.cpp:23-32: NEOX rotation of halves; angle th = pos*inv_freq[i] in double;
 * cs = float(cos th), sn = float(sin th); v[i] = a*cs - b*sn, v[i+half] = a*sn + b*cs. */
ORC_API void orc_rope(float* v, int pos, int dim, const double* inv_freq) {
    const int half = dim / 2;
    for (int i = 0; i < half; ++i) {
        const double th = pos * inv_freq[i];
        const float cs = (float)cos(th), sn = (float)sin(th);
        const float a = v[i], b = v[i + half];
        const float acs = a * cs, bsn = b * sn, asn = a * sn, bcs = b * cs;
        v[i] = acs - bsn;
        v[i + half] = asn + bcs;
    }
}

/* src/cuda/model_cuda.cu:1610-1619: table cs[p][i] = (float(cos th), float(sin th)),
 * th = double(p) * inv_freq[i], stored as interleaved pairs [n_ctx][rope_dim/2][2]. */
ORC_API void orc_rope_table(float* cs, int n_ctx, int rope_dim, double base) {
    const int half = rope_dim / 2;
    double* inv = (double*)malloc(sizeof(double) * (size_t)(half > 0 ? half : 1));
    orc_rope_inv_freq(inv, rope_dim, base);
    for (int p = 0; p < n_ctx; ++p)
        for (int i = 0; i < half; ++i) {
            const double th = (double)p * inv[i];
            cs[((size_t)p * half + i) * 2 + 0] = (float)cos(th);
            cs[((size_t)p * half + i) * 2 + 1] = (float)sin(th);
        }
    free(inv);
}

/* Per-token QK-norm + RoPE over a block of rows, src/model.cpp:176-185: for row b (at
 * position pos0+b) and each head h: rmsnorm(v, v, gamma, D, eps) then rope(v, pos, rope_dim).
 * buf row b starts at buf + b*row_stride; head h at + h*D. */
ORC_API void orc_headnorm_rope(float* buf, int rows, long row_stride, int n_heads, int D, const float* gamma,
                               int pos0, int rope_dim, double base, float eps) {
    double* inv = (double*)malloc(sizeof(double) * (size_t)(rope_dim / 2 > 0 ? rope_dim / 2 : 1));
    orc_rope_inv_freq(inv, rope_dim, base);
    for (int b = 0; b < rows; ++b)
        for (int h = 0; h < n_heads; ++h) {
            float* v = buf + (size_t)b * row_stride + (size_t)h * D;
            orc_rmsnorm(v, v, gamma, D, eps);
            orc_rope(v, pos0 + b, rope_dim, inv);
        }
    free(inv);
}

/* ------------------------------------------------------------------ KV append
 * src/model.cpp:186-189 (per token) and src/cuda/model_cuda.cu:108-117 (per chunk):
 * cache row (pos0+b) of width kd receives the K (and V) slice of input row b. */
ORC_API void orc_kv_append(const float* k_src, const float* v_src, long src_stride, int rows, float* kc, float* vc,
                           int kd, int pos0) {
    for (int b = 0; b < rows; ++b) {
        memcpy(kc + (size_t)(pos0 + b) * kd, k_src + (size_t)b * src_stride, sizeof(float) * (size_t)kd);
        memcpy(vc + (size_t)(pos0 + b) * kd, v_src + (size_t)b * src_stride, sizeof(float) * (size_t)kd);
    }
}

/* ------------------------------------------------------------------ attention, one query row
 * src/model.cpp:191-214.  For each query head hd (OpenMP over heads):
 *   kvh = hd / group;  s_t = (sum_i q_i k_{t,i}) * scale  (sequential float);  mx = running max;
 *   e_t = exp(s_t - mx) (float);  sum = sum double(e_t);  inv = float(1/sum);
 *   out_i = sum_t (e_t * inv) * v_{t,i}, accumulated sequentially in t.
 * Cache layout [pos][HKV][D]; T = number of visible keys (pos+1).
 * `scores` is caller scratch of H*T floats (NULL -> allocated here). */
static void orc_attn_head(const float* q, const float* kc, const float* vc, float* out, int T, int kvh, int HKV,
                          int D, float scale, float* sc) {
    const size_t KD = (size_t)HKV * D;
    float mx = -INFINITY;
    for (int t = 0; t < T; ++t) {
        const float* k = kc + (size_t)t * KD + (size_t)kvh * D;
        float s = 0.f;
        for (int i = 0; i < D; ++i) s += q[i] * k[i];
        sc[t] = s * scale;
        if (sc[t] > mx) mx = sc[t];
    }
    double sum = 0.0;
    for (int t = 0; t < T; ++t) {
        sc[t] = expf(sc[t] - mx);
        sum += sc[t];
    }
    const float inv = (float)(1.0 / sum);
    for (int i = 0; i < D; ++i) out[i] = 0.f;
    for (int t = 0; t < T; ++t) {
        const float* v = vc + (size_t)t * KD + (size_t)kvh * D;
        const float p = sc[t] * inv;
        for (int i = 0; i < D; ++i) out[i] += p * v[i];
    }
}

ORC_API void orc_attn_decode(const float* q, const float* kc, const float* vc, float* out, int T, int H, int HKV,
                             int D, float scale, float* scores) {
    const int group = H / HKV;
    float* sc = scores ? scores : (float*)malloc(sizeof(float) * (size_t)H * (size_t)(T > 0 ? T : 1));
#pragma omp parallel for schedule(static)
    for (int hd = 0; hd < H; ++hd)
        orc_attn_head(q + (size_t)hd * D, kc, vc, out + (size_t)hd * D, T, hd / group, HKV, D, scale,
                      sc + (size_t)hd * T);
    if (!scores) free(sc);
}

/* Causal prefill as the reference CPU backend runs it: one token at a time
 * (src/model.cpp:138-140), query b at position pos0+b seeing keys 0..pos0+b.
 * q row b at q + b*q_stride; out row b at out + b*H*D. */
ORC_API void orc_attn_prefill(const float* q, long q_stride, const float* kc, const float* vc, float* out, int B,
                              int pos0, int H, int HKV, int D, float scale) {
    const int Tmax = pos0 + B;
    float* sc = (float*)malloc(sizeof(float) * (size_t)H * (size_t)(Tmax > 0 ? Tmax : 1));
    for (int b = 0; b < B; ++b)
        orc_attn_decode(q + (size_t)b * q_stride, kc, vc, out + (size_t)b * H * D, pos0 + b + 1, H, HKV, D, scale,
                        sc);
    free(sc);
}

/* Ragged multi-sequence decode: sequence s has its own cache rows starting at kv_offset[s]
 * (row = HKV*D floats) and kv_len[s] visible keys; each sequence is one orc_attn_decode. */
ORC_API void orc_attn_decode_batched(const float* q, const float* kc, const float* vc, float* out,
                                     const int64_t* kv_offset, const int* kv_len, int nseq, int H, int HKV, int D,
                                     float scale) {
    const size_t KD = (size_t)HKV * D;
    for (int s = 0; s < nseq; ++s)
        orc_attn_decode(q + (size_t)s * H * D, kc + (size_t)kv_offset[s] * KD, vc + (size_t)kv_offset[s] * KD,
                        out + (size_t)s * H * D, kv_len[s], H, HKV, D, scale, NULL);
}

/* ------------------------------------------------------------------ split-K restatement
 * src/cuda/model_cuda.cu:1043-1111 (k_attn_split + k_attn_combine): the T keys are cut into
 * nsplit chunks of ceil(T/nsplit); per chunk, 32-key tiles with a running (m, l, acc) and
 * expf; the combine takes M = max m_s, skips empty chunks (m = -inf) and returns
 * sum exp(m_s-M) acc_s / sum exp(m_s-M) l_s.  Scores use a plain sequential dot here (the
 * reference's lane-strided warp sum only changes rounding). */
ORC_API void orc_attn_split_combine(const float* q, const float* kc, const float* vc, float* out, int T, int H,
                                    int HKV, int D, float scale, int nsplit) {
    const int group = H / HKV;
    const size_t KD = (size_t)HKV * D;
    const int chunk = (T + nsplit - 1) / nsplit;
    float* pacc = (float*)malloc(sizeof(float) * (size_t)nsplit * D);
    float* pm = (float*)malloc(sizeof(float) * (size_t)nsplit);
    float* pl = (float*)malloc(sizeof(float) * (size_t)nsplit);
    float sc[32];
    for (int h = 0; h < H; ++h) {
        const float* qh = q + (size_t)h * D;
        const int kvh = h / group;
        for (int s = 0; s < nsplit; ++s) {
            const int tb = s * chunk, te = tb + chunk < T ? tb + chunk : T;
            float m = -INFINITY, l = 0.f;
            float* acc = pacc + (size_t)s * D;
            for (int i = 0; i < D; ++i) acc[i] = 0.f;
            for (int t0 = tb; t0 < te; t0 += 32) {
                float tm = -INFINITY;
                for (int j = 0; j < 32; ++j) {
                    const int t = t0 + j;
                    float sv = -INFINITY;
                    if (t < te) {
                        const float* k = kc + (size_t)t * KD + (size_t)kvh * D;
                        float p = 0.f;
                        for (int i = 0; i < D; ++i) p += qh[i] * k[i];
                        sv = p * scale;
                    }
                    sc[j] = sv;
                    tm = sv > tm ? sv : tm;
                }
                const float mn = m > tm ? m : tm;
                const float corr = expf(m - mn);
                l *= corr;
                for (int i = 0; i < D; ++i) acc[i] *= corr;
                const int lim = te - t0 < 32 ? te - t0 : 32;
                for (int j = 0; j < lim; ++j) {
                    const float p = expf(sc[j] - mn);
                    l += p;
                    const float* v = vc + (size_t)(t0 + j) * KD + (size_t)kvh * D;
                    for (int i = 0; i < D; ++i) acc[i] += p * v[i];
                }
                m = mn;
            }
            pm[s] = m;
            pl[s] = l;
        }
        float M = -INFINITY;
        for (int s = 0; s < nsplit; ++s) M = pm[s] > M ? pm[s] : M;
        for (int i = 0; i < D; ++i) {
            float lsum = 0.f, o = 0.f;
            for (int s = 0; s < nsplit; ++s) {
                if (pm[s] == -INFINITY) continue;
                const float w = expf(pm[s] - M);
                lsum += w * pl[s];
                o += w * pacc[(size_t)s * D + i];
            }
            out[(size_t)h * D + i] = o / lsum;
        }
    }
    free(pacc);
    free(pm);
    free(pl);
}

/* ------------------------------------------------------------------ QKV projection (matvec)
 * binary16 -> binary32, exact (what _mm_cvtph_ps does in f16_to_f32, src/ops.cpp:22-24):
 * normals rebias the exponent, subnormals are normalised, inf/NaN keep their payload. */
ORC_API float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {  /* subnormal: value man * 2^-24 */
        int e = -1;
        do {
            man <<= 1;
            ++e;
        } while (!(man & 0x400u));
        bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* hsum of an 8-lane float vector in the order of src/ops.cpp:84-90:
 * ((v0+v4) + (v2+v6)) + ((v1+v5) + (v3+v7)). */
static float orc_hsum8(const float* v) {
    float lo[4];
    for (int i = 0; i < 4; ++i) lo[i] = v[i] + v[i + 4];
    const float a = lo[0] + lo[2], b = lo[1] + lo[3];
    return a + b;
}

/* dot_f32 (src/ops.cpp:108-118): lanes k of two 8-wide FMA accumulators take elements
 * j+k and j+8+k of each 16-element block; then hsum(a0 + a1), then the scalar tail. */
ORC_API float orc_dot_f32(const float* w, const float* x, long n) {
    float a0[8] = {0}, a1[8] = {0}, v[8];
    long j = 0;
    for (; j + 16 <= n; j += 16)
        for (int k = 0; k < 8; ++k) {
            a0[k] = fmaf(w[j + k], x[j + k], a0[k]);
            a1[k] = fmaf(w[j + 8 + k], x[j + 8 + k], a1[k]);
        }
    for (int k = 0; k < 8; ++k) v[k] = a0[k] + a1[k];
    float s = orc_hsum8(v);
    for (; j < n; ++j) s += w[j] * x[j];
    return s;
}

/* dot_f16 (src/ops.cpp:92-106): four 8-wide FMA accumulators over 32-element blocks, then
 * 8-element blocks into a0; hsum((a0 + a1) + (a2 + a3)); the scalar tail converts each
 * weight and adds its product. */
ORC_API float orc_dot_f16(const uint16_t* w, const float* x, long n) {
    float a[4][8] = {{0}}, v[8];
    long j = 0;
    for (; j + 32 <= n; j += 32)
        for (int u = 0; u < 4; ++u)
            for (int k = 0; k < 8; ++k)
                a[u][k] = fmaf(orc_f16_to_f32(w[j + 8 * u + k]), x[j + 8 * u + k], a[u][k]);
    for (; j + 8 <= n; j += 8)
        for (int k = 0; k < 8; ++k) a[0][k] = fmaf(orc_f16_to_f32(w[j + k]), x[j + k], a[0][k]);
    for (int k = 0; k < 8; ++k) v[k] = (a[0][k] + a[1][k]) + (a[2][k] + a[3][k]);
    float s = orc_hsum8(v);
    for (; j < n; ++j) s += orc_f16_to_f32(w[j]) * x[j];
    return s;
}

/* ------------------------------------------------------------------ quantised rows
 * GGML block formats the reference computes with (src/quant.h:21-39), decoded to float in the
 * reference's operation order (src/quant.cpp:7-60); a row of n values is n / block_size blocks
 * one after another.
 *   Q8_0 (type 8):  32 values in 34 bytes: binary16 d, 32 int8 q;       y = q * d
 *   Q4_K (type 12): 256 values in 144 bytes: binary16 d, dmin, 12 bytes of packed 6-bit
 *                   (scale, min) for 8 sub-blocks of 32, 128 bytes of nibbles;
 *                   y = (d * sc) * q - dmin * m
 *   Q6_K (type 14): 256 values in 210 bytes: 128 bytes of low nibbles, 64 of high 2-bit
 *                   pairs, 16 int8 scales, binary16 d;  y = (d * sc) * (q - 32)          */
static uint16_t orc_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

ORC_API void orc_dequant_q8_0(const uint8_t* src, float* y, long n) {
    for (long b = 0; b < n / 32; ++b) {
        const uint8_t* blk = src + 34 * b;
        const float d = orc_f16_to_f32(orc_u16(blk));
        for (int j = 0; j < 32; ++j) y[32 * b + j] = (float)(int8_t)blk[2 + j] * d;
    }
}

/* the 6-bit scale and min of sub-block j (0..7) from the 12 packed bytes (src/quant.h:43-52):
 * j < 4 keeps the low 6 bits of bytes j and j+4; j >= 4 joins the nibbles of byte j+4 with the
 * top two bits of bytes j-4 (scale) and j (min) */
static void orc_q4k_sm(const uint8_t* q, int j, int* sc, int* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

ORC_API void orc_dequant_q4_K(const uint8_t* src, float* y, long n) {
    for (long b = 0; b < n / 256; ++b) {
        const uint8_t* blk = src + 144 * b;
        const float d = orc_f16_to_f32(orc_u16(blk)), dmin = orc_f16_to_f32(orc_u16(blk + 2));
        const uint8_t* packed = blk + 4;
        const uint8_t* qs = blk + 16;
        float* out = y + 256 * b;
        /* chunk c of 64 values: sub-block 2c from the low nibbles of 32 bytes, 2c+1 from their
         * high nibbles */
        for (int c = 0; c < 4; ++c) {
            for (int half = 0; half < 2; ++half) {
                int sc, m;
                orc_q4k_sm(packed, 2 * c + half, &sc, &m);
                const float dl = d * (float)sc, ml = dmin * (float)m;
                for (int l = 0; l < 32; ++l) {
                    const int q = half ? qs[32 * c + l] >> 4 : qs[32 * c + l] & 15;
                    out[64 * c + 32 * half + l] = dl * (float)q - ml;
                }
            }
        }
    }
}

ORC_API void orc_dequant_q6_K(const uint8_t* src, float* y, long n) {
    for (long b = 0; b < n / 256; ++b) {
        const uint8_t* blk = src + 210 * b;
        const float d = orc_f16_to_f32(orc_u16(blk + 208));
        float* out = y + 256 * b;
        /* value v = 128 h + 32 g + l (g = 0..3, l = 0..31): the low nibble (g = 0, 1) or the high
         * nibble (g = 2, 3) of ql[64 h + l + 32 (g & 1)], bits 2g, 2g+1 of qh[32 h + l] on top,
         * scale scales[8 h + l / 16 + 2 g] */
        for (int h = 0; h < 2; ++h)
            for (int g = 0; g < 4; ++g)
                for (int l = 0; l < 32; ++l) {
                    const uint8_t lo = blk[64 * h + l + 32 * (g & 1)];
                    const int nib = g < 2 ? lo & 15 : lo >> 4;
                    const int hi = (blk[128 + 32 * h + l] >> (2 * g)) & 3;
                    const int q = (nib | (hi << 4)) - 32;
                    const int sc = (int8_t)blk[192 + 8 * h + l / 16 + 2 * g];
                    out[128 * h + 32 * g + l] = d * (float)sc * (float)q;
                }
    }
}

/* bytes of one row of n values */
ORC_API long orc_row_bytes(int type, long n) {
    switch (type) {
        case 0: return 4 * n;
        case 1: return 2 * n;
        case 8: return n / 32 * 34;
        case 12: return n / 256 * 144;
        case 14: return n / 256 * 210;
        default: return 0;
    }
}

/* matvec (src/ops.cpp:126-153): y[r] = row r . x, rows stored one after another (GGUF ne[0] =
 * n is the contiguous dimension).  F32 (type 0) and F16 (type 1) rows go through dot_f32 /
 * dot_f16; quantised rows are decoded into a float buffer first, then dot_f32 (the reference's
 * convert_row + dot_f32 path). */
ORC_API void orc_matvec(int type, const void* w, const float* x, float* y, long rows, long n) {
    const long rb = orc_row_bytes(type, n);
#pragma omp parallel
    {
        float* buf = (type == 0 || type == 1) ? NULL : (float*)malloc((size_t)n * sizeof(float));
#pragma omp for schedule(static)
        for (long r = 0; r < rows; ++r) {
            const uint8_t* row = (const uint8_t*)w + r * rb;
            if (type == 0) y[r] = orc_dot_f32((const float*)row, x, n);
            else if (type == 1) y[r] = orc_dot_f16((const uint16_t*)row, x, n);
            else {
                if (type == 8) orc_dequant_q8_0(row, buf, n);
                else if (type == 12) orc_dequant_q4_K(row, buf, n);
                else orc_dequant_q6_K(row, buf, n);
                y[r] = orc_dot_f32(buf, x, n);
            }
        }
        free(buf);
    }
}

/* ------------------------------------------------------------------ float64 brute force
 * Textbook softmax attention for one query row with T visible keys, everything in double:
 * out_h = sum_t softmax_t(q_h . k_t * scale) v_t, GQA kvh = h / (H/HKV).  Used to measure
 * the fp32 paths' distance from exact arithmetic.  Writes double outputs. */
ORC_API void orc_attn_f64(const float* q, const float* kc, const float* vc, double* out, int T, int H, int HKV,
                          int D, double scale) {
    const int group = H / HKV;
    const size_t KD = (size_t)HKV * D;
    double* s = (double*)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
    for (int h = 0; h < H; ++h) {
        const int kvh = h / group;
        double mx = -INFINITY;
        for (int t = 0; t < T; ++t) {
            double a = 0.0;
            for (int i = 0; i < D; ++i) a += (double)q[(size_t)h * D + i] * kc[(size_t)t * KD + (size_t)kvh * D + i];
            s[t] = a * scale;
            if (s[t] > mx) mx = s[t];
        }
        double sum = 0.0;
        for (int t = 0; t < T; ++t) {
            s[t] = exp(s[t] - mx);
            sum += s[t];
        }
        for (int i = 0; i < D; ++i) {
            double o = 0.0;
            for (int t = 0; t < T; ++t) o += s[t] * vc[(size_t)t * KD + (size_t)kvh * D + i];
            out[(size_t)h * D + i] = o / sum;
        }
    }
    free(s);
}

ORC_API int orc_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

ORC_API void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
