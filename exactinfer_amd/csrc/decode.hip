// decode.hip — split-K decode attention for gfx950 (one query token per sequence).
//
// Work decomposition: grid (nsplit, HKV, n_seq), 256 threads.  A workgroup owns one KV
// head of one sequence and one chunk of keys, and serves all G = H/HKV query heads of
// that GQA group from the same K/V bytes (the reference re-reads K/V once per query head,
// src/cuda/model_cuda.cu:1051, :1066).  The chunk is walked in 64-key sub-tiles:
//
//   K phase   wave w scores keys 16w..16w+15 of the sub-tile.  Lane (r = l/8, c = l%8)
//             loads float4s of rows r and r+8 at d = 4c + 32i (i < 4): every load
//             instruction covers 8 rows x 128 contiguous bytes.  The 8 lanes of a row
//             hold partial dots for (2 rows x G heads); a transposing butterfly over
//             lanes xor 1/2/4 leaves one finished score per lane (7 exchanges for G=4).
//   softmax   scores go through LDS; every wave takes the sub-tile max per head with a
//             64-lane reduction (lane = key), rescales its running (m, l, acc) and writes
//             p = exp(s - m) to a wave-private LDS row.
//   V phase   wave w owns d in [32w, 32w+32) for all 64 keys: lane (r, c) loads
//             V[r + 8i][32w + 4c ..+4] (8 rows x 128 B per instruction) and accumulates
//             p * v for the G heads.
//
// Every K and V byte is loaded exactly once per launch, with 128-byte coalesced wavefront
// loads; K and V for a sub-tile are issued together so a workgroup has 64 KB in flight.
//
// Split combine: each workgroup writes its unnormalised partial (m, l, acc[G][128]); the
// last workgroup of a (sequence, kv head) to arrive (device-scope counter) merges them,
// o = sum_s e^(m_s-M) acc_s / sum_s e^(m_s-M) l_s, skipping empty splits, and re-arms the
// counter (src/cuda/model_cuda.cu:1097-1111 semantics, one launch instead of two).
//
// Fused variant: the workgroup also applies QK-norm + RoPE to its G query heads, and the
// workgroup whose chunk holds the new position writes the normed K row and the V row to
// the cache and scores that key from LDS.
#include "common.h"
#include "launch.h"

namespace ei {

constexpr int kThreads = 256;
constexpr int kSub = 64;  // keys per sub-tile

// Transposing butterfly over the 8 lanes c = lane%8 (masks 1, 2, 4).  At each step a
// lane keeps one half of its array and receives the partner's copy of that half, so N
// values are reduced with N/2 + N/4 + ... exchanges instead of 3N.  When fewer than 2
// values remain the step is a plain butterfly (both partners end with the same sum).
template <int M, int N>
__device__ __forceinline__ void xstep(float* v, bool up) {
    if constexpr (N > 1) {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) {
            const float send = up ? v[i] : v[i + N / 2];
            const float keep = up ? v[i + N / 2] : v[i];
            v[i] = keep + lane_xor<M>(send);
        }
    } else {
        v[0] += lane_xor<M>(v[0]);
    }
}

template <int N>
struct Halve {
    static constexpr int value = N > 1 ? N / 2 : 1;
};

// After xreduce8<N>, v[k] (k < max(N/8,1)) holds the full 8-lane sum of original index
// xreduce8_index<N>(c) + k.
template <int N>
__device__ __forceinline__ void xreduce8(float* v, int c) {
    constexpr int N1 = Halve<N>::value, N2 = Halve<N1>::value;
    xstep<1, N>(v, c & 1);
    xstep<2, N1>(v, c & 2);
    xstep<4, N2>(v, c & 4);
}

template <int N>
__device__ __forceinline__ int xreduce8_index(int c) {
    int base = 0, n = N;
#pragma unroll
    for (int m = 1; m <= 4; m <<= 1) {
        if (n > 1) {
            if (c & m) base += n / 2;
            n /= 2;
        }
    }
    return base;
}

__device__ __forceinline__ float dot4(const float4 a, const float4 b, float acc) {
    acc = fmaf(a.x, b.x, acc);
    acc = fmaf(a.y, b.y, acc);
    acc = fmaf(a.z, b.z, acc);
    return fmaf(a.w, b.w, acc);
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

template <int G, bool FUSED>
__global__ __launch_bounds__(kThreads) void k_decode(const DecodeArgs a) {
    constexpr int D = kHeadDim;
    constexpr int NV = 2 * G;                     // partial dots per lane in the K phase
    constexpr int NF = NV / 8 > 0 ? NV / 8 : 1;   // finished scores per lane after xreduce8
    __shared__ __align__(16) float qs[G * D];
    __shared__ __align__(16) float sc[kSub * G];
    __shared__ __align__(16) float pw[4][kSub * G];
    __shared__ __align__(16) float knew[4][D];   // fused: [0] normed K row, [1] V row, [2..3] scratch
    __shared__ float red[4][2 * G];
    __shared__ float wts[kDecodeMaxSplits * G];
    __shared__ float4 ored[kThreads];
    __shared__ int s_last;

    const int split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane >> 3, c = lane & 7;
    const int len = a.kv_len ? a.kv_len[seq] : (*a.pos_dev + 1);
    const size_t KD = (size_t)a.HKV * D;
    const size_t row0 = a.kv_offset ? (size_t)a.kv_offset[seq] : 0;
    float* kbase = a.kc + row0 * KD + (size_t)kvh * D;
    float* vbase = a.vc + row0 * KD + (size_t)kvh * D;
    const int t_begin = split * a.chunk;
    const int t_end = min(len, t_begin + a.chunk);
    const int pos = len - 1;
    const float* qrow = a.q + (size_t)seq * a.q_stride;
    const int h0 = kvh * G;

    bool owner = false;
    if constexpr (FUSED) {
        const float2* cs_row = a.cs + (size_t)pos * (a.rope_dim >> 1);
        for (int g = w; g < G; g += 4) {
            float o0, o1;
            norm_rope_head(qrow + (size_t)(h0 + g) * D, a.q_gamma, cs_row, a.rope_dim, a.eps, qs + g * D, lane,
                           &o0, &o1);
            qs[g * D + lane] = o0;
            qs[g * D + lane + 64] = o1;
        }
        owner = t_begin <= pos && pos < t_end;
        if (owner) {
            const float* krow = qrow + (size_t)a.H * D + (size_t)kvh * D;
            const float* vrow = qrow + (size_t)(a.H + a.HKV) * D + (size_t)kvh * D;
            if (w == 0) {
                float o0, o1;
                norm_rope_head(krow, a.k_gamma, cs_row, a.rope_dim, a.eps, knew[2], lane, &o0, &o1);
                knew[0][lane] = o0;
                knew[0][lane + 64] = o1;
            } else if (w == 1) {
                knew[1][lane] = vrow[lane];
                knew[1][lane + 64] = vrow[lane + 64];
            }
        }
        __syncthreads();
        if (owner && tid < 2 * D) {
            float* dst = (tid < D ? kbase : vbase) + (size_t)pos * KD + (tid & (D - 1));
            *dst = knew[tid >> 7][tid & (D - 1)];
        }
    } else {
        for (int i = tid; i < G * D; i += kThreads) qs[i] = qrow[(size_t)h0 * D + i];
        __syncthreads();
    }

    float4 qreg[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) qreg[g][i] = *reinterpret_cast<const float4*>(qs + g * D + 4 * c + 32 * i);

    float m[G], l[G];
    float4 acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
        acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const int sidx = xreduce8_index<NV>(c);

    for (int t0 = t_begin; t0 < t_end; t0 += kSub) {
        // ---- issue K and V loads of the sub-tile
        float4 kr[2][4], vr[8];
        bool kval[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int tk = t0 + 16 * w + 8 * j + r;
            kval[j] = tk < t_end;
            const float* src = kbase + (size_t)tk * KD + 4 * c;
#pragma unroll
            for (int i = 0; i < 4; ++i) kr[j][i] = kval[j] ? ld4(src + 32 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int tv = t0 + r + 8 * i;
            vr[i] = tv < t_end ? ld4(vbase + (size_t)tv * KD + 32 * w + 4 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if constexpr (FUSED) {
            if (owner) {  // the new row: use the LDS copy, not the (possibly stale) loaded bytes
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    if (t0 + 16 * w + 8 * j + r == pos)
#pragma unroll
                        for (int i = 0; i < 4; ++i) kr[j][i] = *reinterpret_cast<const float4*>(&knew[0][4 * c + 32 * i]);
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (t0 + r + 8 * i == pos) vr[i] = *reinterpret_cast<const float4*>(&knew[1][32 * w + 4 * c]);
            }
        }

        // ---- scores: partial dots, 8-lane transposing reduction, to LDS
        float part[NV];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) s = dot4(qreg[g][i], kr[j][i], s);
                part[j * G + g] = s;
            }
        xreduce8<NV>(part, c);
#pragma unroll
        for (int k = 0; k < NF; ++k) {
            const int idx = sidx + k;
            const int j = idx / G, g = idx % G;
            const bool valid = j == 0 ? kval[0] : kval[1];
            sc[(16 * w + 8 * j + r) * G + g] = valid ? part[k] * a.scale : -INFINITY;
        }
        __syncthreads();

        // ---- online softmax over the sub-tile (lane = key slot), identical in every wave
        float p[G], corr[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float sv = sc[lane * G + g];
            const float mt = wave_max(sv);
            const float mn = fmaxf(m[g], mt);  // finite: the sub-tile holds at least one key
            corr[g] = expf(m[g] - mn);
            p[g] = expf(sv - mn);
            l[g] = l[g] * corr[g] + p[g];
            m[g] = mn;
            pw[w][lane * G + g] = p[g];
            acc[g].x *= corr[g];
            acc[g].y *= corr[g];
            acc[g].z *= corr[g];
            acc[g].w *= corr[g];
        }
        __builtin_amdgcn_wave_barrier();

        // ---- V phase: acc[g][d] += p[key][g] * V[key][d], d = 32w + 4c .. +4
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float* pk = &pw[w][(r + 8 * i) * G];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float pv = pk[g];
                acc[g].x = fmaf(pv, vr[i].x, acc[g].x);
                acc[g].y = fmaf(pv, vr[i].y, acc[g].y);
                acc[g].z = fmaf(pv, vr[i].z, acc[g].z);
                acc[g].w = fmaf(pv, vr[i].w, acc[g].w);
            }
        }
        __syncthreads();  // sc and pw are rewritten by the next sub-tile
    }

    // ---- chunk partial: sum acc over the 8 key rows (lanes xor 8/16/32), l over 64 slots
#pragma unroll
    for (int g = 0; g < G; ++g) {
        acc[g].x += lane_xor8(acc[g].x);
        acc[g].y += lane_xor8(acc[g].y);
        acc[g].z += lane_xor8(acc[g].z);
        acc[g].w += lane_xor8(acc[g].w);
        acc[g].x += lane_xor16(acc[g].x);
        acc[g].y += lane_xor16(acc[g].y);
        acc[g].z += lane_xor16(acc[g].z);
        acc[g].w += lane_xor16(acc[g].w);
        acc[g].x += lane_xor32(acc[g].x);
        acc[g].y += lane_xor32(acc[g].y);
        acc[g].z += lane_xor32(acc[g].z);
        acc[g].w += lane_xor32(acc[g].w);
        l[g] = wave_sum(l[g]);
    }
    const size_t head_slot = (size_t)seq * a.HKV + kvh;
    const size_t slot = head_slot * a.nsplit + split;
    float* pacc = a.part_acc + slot * G * D;
    if (lane < 8) {
#pragma unroll
        for (int g = 0; g < G; ++g) *reinterpret_cast<float4*>(pacc + g * D + 32 * w + 4 * c) = acc[g];
    }
    if (tid < G) {
        a.part_ml[(slot * G + tid) * 2 + 0] = m[tid];
        a.part_ml[(slot * G + tid) * 2 + 1] = l[tid];
    }

    // ---- arrival; the last workgroup of this (sequence, kv head) merges the splits
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(&a.counters[head_slot], 1u) == (unsigned)(a.nsplit - 1);
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    const int S = a.nsplit;
    const float* pml = a.part_ml + head_slot * S * G * 2;
    const float* pa = a.part_acc + head_slot * S * G * D;
    float M[G], L[G];
#pragma unroll
    for (int g = 0; g < G; ++g) M[g] = -INFINITY;
    for (int s = tid; s < S; s += kThreads)
#pragma unroll
        for (int g = 0; g < G; ++g) M[g] = fmaxf(M[g], pml[(s * G + g) * 2]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        M[g] = wave_max(M[g]);
        if (lane == 0) red[w][g] = M[g];
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) M[g] = fmaxf(fmaxf(red[0][g], red[1][g]), fmaxf(red[2][g], red[3][g]));
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) L[g] = 0.f;
    for (int s = tid; s < S; s += kThreads)
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float ms = pml[(s * G + g) * 2], ls = pml[(s * G + g) * 2 + 1];
            const float wv = ms == -INFINITY ? 0.f : expf(ms - M[g]);  // empty split: skipped
            wts[s * G + g] = wv;
            L[g] = fmaf(wv, ls, L[g]);
        }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        L[g] = wave_sum(L[g]);
        if (lane == 0) red[w][G + g] = L[g];
    }
    __syncthreads();

    // outputs: G*32 float4 columns; kThreads/(G*32) threads share a column over the splits
    constexpr int NCOL = G * 32, NPART = kThreads / NCOL > 0 ? kThreads / NCOL : 1;
    {
        const int col = tid % NCOL, part = tid / NCOL;
        if (part < NPART) {
            const int g = col / 32, d4 = col % 32;
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int s = part; s < S; s += NPART) {
                const float wv = wts[s * G + g];
                if (wv != 0.f) {
                    const float4 v = ld4(pa + ((size_t)s * G + g) * D + 4 * d4);
                    o.x = fmaf(wv, v.x, o.x);
                    o.y = fmaf(wv, v.y, o.y);
                    o.z = fmaf(wv, v.z, o.z);
                    o.w = fmaf(wv, v.w, o.w);
                }
            }
            ored[part * NCOL + col] = o;
        }
    }
    __syncthreads();
    if (tid < NCOL) {
        const int g = tid / 32, d4 = tid % 32;
        float4 o = ored[tid];
        for (int part = 1; part < NPART; ++part) {
            const float4 v = ored[part * NCOL + tid];
            o.x += v.x;
            o.y += v.y;
            o.z += v.z;
            o.w += v.w;
        }
        const float Lg = red[0][G + g] + red[1][G + g] + red[2][G + g] + red[3][G + g];
        o.x /= Lg;
        o.y /= Lg;
        o.z /= Lg;
        o.w /= Lg;
        *reinterpret_cast<float4*>(a.out + (size_t)seq * a.H * D + (size_t)(h0 + g) * D + 4 * d4) = o;
    }
    if (tid == 0) a.counters[head_slot] = 0u;  // re-arm for the next call
}

__global__ void k_ws_clear(uint32_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

// ------------------------------------------------------------------ host side
DecodePlan decode_plan(int n_seq, int HKV, int max_kv) {
    // Smallest chunk (multiple of the 64-key sub-tile) that keeps the split count within
    // the combine's LDS table and the total grid (empty splits included) bounded.
    int chunk = kSub;
    for (;;) {
        const long ns = ((long)max_kv + chunk - 1) / chunk;
        if (ns <= kDecodeMaxSplits && (long)n_seq * HKV * ns <= 32768) break;
        chunk *= 2;
    }
    DecodePlan p;
    p.chunk = chunk;
    p.nsplit = (max_kv + chunk - 1) / chunk;
    if (p.nsplit < 1) p.nsplit = 1;
    return p;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t decode_ws_bytes(int n_seq, int H, int HKV, int max_kv) {
    const DecodePlan p = decode_plan(n_seq, HKV, max_kv);
    const size_t slots = (size_t)n_seq * HKV * p.nsplit;
    const int G = H / HKV;
    return align256(slots * G * kHeadDim * 4) + align256(slots * G * 2 * 4) + align256((size_t)n_seq * HKV * 4);
}

template <int G>
static void launch_g(hipStream_t st, const DecodeArgs& a, int n_seq, bool fused) {
    const dim3 grid(a.nsplit, a.HKV, n_seq);
    if (fused) k_decode<G, true><<<grid, kThreads, 0, st>>>(a);
    else k_decode<G, false><<<grid, kThreads, 0, st>>>(a);
}

hipError_t launch_decode(hipStream_t st, const DecodeArgs& a, int n_seq, bool fused) {
    switch (a.H / a.HKV) {
        case 1: launch_g<1>(st, a, n_seq, fused); break;
        case 2: launch_g<2>(st, a, n_seq, fused); break;
        case 4: launch_g<4>(st, a, n_seq, fused); break;
        case 8: launch_g<8>(st, a, n_seq, fused); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_ws_clear(hipStream_t st, void* ws, size_t bytes) {
    const size_t n = bytes / 4;
    if (n == 0) return hipSuccess;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    k_ws_clear<<<(unsigned)blocks, 256, 0, st>>>(static_cast<uint32_t*>(ws), n);
    return hipGetLastError();
}

}  // namespace ei
