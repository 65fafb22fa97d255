// prefill.hip — causal GQA prefill attention on gfx950 fp32 matrix cores.
//
// Contraction on v_mfma_f32_32x32x2_f32 (fp32 inputs, fp32 accumulate; 4096 FLOP per
// instruction), online softmax in fp32 VALU between the two products.
//
// Each wave owns 32 queries of one head.  It computes the transposed score tile
//     S^T[key][query] = K . Q^T          (A = K rows from LDS, B = Q^T held in registers)
// so that in the 32x32 accumulator layout every lane owns ONE query column and 16 key
// rows: the row max / row sum of the softmax need only the lane's own 16 values plus one
// exchange with lane^32.  The same registers, unchanged, are the B operand of
//     O^T[d][query] = V^T . P^T          (A = V columns from LDS)
// because the accumulator row order (8*(r/4) + 4*(lane/32) + r%4) is used as the
// contraction order of the second product.  The contraction order over d in the first
// product is (lane/32)*64 + step, so each lane's Q^T and K operands are 64 contiguous
// floats of one row.
//
// A workgroup holds GW = min(G, 4) waves, the GW query heads of one KV head that share
// every K/V tile: the tile (32 keys x 128 d of K and of V) is staged once into LDS,
// double-buffered, with the next tile's global loads in flight during the MFMA work.
// Causal balance: query block qb needs qb+1+pos0/32 tiles, so a workgroup runs block p
// and then block nb-1-p; every workgroup has the same amount of work.  Workgroup id
// L -> kv head L % HKV first, so with 8 KV heads all blocks of one KV head share an
// XCD (and its L2) under the round-robin XCD dispatch.
#include "common.h"
#include "launch.h"

namespace ei {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kQB = 32;           // queries per wave (and per block)
constexpr int kKT = 32;           // keys per tile
constexpr int kKS = kHeadDim + 4;  // K row stride in LDS (floats): conflict-free row-wise b128 reads
constexpr int kVS = kHeadDim + 8;  // V row stride in LDS: the two half-waves hit disjoint banks
constexpr int kTileFloats = kKT * kKS + kKT * kVS;
constexpr int kBufs = 3;  // LDS tile buffers (software pipeline depth)

template <int GW>
__global__ __launch_bounds__(64 * GW) void k_prefill(const float* __restrict__ q, long q_stride,
                                                     float* __restrict__ out, const float* __restrict__ kc,
                                                     const float* __restrict__ vc, const int* __restrict__ pos_dev,
                                                     int B, int H, int HKV, int GG, float scale) {
    constexpr int D = kHeadDim;
    constexpr int NT = 64 * GW;
    extern __shared__ __align__(16) float smem[];  // kBufs x [K tile | V tile]

    const int L = blockIdx.x;
    const int kvh = L % HKV;
    const int rest = L / HKV;
    const int hg = rest % GG;
    const int pair = rest / GG;
    const int G = GW * GG;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int col = lane & 31, hh = lane >> 5;
    const int h = kvh * G + hg * GW + w;
    const int pos0 = *pos_dev;
    const size_t KD = (size_t)HKV * D;
    const float* kbase = kc + (size_t)kvh * D;
    const float* vbase = vc + (size_t)kvh * D;
    const int nb = (B + kQB - 1) / kQB;

    for (int pass = 0; pass < 2; ++pass) {
        const int qb = pass == 0 ? pair : nb - 1 - pair;
        if (pass == 1 && qb == pair) break;
        const int b = qb * kQB + col;  // this lane's query row
        const int qpos = pos0 + b;

        // Q^T operand: q[b][h][hh*64 + kk], kk < 64
        float qreg[64];
        if (b < B) {
            const float* src = q + (size_t)b * q_stride + (size_t)h * D + hh * 64;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float4 v = *reinterpret_cast<const float4*>(src + 4 * i);
                qreg[4 * i] = v.x;
                qreg[4 * i + 1] = v.y;
                qreg[4 * i + 2] = v.z;
                qreg[4 * i + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 64; ++i) qreg[i] = 0.f;
        }

        floatx16 o[4];
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
        float m = -INFINITY, lsum = 0.f;

        const int T = pos0 + min(B, qb * kQB + kQB);  // keys seen by the block's last query
        const int ntile = (T + kKT - 1) / kKT;

        // cooperative tile staging: 32 rows x 32 float4 for K and for V
        constexpr int PER = kKT * (D / 4) / NT;
        float4 stk[PER], stv[PER];
        auto fetch = [&](int kt) {
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int i = tid + NT * j, row = i >> 5, c4 = (i & 31) * 4;
                const int t = kt * kKT + row;
                if (t < T) {
                    stk[j] = *reinterpret_cast<const float4*>(kbase + (size_t)t * KD + c4);
                    stv[j] = *reinterpret_cast<const float4*>(vbase + (size_t)t * KD + c4);
                } else {
                    stk[j] = make_float4(0.f, 0.f, 0.f, 0.f);
                    stv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
        };
        auto stash = [&](float* Ks) {
            float* Vs = Ks + kKT * kKS;
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int i = tid + NT * j, row = i >> 5, c4 = (i & 31) * 4;
                *reinterpret_cast<float4*>(Ks + row * kKS + c4) = stk[j];
                *reinterpret_cast<float4*>(Vs + row * kVS + c4) = stv[j];
            }
        };

        auto tile = [&](int kt) { return smem + (kt % kBufs) * kTileFloats; };
        const float sl2 = scale * 1.44269504088896340736f;  // scores in the exp2 domain

        // S^T = K . Q^T over d = hh*64 + kk for the K tile at Ks; the K operand of step
        // k4+1 is read while the four MFMAs of step k4 run
        auto qk = [&](const float* Ks) {
            floatx16 acc;
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = 0.f;
            const float* krow = Ks + col * kKS + hh * 64;
            float4 kv = *reinterpret_cast<const float4*>(krow);
#pragma unroll
            for (int k4 = 0; k4 < 16; ++k4) {
                const float4 kn = *reinterpret_cast<const float4*>(krow + 4 * ((k4 + 1) & 15));
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qreg[4 * k4 + 0], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qreg[4 * k4 + 1], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qreg[4 * k4 + 2], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qreg[4 * k4 + 3], acc, 0, 0, 0);
                kv = kn;
            }
            return acc;
        };
        // causal mask + online softmax of one score tile (VALU only): p replaces s, the
        // running (m, lsum) advance and O is rescaled.  Key of register r:
        // kt*32 + 8(r/4) + 4hh + r%4.
        auto softmax = [&](floatx16& sc, int kt) {
            const int kbase_t = kt * kKT + 4 * hh;
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kbase_t + 8 * (r >> 2) + (r & 3);
                const float sv = key <= qpos ? sc[r] * sl2 : -INFINITY;
                sc[r] = sv;
                mx = fmaxf(mx, sv);
            }
            mx = fmaxf(mx, lane_xor32(mx));
            const float mn = fmaxf(m, mx);
            const float base = mn == -INFINITY ? 0.f : mn;  // fully masked so far: keep exp finite
            const float corr = __builtin_amdgcn_exp2f(m - base);
            float ps = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                sc[r] = __builtin_amdgcn_exp2f(sc[r] - base);
                ps += sc[r];
            }
            lsum = lsum * corr + ps;
            m = mn;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[db][i] *= corr;
        };
        // O^T += V^T . P^T; contraction step r pairs keys 8(r/4) + r%4 (+4 for hh = 1)
        auto pv = [&](const floatx16& p, const float* Vs) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float* vrow = Vs + (8 * (r >> 2) + 4 * hh + (r & 3)) * kVS + col;
#pragma unroll
                for (int db = 0; db < 4; ++db)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * db], p[r], o[db], 0, 0, 0);
            }
        };

        // three LDS tile buffers: at step kt the V half of tile kt and the K half of tile
        // kt+1 are read while tile kt+2 is written; tile kt+3 travels in registers
        __syncthreads();  // previous pass finished reading every buffer
        fetch(0);
        stash(tile(0));
        if (ntile > 1) {
            fetch(1);
            stash(tile(1));
        }
        __syncthreads();
        if (ntile > 2) fetch(2);
        floatx16 s = qk(tile(0));

        for (int kt = 0; kt + 1 < ntile; ++kt) {
            // one basic block: the next tile's score MFMAs are interleaved with this
            // tile's softmax VALU work, then this tile's P.V MFMAs
            const floatx16 s_next = qk(tile(kt + 1));
            softmax(s, kt);
            pv(s, tile(kt) + kKT * kKS);
            // issue order: per K step 1 LDS read, 4 MFMAs, 8 VALU ops
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
            }
            if (kt + 2 < ntile) stash(tile(kt + 2));
            __syncthreads();
            if (kt + 3 < ntile) fetch(kt + 3);
            s = s_next;
        }
        softmax(s, ntile - 1);
        pv(s, tile(ntile - 1) + kKT * kKS);

        // ---- normalise and store: O^T register r of block db is d = 32db + 8(r/4) + 4hh + r%4
        lsum += lane_xor32(lsum);
        if (b < B) {
            float* dst = out + ((size_t)b * H + h) * D + 4 * hh;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    float4 v;
                    v.x = o[db][4 * r4 + 0] / lsum;
                    v.y = o[db][4 * r4 + 1] / lsum;
                    v.z = o[db][4 * r4 + 2] / lsum;
                    v.w = o[db][4 * r4 + 3] / lsum;
                    *reinterpret_cast<float4*>(dst + 32 * db + 8 * r4) = v;
                }
        }
    }
}

hipError_t launch_prefill(hipStream_t st, const float* q, long q_stride, float* out, const float* kc,
                          const float* vc, const int* pos_dev, int B, int H, int HKV, float scale) {
    const int G = H / HKV;
    const int GW = G < 4 ? G : 4;
    const int GG = G / GW;
    const int nb = (B + kQB - 1) / kQB;
    const int npairs = (nb + 1) / 2;
    const unsigned grid = (unsigned)npairs * HKV * GG;
    const size_t lds = kBufs * kTileFloats * sizeof(float);  // > 64 KB: opt in once per instantiation
    static bool opted[3] = {false, false, false};
    const int oi = GW == 1 ? 0 : GW == 2 ? 1 : 2;
    if (!opted[oi]) {
        hipError_t e = GW == 1   ? hipFuncSetAttribute((const void*)k_prefill<1>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds)
                       : GW == 2 ? hipFuncSetAttribute((const void*)k_prefill<2>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds)
                                 : hipFuncSetAttribute((const void*)k_prefill<4>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        opted[oi] = true;
    }
    switch (GW) {
        case 1: k_prefill<1><<<grid, 64, lds, st>>>(q, q_stride, out, kc, vc, pos_dev, B, H, HKV, GG, scale); break;
        case 2: k_prefill<2><<<grid, 128, lds, st>>>(q, q_stride, out, kc, vc, pos_dev, B, H, HKV, GG, scale); break;
        case 4: k_prefill<4><<<grid, 256, lds, st>>>(q, q_stride, out, kc, vc, pos_dev, B, H, HKV, GG, scale); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace ei
