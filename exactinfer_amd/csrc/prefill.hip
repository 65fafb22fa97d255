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
//     O^T[d][query] = V^T . P^T          (A = V from LDS)
// because the accumulator row order (8*(r/4) + 4*(lane/32) + r%4) is used as the
// contraction order of the second product.  In the first product, step 4*k4 + j of lane
// half hh contracts d = 8*k4 + 4*hh + j.
// Output block db (0..3) of O^T holds d = 4*i + db for accumulator row i, so the A operand
// of all four blocks for one key is a single 16-byte LDS read V[key][4*lane .. 4*lane+3].
//
// Workgroup = KS key groups x 4 query slots of one KV head.  A slot is one (query block,
// head) pair; slots are numbered s = qb*G + g over the G heads that share the KV head, and
// unit U of a KV head holds slots 4U..4U+3.  For G = 4 a unit is the four heads of one
// block, for G = 8 half of them, for G = 2 two heads of two neighbouring blocks, for G = 1
// four neighbouring blocks of the head, for odd G at most two neighbouring blocks: every
// wave of the unit shares every K/V tile, and the unit's key range ends at its last
// block's diagonal (a wave of an earlier block masks the few tiles past its own).  Slots
// past the last block are idle waves (zero queries, no output).  Key group g takes the
// tiles kt = KS*i + g of the unit's causal range and keeps its own (m, l, O); the groups
// merge through LDS at the end of the unit.  With KS = 2 every SIMD runs two waves whose
// matrix streams interleave: one streams while the other waits on LDS or the per-tile
// barrier (their VALU work still adds to the matrix time: on this part a wave's fp32 MFMA
// stream holds the SIMD's issue).  Inside a wave's stream the next score chain alternates
// with this tile's P.V chains, and the next tiles' DMA instructions are issued between them
// (VMEM work outside the stream idles the pipe).  When one unit pair per KV head would not
// fill the CUs (short chunks at long positions, GQA groups under 4 heads;
// ei_attn_prefill_split) the pair's key tiles are split over ksplit workgroups of equal cost
// (a share that crosses from one unit to the other pays a second pass), whose unnormalised
// shares k_prefill_combine merges.
//
// K/V tiles (32 keys) reach LDS by LDS DMA (global_load_lds_dwordx4) straight from the
// cache, two tiles ahead for K and one for V, per key group:
//   K tile row-major, rows padded to 132 floats: the 32 lanes reading one 16-byte d-chunk
//     of 32 different keys hit 32 distinct bank quads; each row is one 32-lane DMA
//     instruction (a contiguous 512-byte global read: LDS DMA of 16-byte pieces gathered
//     from many rows runs ~3.5x slower per CU than contiguous DMA);
//   V tile row-major    [32 keys][128 floats], two rows per 64-lane DMA instruction.
// Rows past the causal end are clamped to the last visible row (valid memory, masked out).
// q and the output pass through LDS too, so that global memory sees whole 512-byte rows:
// at the start of each unit the workgroup DMAs its 128 query rows (once, for both key
// groups) into a padded staging area and each wave reads its Q^T operand from there; at the
// end the finished rows are written there in row order and stored two rows per instruction.
// (Gathering q straight into registers, 32 bytes per row per instruction, twice, and storing
// 8-byte pieces of 32 rows per instruction held each pass up for several microseconds.)
//
// Softmax runs in the exp2 domain (scores x scale x log2 e, one FMA per score).  The
// running maximum is raised only when a tile's maximum exceeds it by more than kLazy
// (log2 units), so P <= 2^kLazy and O / l are rescaled rarely; the result is the same
// softmax (the common factor cancels in O / l).  The causal mask is applied only on the
// (at most two) tiles that cross the block's diagonal.
//
// Causal balance: unit U needs about (4U+4)/G + pos0/32 tiles, so a workgroup runs unit p
// and then unit nu-1-p; every workgroup has the same amount of work.  Workgroup id
// L -> kv head L % HKV first, so with 8 KV heads all blocks of one KV head share an
// XCD (and its L2) under the round-robin XCD dispatch.
#include <cstdlib>

#include "common.h"
#include "launch.h"

namespace ei {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kQB = 32;                          // queries per wave (and per block)
constexpr int kKT = 32;                          // keys per tile
constexpr int kKS_F = kHeadDim + 4;             // padded K row (floats)
constexpr int kKTileF = kKT * kKS_F;             // floats in one K tile
constexpr int kVTileF = kKT * kHeadDim;          // floats in one V tile (16 KB)
constexpr int kGroupF = 2 * kKTileF + 2 * kVTileF;  // per key group: 2 K + 2 V tile buffers
constexpr int kKS = 2;                           // key groups per workgroup
constexpr float kLazy = 8.f;                     // lazy-rescale threshold (log2 units)
constexpr int kXchF = 34;                        // floats per lane exchanged by the merge
constexpr int kSlots = 4;                        // query slots (waves) per key group
constexpr int kPassTiles = 3;                    // a pass's fixed cost, in tiles (key-share balance; 1..4 tried)

// n / d for small d (1..8) and n * d < 2^32 as one multiply-high: the per-pass index math
// runs on the scalar unit, which the eight waves of a CU share, so a division loop per use
// would cost thousands of cycles per pass.  m = ceil(2^32 / d); d = 1 is taken as is.
struct FastDiv {
    uint32_t m, d;
};
__device__ __forceinline__ FastDiv fast_div(uint32_t d) { return {d == 1 ? 0u : 0xFFFFFFFFu / d + 1u, d}; }
__device__ __forceinline__ int fdiv(int n, FastDiv f) {
    return f.d == 1 ? n : (int)__umulhi((uint32_t)n, f.m);
}
// Key shares.  A workgroup runs units `pair` and nu-1-pair (causal balance).  With ksplit
// shares, the pair's tiles, unit pair's then unit nu-1-pair's, are cut into ksplit contiguous
// shares of equal cost, where the boundary between the units counts as kPassTiles extra tiles:
// a share that crosses it runs two passes (q staging, first tiles, key-group merge and store
// twice), so it gets that many fewer tiles, and every other share runs one pass.  Share
// `split` holds tiles [lo0, lo0 + r0) of unit pair and [lo1, lo1 + r1) of unit nu-1-pair; a
// unit without tiles in a share has no pass there and no partial, and k_prefill_combine,
// which evaluates the same cut, does not read one.  With ksplit = 1 the share is both units.
__device__ __forceinline__ int prefill_unit_tiles(int u, int pos0, int B, int nslot, FastDiv fG) {
    const int ql = fdiv(min(kSlots * u + kSlots - 1, nslot - 1), fG);  // the unit's last block
    return (pos0 + min(B, ql * kQB + kQB) + kKT - 1) / kKT;
}
__device__ __forceinline__ void prefill_share(int pair, int u_second, int split, FastDiv fK, int pos0, int B,
                                              int nslot, FastDiv fG, int& lo0, int& r0, int& lo1, int& r1) {
    const int n0 = prefill_unit_tiles(pair, pos0, B, nslot, fG);
    const int n1 = u_second != pair ? prefill_unit_tiles(u_second, pos0, B, nslot, fG) : 0;
    const int pen = n1 > 0 ? kPassTiles : 0;
    const int n_all = n0 + n1 + pen;
    auto real_tile = [&](int x) { return x <= n0 ? x : (x <= n0 + pen ? n0 : x - pen); };
    const int lo = real_tile(fdiv(split * n_all, fK)), hi = real_tile(fdiv((split + 1) * n_all, fK));
    lo0 = lo;
    r0 = max(min(hi, n0) - lo, 0);
    lo1 = max(lo, n0) - n0;
    r1 = max(hi - max(lo, n0), 0);
}

// LDS (plain kernel): the four K tile buffers (two per key group) from 0; the merge exchange
// area from 0 as well (used only after the unit's last tile); the four V tile buffers and,
// overlapping them, the q staging area (the unit's 4 x 32 query rows, padded like K rows)
// after the exchange area.  A unit's q rows and its first two K tiles land at the same time;
// its first V tile is fetched once q has moved to registers.  (The kernel that norms q keeps
// each key group's K0 K1 V0 V1 side by side from 0, and fetches the tiles after q.)
constexpr int kQStageF = 2 * kSlots * kXchF * 64;
constexpr int kVBaseF = kQStageF;
constexpr int kLdsF = kQStageF + kSlots * kQB * kKS_F;
static_assert(kKS * 2 * kKTileF <= kVBaseF, "K buffers below the V buffers and the q staging area");
static_assert(kVBaseF + kKS * 2 * kVTileF <= kLdsF, "V buffers within the staging span");
static_assert(kKS * kGroupF <= kLdsF, "grouped layout within the LDS budget");

// QK-norm + RoPE of one q row in LDS (rope_dim = 128), eight lanes per row: lane k of the row
// holds elements 8k..8k+7 and their rotate-half partners 64+8k..64+8k+7.  Same arithmetic as the
// prologue's head-norm, which follows the reference CPU path (rmsnorm, src/ops.cpp:155-160; rope,
// src/model.cpp:23-32): sum of squares in double, inv = float(1/sqrt(ss/128 + eps)),
// y = (x*inv)*gamma, then (y_e, y_e+64) -> (y_e c - y_e+64 s, y_e s + y_e+64 c).  The double sum runs over the eight
// lanes' partial sums (a different order of exact products than the prologue's lane pairs; the
// float result is the same unless the double rounds across a float boundary).
__device__ __forceinline__ void norm_rope_q8(float* row, const float (&g)[16], const float4 (&t)[4], float eps,
                                             int k) {
#pragma clang fp contract(off)
    float x[16];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float4 a = *reinterpret_cast<const float4*>(row + 8 * k + 4 * i);
        const float4 b = *reinterpret_cast<const float4*>(row + 64 + 8 * k + 4 * i);
        x[4 * i] = a.x, x[4 * i + 1] = a.y, x[4 * i + 2] = a.z, x[4 * i + 3] = a.w;
        x[8 + 4 * i] = b.x, x[8 + 4 * i + 1] = b.y, x[8 + 4 * i + 2] = b.z, x[8 + 4 * i + 3] = b.w;
    }
    // float x float is exact in double, so fma(x, x, ss) rounds like ss + x*x
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < 16; ++i) ss = __builtin_fma((double)x[i], (double)x[i], ss);
    ss += lane_xor_f64<1>(ss);
    ss += lane_xor_f64<2>(ss);
    ss += lane_xor_f64<4>(ss);
    const float inv = (float)(1.0 / sqrt(ss / (double)kHeadDim + (double)eps));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float c = (i & 1) ? t[i >> 1].z : t[i >> 1].x, sn = (i & 1) ? t[i >> 1].w : t[i >> 1].y;
        const float a = (x[i] * inv) * g[i];
        const float b = (x[8 + i] * inv) * g[8 + i];
        const float acs = a * c, bsn = b * sn;
        const float asn = a * sn, bcs = b * c;
        x[i] = acs - bsn;
        x[8 + i] = asn + bcs;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        *reinterpret_cast<float4*>(row + 8 * k + 4 * i) = make_float4(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
        *reinterpret_cast<float4*>(row + 64 + 8 * k + 4 * i) =
            make_float4(x[8 + 4 * i], x[8 + 4 * i + 1], x[8 + 4 * i + 2], x[8 + 4 * i + 3]);
    }
}

#ifdef EI_EXP_STAMPS
__device__ unsigned long long g_pstamps[4096 * 16];
#define PSTAMP(i) do { if (threadIdx.x == 0) g_pstamps[blockIdx.x * 16 + (i)] = __builtin_amdgcn_s_memtime(); } while (0)
#define PSTAMPV(i, v) do { if (threadIdx.x == 0) g_pstamps[blockIdx.x * 16 + (i)] = (unsigned long long)(v); } while (0)
#else
#define PSTAMP(i) do { } while (0)
#define PSTAMPV(i, v) do { } while (0)
#endif

// kPaged: key t of the sequence sits in pool row btab[t >> bshift] << bshift | (t & mask), the
// block size 2^bshift >= 32, so a 32-key tile lies in one block and its rows are consecutive.
template <bool kNormQ, bool kPaged, bool kEarlyK = false>
__global__ __launch_bounds__(64 * kSlots * kKS) void k_prefill(const float* __restrict__ q, long q_stride,
                                                           float* __restrict__ out, const float* __restrict__ kc,
                                                           const float* __restrict__ vc,
                                                           const int* __restrict__ pos_dev, int B, int H, int HKV,
                                                           float scale, int ksplit,
                                                           float* __restrict__ part_o, float* __restrict__ part_ml,
                                                           const float* __restrict__ q_gamma,
                                                           const float2* __restrict__ cs, float eps,
                                                           const int* __restrict__ btab, int bshift,
                                                           int max_blocks) {
    constexpr int D = kHeadDim;
    constexpr int GW = kSlots;
    constexpr int DMA_PER_WAVE = 16 / GW;  // V DMA instructions per wave per tile (K: twice as many, 32 lanes each)
    extern __shared__ __align__(16) float smem[];

    PSTAMP(0);
    const int L = blockIdx.x;
    const int kvh = L % HKV;
    const int rest = L / HKV;
    const int split = rest % ksplit;  // which contiguous share of each unit's key tiles
    const int pair = rest / ksplit;
    const int G = H / HKV;
    const FastDiv fG = fast_div((uint32_t)G), fK = fast_div((uint32_t)ksplit);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wu = __builtin_amdgcn_readfirstlane(w);  // wave-uniform: keeps the branches scalar
    const int hw = wu % GW, grp = wu / GW;
    const int col = lane & 31, hh = lane >> 5;
    const int pos0 = *pos_dev;
    const size_t KD = (size_t)HKV * D;
    const float* kbase = kc + (size_t)kvh * D;
    const float* vbase = vc + (size_t)kvh * D;
    const uint64_t kb_bytes = (uint64_t)(uintptr_t)kbase, vb_bytes = (uint64_t)(uintptr_t)vbase;
    const uint32_t row_bytes = (uint32_t)(KD * sizeof(float));          // one cache row (all KV heads)
    // cache row of key t (wave-uniform t: one scalar load of the block table when paged)
    auto crow = [&](int t) -> uint32_t {
        // (a key past the table's blocks, outside the contract, reads the last entry: no fault)
        if constexpr (kPaged)
            return ((uint32_t)btab[min(t >> bshift, max_blocks - 1)] << bshift) | ((uint32_t)t & ((1u << bshift) - 1u));
        else return (uint32_t)t;
    };
    const uint32_t voff_k = 16u * col;                                  // K: lanes 0..31, one row
    const uint32_t voff_v = (uint32_t)hh * row_bytes + 16u * col;        // V: two rows per instruction
    const int nb = (B + kQB - 1) / kQB;
    const int nslot = G * nb;                    // (block, head) slots of this KV head
    const int nu = (nslot + kSlots - 1) / kSlots;  // units
    // this key group's K0 K1 and V0 V1: K buffers below the staging area for the plain kernel,
    // which fetches q and the first K tiles together; with the in-kernel q norm (q first,
    // then the tiles) a group's four buffers side by side measured 0.7% faster
    constexpr bool kGrouped = kNormQ && !kEarlyK;
    float* gsm = kGrouped ? smem + grp * kGroupF : smem + grp * 2 * kKTileF;
    float* gsv = kGrouped ? gsm + 2 * kKTileF : smem + kVBaseF + grp * 2 * kVTileF;
    const float sl2 = scale * 1.44269504088896340736f;

    // q of unit u reaches LDS by LDS DMA, once per workgroup: row r = 32*slot + j holds query
    // qb*32 + j of the slot's head (one contiguous 512-byte DMA per row; rows past B and idle
    // slots are clamped to valid rows, never written out).  Both key groups then read their
    // Q^T operand from it: qreg[4*k4 + j] = q[qb*32 + col][h][8*k4 + 4*hh + j].
    float* qst = smem + kQStageF;
    // wave wu stages rows 16*wu .. 16*wu+15 of unit u: half of slot wu/2, query rows r0 + min(j, jm)
    auto stage_rows = [&](int u, int& r0, int& jm, int& hq) {
        const int sl = kSlots * u + (wu >> 1);
        const int qsl = fdiv(sl, fG);
        const int qbs = sl < nslot ? qsl : nb - 1;
        r0 = min(qbs * kQB + (kQB / 2) * (wu & 1), B - 1);
        jm = B - 1 - r0;  // rows past B repeat the last row
        hq = kvh * G + sl - qsl * G;
    };
    auto stage_q = [&](int u) {
        // (scalar work is shared by the CU's eight waves, so the per-row address step is one add)
        int r0, jm, hq;
        stage_rows(u, r0, jm, hq);
        uint64_t sb = (uint64_t)(uintptr_t)(q + (size_t)r0 * q_stride + (size_t)hq * D);
        const uint32_t rs = (uint32_t)(q_stride * sizeof(float));
        const uint32_t lb = __builtin_amdgcn_readfirstlane(lds_addr(qst + (kQB / 2) * wu * kKS_F));
        if (hh == 0) {
#pragma unroll
            for (int j = 0; j < kQB / 2; ++j) {
                dma16_s(sb, voff_k, lb + j * (kKS_F * 4));
                if (j < jm) sb += rs;
            }
        }
    };
    float qreg[64];
    // raw q rows (kNormQ): QK-norm + RoPE in place, each wave on the 16 rows it staged, 8 lanes
    // per row, two rounds of 8 rows; gamma and both rounds' RoPE rows are loaded (load_norm)
    // while the q rows are still in flight, and used once they have landed (read_q)
    float qg[kNormQ ? 16 : 1];
    float4 qt[kNormQ ? 2 : 1][4];
    auto load_norm = [&](int u) {
        if constexpr (kNormQ) {
            int r0, jm, hq;
            stage_rows(u, r0, jm, hq);
            const int k = lane & 7, j = lane >> 3;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const float4 ga = *reinterpret_cast<const float4*>(q_gamma + 8 * k + 4 * i);
                const float4 gb = *reinterpret_cast<const float4*>(q_gamma + 64 + 8 * k + 4 * i);
                qg[4 * i] = ga.x, qg[4 * i + 1] = ga.y, qg[4 * i + 2] = ga.z, qg[4 * i + 3] = ga.w;
                qg[8 + 4 * i] = gb.x, qg[8 + 4 * i + 1] = gb.y, qg[8 + 4 * i + 2] = gb.z, qg[8 + 4 * i + 3] = gb.w;
            }
            const int p0 = *pos_dev + r0;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float2* row = cs + (size_t)(p0 + min(8 * h + j, jm)) * (kHeadDim / 2);
                const float4* tr = reinterpret_cast<const float4*>(row + 8 * k);
#pragma unroll
                for (int i = 0; i < 4; ++i) qt[h][i] = tr[i];
            }
        }
    };
    // q rows (and the norm's operands) have landed in this wave: the caller has waited
    auto read_q = [&]() {
        if constexpr (kNormQ) {
            const int k = lane & 7, j = lane >> 3;
#pragma unroll
            for (int h = 0; h < 2; ++h)
                norm_rope_q8(qst + ((kQB / 2) * wu + 8 * h + j) * kKS_F, qg, qt[h], eps, k);
        }
        __syncthreads();
        const float* qs = qst + (hw * kQB + col) * kKS_F + 4 * hh;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(qs + 8 * i);
            qreg[4 * i] = v.x;
            qreg[4 * i + 1] = v.y;
            qreg[4 * i + 2] = v.z;
            qreg[4 * i + 3] = v.w;
        }
    };
    const int u_second = nu - 1 - pair;  // the pass-1 unit (none when it equals pair)
    // this workgroup's share of the pair (prefill_share); wave-uniform: readfirstlane keeps the
    // values in scalar registers, the vector budget is full
    int lo0, r0, lo1, r1;
    prefill_share(pair, u_second, split, fK, pos0, B, nslot, fG, lo0, r0, lo1, r1);
    lo0 = __builtin_amdgcn_readfirstlane(lo0);
    r0 = __builtin_amdgcn_readfirstlane(r0);
    lo1 = __builtin_amdgcn_readfirstlane(lo1);
    r1 = __builtin_amdgcn_readfirstlane(r1);
    const int npass = (r0 > 0) + (r1 > 0);
    PSTAMPV(12, r0);
    PSTAMPV(13, r1);

    for (int pass = 0; pass < npass; ++pass) {
        const bool first_unit = pass == 0 && r0 > 0;  // this pass runs unit `pair`
        const int u = first_unit ? pair : u_second;
        const int sl = kSlots * u + hw;            // this wave's slot (wave-uniform)
        const bool live = sl < nslot;
        const int qb = fdiv(sl, fG), h = kvh * G + sl - qb * G;
        const int qb_last = fdiv(min(kSlots * u + kSlots - 1, nslot - 1), fG);  // the unit's last block
        const int b = qb * kQB + col;  // this lane's query row
        const int qpos = pos0 + b;

        floatx16 o[4];
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
        float m = -INFINITY, lsum = 0.f;

        const int T = pos0 + min(B, qb_last * kQB + kQB);  // keys seen by the unit's last query
        const int ntile = (T + kKT - 1) / kKT;
        const int nfull = live ? (pos0 + qb * kQB + 1) / kKT : ntile;  // tiles below this wave's diagonal
        const int kt_lo = first_unit ? lo0 : lo1;  // this workgroup's tiles of the unit: [kt_lo, kt_lo + nrange)
        const int nrange = first_unit ? r0 : r1;
        const int n_it = (nrange + kKS - 1) / kKS;
        const int n_mine = (nrange - grp + kKS - 1) / kKS;  // tiles of this key group

        // DMA of this group's i-th tile (kt = KS*i + grp) into a K or V buffer
        // DMA of this group's i-th tile (kt = KS*i + grp).  A tile wholly below T uses the
        // scalar-base form with per-lane byte offsets fixed for the pass; the tile that
        // reaches past T clamps each row to the last visible one (valid memory, masked out).
        auto dma_k = [&](int i, int buf) {
            const int t0 = (kt_lo + kKS * i + grp) * kKT;
            const uint32_t lb = __builtin_amdgcn_readfirstlane(lds_addr(gsm + buf * kKTileF));
            const int r0 = hw * 2 * DMA_PER_WAVE;  // this wave's first row of the tile
            if (hh == 0) {
                const uint32_t row0 = crow(t0);  // the tile's rows are consecutive from here
                if (t0 + kKT <= T) {
                    const uint64_t sb = kb_bytes + (uint64_t)(row0 + r0) * row_bytes;
#pragma unroll
                    for (int j = 0; j < 2 * DMA_PER_WAVE; ++j)  // one padded row per instruction
                        dma16_s(sb + (uint64_t)j * row_bytes, voff_k, lb + (r0 + j) * (kKS_F * 4));
                } else {
#pragma unroll
                    for (int j = 0; j < 2 * DMA_PER_WAVE; ++j) {
                        const int key = min(t0 + r0 + j, T - 1);
                        dma16(kbase + (size_t)(row0 + (key - t0)) * KD + 4 * col, lb + (r0 + j) * (kKS_F * 4));
                    }
                }
            }
        };
        auto dma_v = [&](int i, int buf) {
            const int t0 = (kt_lo + kKS * i + grp) * kKT;
            const uint32_t lb = __builtin_amdgcn_readfirstlane(lds_addr(gsv + buf * kVTileF));
            const int i0 = hw * DMA_PER_WAVE;  // 1 KB instruction = keys 2*ins, 2*ins+1
            const uint32_t row0 = crow(t0);
            if (t0 + kKT <= T) {
                const uint64_t sb = vb_bytes + (uint64_t)(row0 + 2 * i0) * row_bytes;
#pragma unroll
                for (int j = 0; j < DMA_PER_WAVE; ++j)
                    dma16_s(sb + (uint64_t)(2 * j) * row_bytes, voff_v, lb + (i0 + j) * 1024);
            } else {
#pragma unroll
                for (int j = 0; j < DMA_PER_WAVE; ++j) {
                    const int key = min(t0 + 2 * (i0 + j) + hh, T - 1);
                    dma16(vbase + (size_t)(row0 + (key - t0)) * KD + 4 * col, lb + (i0 + j) * 1024);
                }
            }
        };

        // S^T = K . Q^T for the K tile at Kt (padded rows); the operand of step k4+1 is
        // read while the four MFMAs of step k4 run
        auto qk = [&](const float* Kt, floatx16& acc) {
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = 0.f;
            const float* kp = Kt + col * kKS_F + 4 * hh;  // K[key col][8*k4 + 4*hh ..]
            float4 kv = *reinterpret_cast<const float4*>(kp);
#pragma unroll
            for (int k4 = 0; k4 < 16; ++k4) {
                const float4 kn = *reinterpret_cast<const float4*>(kp + 8 * ((k4 + 1) & 15));
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qreg[4 * k4 + 0], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qreg[4 * k4 + 1], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qreg[4 * k4 + 2], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qreg[4 * k4 + 3], acc, 0, 0, 0);
                kv = kn;
            }
        };

        // One tile kt of this group: softmax of its scores s (in place: s becomes P^T) and
        // O^T += V^T . P^T with V at Vt, while the scores of the K tile at Kn go to sn.  The
        // group's last tile passes the other (stale) K buffer as Kn and discards sn: a straight-line
        // body keeps O in 64 VGPRs (a branch around either product makes the compiler
        // split O across register files and spill at two waves per SIMD).
        // In-loop DMA for the next tiles: issued one or two instructions per MFMA sub-step, so
        // their issue time hides under the matrix pipe instead of idling it.  kin / vin: a K
        // (V) tile lies wholly below T and is fetched from scalar bases sbk / sbv into LDS at
        // lbk / lbv (tiles reaching past T are fetched up front through the clamped path).
        constexpr int NKI = 2 * DMA_PER_WAVE, NVI = DMA_PER_WAVE, NDI = NKI + NVI;
        const int r0k = hw * 2 * DMA_PER_WAVE, i0v = hw * DMA_PER_WAVE;
        auto step = [&](floatx16& s, floatx16& sn, int kt, const float* Kn, const float* Vt, bool kin, uint64_t sbk,
                        uint32_t lbk, bool vin, uint64_t sbv, uint32_t lbv) {
            if (kt >= nfull) {  // tile crosses the diagonal (wave-uniform)
                const int k0 = kt * kKT + 4 * hh;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (k0 + 8 * (r >> 2) + (r & 3) > qpos) s[r] = -INFINITY;
            }
            float mx = s[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
            const float ms = half_max(mx) * sl2;
            if (__builtin_amdgcn_ballot_w64(ms > m + kLazy)) {  // rare after the first tile
                const float mn = fmaxf(m, ms);
                const float corr = m == mn ? 1.f : __builtin_amdgcn_exp2f(m - mn);
                lsum *= corr;
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[db][i] *= corr;
                m = mn;
            }
            const float nb_ = m == -INFINITY ? 0.f : -m;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], sl2, nb_));
                lsum += s[r];
            }
            // the next tile's score chain (64 dependent MFMAs) interleaved with this tile's
            // P.V (four independent chains): one wave keeps the matrix pipe busy without
            // waiting on its own accumulator
            const float* vp = Vt + 4 * hh * D + 4 * col;
            auto vrow = [&](int r) {
                return *reinterpret_cast<const float4*>(vp + (8 * (r >> 2) + (r & 3)) * D);
            };
#pragma unroll
            for (int i = 0; i < 16; ++i) sn[i] = 0.f;
            const float* kp = Kn + col * kKS_F + 4 * hh;
            float4 kv = *reinterpret_cast<const float4*>(kp);
            float4 vv = vrow(0);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float4 kn = *reinterpret_cast<const float4*>(kp + 8 * ((r + 1) & 15));
                const float4 vn = vrow((r + 1) & 15);
#pragma unroll
                for (int x = r * NDI / 16; x < (r + 1) * NDI / 16; ++x) {
                    if (x < NKI) {
                        if (kin && hh == 0)  // one padded K row per instruction (lanes 0..31)
                            dma16_s(sbk + (uint64_t)x * row_bytes, voff_k, lbk + (r0k + x) * (kKS_F * 4));
                    } else if (vin) {  // two V rows per instruction
                        dma16_s(sbv + (uint64_t)(2 * (x - NKI)) * row_bytes, voff_v, lbv + (i0v + x - NKI) * 1024);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);  // step r+1's operands are read before step r's MFMAs
                sn = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qreg[4 * r + 0], sn, 0, 0, 0);
                o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, s[r], o[0], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                sn = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qreg[4 * r + 1], sn, 0, 0, 0);
                o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, s[r], o[1], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                sn = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qreg[4 * r + 2], sn, 0, 0, 0);
                o[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.z, s[r], o[2], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                sn = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qreg[4 * r + 3], sn, 0, 0, 0);
                o[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.w, s[r], o[3], 0, 0, 0);
                kv = kn;
                vv = vn;
                __builtin_amdgcn_sched_barrier(0);  // prefetch distance stays one step (register budget)
            }
        };

        // K buffers hold tiles i (even i in K0) and i+1; V buffers tile i.  At iteration
        // i: DMA K(i+2) -> K[i%2] and V(i+1) -> V[(i+1)%2] (both last read in iteration
        // i-1), read K(i+1) and V(i) (both landed by the wait + barrier ending i-1).
        // The score tiles alternate between sa and sb (loop unrolled by two).
        if (pass > 0) __syncthreads();  // every wave has stored its rows from the staging area
        PSTAMP(1 + 5 * pass);
        stage_q(u);
        load_norm(u);
        floatx16 sa, sb;
        if constexpr (!kNormQ) {
            // q rows and the first two K tiles are fetched together (K buffers lie outside the
            // staging area); the first V tile, which the staging area overlaps, once q is in
            // registers, and it lands while the first score chain runs.  (With the q norm
            // between, the same order measured 0.5% slower than fetching the tiles after it.)
            constexpr int kKI = 2 * DMA_PER_WAVE, kVI = DMA_PER_WAVE;  // DMA instructions per wave per K / V tile
            if (n_mine > 0) dma_k(0, 0);
            if (n_mine > 1) dma_k(1, 1);
            if (n_mine > 1) wait_vmcnt<2 * kKI>();  // older than the K tiles: the q rows
            else if (n_mine > 0) wait_vmcnt<kKI>();
            else wait_vmcnt<0>();
            read_q();
            __syncthreads();  // every wave has its q: the staging area is free for the V tiles
            if (n_mine > 0) dma_v(0, 0);
            if (n_mine > 1) wait_vmcnt<kKI + kVI>();  // K0 has landed (K1 and V0 may fly)
            else if (n_mine > 0) wait_vmcnt<kVI>();
            __syncthreads();
            if (n_mine > 0) qk(gsm, sa);
            wait_vmcnt<0>();  // K1 and V0
            __syncthreads();
        } else if constexpr (kEarlyK) {
            // the first two K tiles fly with the raw q rows and the norm's operands (K buffers lie
            // outside the staging area): one round trip before the norm instead of two; the first V
            // tile, which the staging area overlaps, once q is in registers, landing under the
            // first score chain
            if (n_mine > 0) dma_k(0, 0);
            if (n_mine > 1) dma_k(1, 1);
            wait_vmcnt<0>();
            read_q();
            __syncthreads();  // every wave has its q: the staging area is free for the V tiles
            if (n_mine > 0) dma_v(0, 0);
            if (n_mine > 0) qk(gsm, sa);
            wait_vmcnt<0>();  // V0
            __syncthreads();
        } else {
            wait_vmcnt<0>();
            read_q();
            __syncthreads();  // every wave has its q (the staging area is reused by the tile buffers)
            if (n_mine > 0) {
                dma_k(0, 0);
                dma_v(0, 0);
            }
            if (n_mine > 1) dma_k(1, 1);
            wait_vmcnt<0>();
            __syncthreads();
            if (n_mine > 0) qk(gsm, sa);
        }
        // paged: the cache row of the K tile fetched at iteration i + 1 is looked up at iteration
        // i (one scalar load in flight across an MFMA stream), and the V tile fetched at i + 1 is
        // the K tile of i, whose row is known by then; tiles past the range read no table entry
        PSTAMP(2 + 5 * pass);
        auto tile_row = [&](int i) -> uint32_t {  // cache row of this group's i-th tile, or 0
            const int kt = kt_lo + kKS * i + grp;
            return i < n_mine && (kt + 1) * kKT <= T ? crow(kt * kKT) : 0u;
        };
        uint32_t row_k = 0, row_v = 0;
        if constexpr (kPaged) {
            row_k = tile_row(2);
            row_v = tile_row(1);
        }
        auto iter = [&](int i, floatx16& s, floatx16& sn) {
            const int tk = (kt_lo + kKS * (i + 2) + grp) * kKT, tv = (kt_lo + kKS * (i + 1) + grp) * kKT;
            const bool kdo = i + 2 < n_mine, vdo = i + 1 < n_mine;
            const bool kin = kdo && tk + kKT <= T, vin = vdo && tv + kKT <= T;
            if (kdo && !kin) dma_k(i + 2, i & 1);
            if (vdo && !vin) dma_v(i + 1, (i + 1) & 1);
            const uint32_t rk = kPaged ? row_k : (uint32_t)tk, rv = kPaged ? row_v : (uint32_t)tv;
            if constexpr (kPaged) {
                row_v = row_k;
                row_k = tile_row(i + 3);
            }
            const uint64_t sbk = kb_bytes + (uint64_t)(rk + r0k) * row_bytes;
            const uint64_t sbv = vb_bytes + (uint64_t)(rv + 2 * i0v) * row_bytes;
            const uint32_t lbk = __builtin_amdgcn_readfirstlane(lds_addr(gsm + (i & 1) * kKTileF));
            const uint32_t lbv = __builtin_amdgcn_readfirstlane(lds_addr(gsv + ((i + 1) & 1) * kVTileF));
            if (i < n_mine)
                step(s, sn, kt_lo + kKS * i + grp, gsm + ((i + 1) & 1) * kKTileF, gsv + (i & 1) * kVTileF, kin, sbk,
                     lbk, vin, sbv, lbv);
            wait_vmcnt<0>();
            __syncthreads();
        };
        for (int i = 0; i < n_it; i += 2) {
            iter(i, sa, sb);
            if (i + 1 < n_it) iter(i + 1, sb, sa);
        }

        PSTAMP(3 + 5 * pass);
        // ---- merge the key groups through LDS (tile buffers are free after the barrier):
        // group g finalises output blocks db = 2g, 2g+1 and hands the other two to its partner
        float* xw = smem + w * (kXchF * 64) + lane;
        xw[0] = m;
        xw[64] = lsum;
        // (grp is wave-uniform: selects, not a dynamic register index)
        const floatx16 give0 = grp ? o[0] : o[2], give1 = grp ? o[1] : o[3];
        const floatx16 keep0 = grp ? o[2] : o[0], keep1 = grp ? o[3] : o[1];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            xw[(2 + i) * 64] = give0[i];
            xw[(18 + i) * 64] = give1[i];
        }
        __syncthreads();
        const float* xp = smem + ((1 - grp) * GW + hw) * (kXchF * 64) + lane;
        const float mp = xp[0], lp = xp[64];
        const float mt = fmaxf(m, mp);  // -inf only when this share holds no visible key for the query
        const float c0 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mt);
        const float cp = mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp - mt);
        const float l = half_sum(lsum * c0 + lp * cp);
        // finished rows (normalised, or the unnormalised share for k_prefill_combine) go to the
        // staging area in row order, then every wave stores two whole 512-byte rows per instruction
        {
            const float inv = ksplit == 1 ? 1.f / l : 1.f;
            float* ost = qst + (hw * kQB + col) * kKS_F + 2 * grp;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                // O^T register r of block db is d = 4*(8(r/4) + 4hh + r%4) + db
                float2 v;
                v.x = (keep0[r] * c0 + xp[(2 + r) * 64] * cp) * inv;
                v.y = (keep1[r] * c0 + xp[(18 + r) * 64] * cp) * inv;
                *reinterpret_cast<float2*>(ost + 4 * (8 * (r >> 2) + 4 * hh + (r & 3))) = v;
            }
            if (ksplit > 1 && live && b < B && hh == 0 && grp == 0)
                *reinterpret_cast<float2*>(part_ml + ((size_t)split * B * H + (size_t)b * H + h) * 2) =
                    make_float2(mt, l);
        }
        __syncthreads();
        {
            const int sl = kSlots * u + (wu >> 1);  // wave wu stores rows 16*(wu&1).. of slot wu/2
            const int qbo = fdiv(sl, fG), ho = kvh * G + sl - qbo * G;
            float* dst0 = ksplit == 1 ? out : part_o + (size_t)split * B * H * D;
#pragma unroll
            for (int j = 0; j < kQB / 4; ++j) {
                const int jj = (kQB / 2) * (wu & 1) + 2 * j + hh;
                const int bo = qbo * kQB + jj;
                const float4 v = *reinterpret_cast<const float4*>(qst + ((wu >> 1) * kQB + jj) * kKS_F + 4 * col);
                if (sl < nslot && bo < B)
                    *reinterpret_cast<float4*>(dst0 + ((size_t)bo * H + ho) * D + 4 * col) = v;
            }
        }
        PSTAMP(4 + 5 * pass);
    }
    PSTAMP(11);
}

// Merge of the ksplit shares of every (query, head): grid ceil(B*H/4), 128 threads; thread
// = float4 column d4 of row (b, h).  o = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s, empty
// shares (m = -inf) skipped.
__global__ __launch_bounds__(128) void k_prefill_combine(const float* __restrict__ part_o,
                                                         const float* __restrict__ part_ml, float* __restrict__ out,
                                                         int rows, int ksplit, const int* __restrict__ pos_dev, int B,
                                                         int H, int HKV) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 5), d4 = threadIdx.x & 31;
    if (row >= rows) return;
    // the row's unit and pair, as k_prefill numbers them; the shares holding tiles of that unit
    const int G = H / HKV, b = row / H, hq = row - b * H, g = hq % G;
    const int nb = (B + kQB - 1) / kQB, nslot = G * nb, nu = (nslot + kSlots - 1) / kSlots;
    const int u = ((b / kQB) * G + g) / kSlots, pair = min(u, nu - 1 - u);
    const FastDiv fG = fast_div((uint32_t)G), fK = fast_div((uint32_t)ksplit);
    const int pos0 = *pos_dev;
    // the covered shares' (m, l) and accumulator pieces are loaded before any is used: one
    // round trip, and no read of a share without tiles of this unit
    float2 ml[kPrefillMaxSplit];
    float4 v[kPrefillMaxSplit];
#pragma unroll
    for (int s = 0; s < kPrefillMaxSplit; ++s) {
        ml[s] = make_float2(-INFINITY, 0.f);
        if (s >= ksplit) continue;
        int lo0, r0, lo1, r1;
        prefill_share(pair, nu - 1 - pair, s, fK, pos0, B, nslot, fG, lo0, r0, lo1, r1);
        if ((u == pair ? r0 : r1) == 0) continue;
        const size_t slot = (size_t)s * rows + row;
        ml[s] = *reinterpret_cast<const float2*>(part_ml + slot * 2);
        v[s] = *reinterpret_cast<const float4*>(part_o + slot * kHeadDim + 4 * d4);
    }
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < kPrefillMaxSplit; ++s)
        if (s < ksplit) M = fmaxf(M, ml[s].x);
    float L = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < kPrefillMaxSplit; ++s) {
        if (s >= ksplit || ml[s].x == -INFINITY) continue;  // an empty share adds nothing
        const float wv = __builtin_amdgcn_exp2f(ml[s].x - M);
        L = fmaf(wv, ml[s].y, L);
        o.x = fmaf(wv, v[s].x, o.x);
        o.y = fmaf(wv, v[s].y, o.y);
        o.z = fmaf(wv, v[s].z, o.z);
        o.w = fmaf(wv, v[s].w, o.w);
    }
    const float inv = 1.f / L;
    o.x *= inv;
    o.y *= inv;
    o.z *= inv;
    o.w *= inv;
    *reinterpret_cast<float4*>(out + (size_t)row * kHeadDim + 4 * d4) = o;
}

static int prefill_grid1(int B, int H, int HKV) {
    const int G = H / HKV;
    const int nb = (B + kQB - 1) / kQB;
    const int nu = (G * nb + kSlots - 1) / kSlots;
    return ((nu + 1) / 2) * HKV;
}

int prefill_split(int B, int H, int HKV, int max_kv) {
    // One workgroup per (unit pair, KV head), all with the same work, one per CU at a time
    // (134 KB of LDS): the launch takes ceil(g1 / 256) rounds.  Splitting every unit's key
    // tiles into k contiguous shares makes g1*k workgroups of 1/k the work, so the time goes
    // as ceil(g1*k / 256) / k.  The plan takes the k in 1..8 with the shortest time, a larger
    // k only when it gains >= 10% (each share adds a combine read and write), and keeps >= 4
    // tiles per share on average (max_kv bounds pos0 + B on the host, which does not see the
    // device-resident position).
    const int g1 = prefill_grid1(B, H, HKV);
    const long avg_tiles = ((long)max_kv - B / 2 + kKT - 1) / kKT;
    long kmax = avg_tiles / 4 > 1 ? avg_tiles / 4 : 1;
    if (kmax > kPrefillMaxSplit) kmax = kPrefillMaxSplit;
    auto rounds = [&](long k) { return (double)((g1 * k + 255) / 256) / (double)k; };
    int best = 1;
    for (int k = 2; k <= kmax; ++k)
        if (rounds(k) < 0.9 * rounds(best)) best = k;
    if (const char* env = std::getenv("EI_PREFILL_SPLIT")) {  // tuning override (1..8)
        const int v = std::atoi(env);
        if (v >= 1 && v <= kPrefillMaxSplit) best = v;
    }
    return best;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t prefill_ws_bytes(int B, int H, int HKV, int max_kv) {
    const int k = prefill_split(B, H, HKV, max_kv);
    if (k <= 1) return 0;
    const size_t rows = (size_t)B * H;
    return align256((size_t)k * rows * kHeadDim * sizeof(float)) + align256((size_t)k * rows * 2 * sizeof(float));
}

template <bool kNormQ, bool kPaged, bool kEarlyK = false>
static hipError_t launch_prefill_kernel(hipStream_t st, unsigned grid, size_t lds, const float* q, long q_stride,
                                        float* out, const float* kc, const float* vc, const int* pos_dev, int B, int H,
                                        int HKV, float scale, int ksplit, float* part_o, float* part_ml,
                                        const float* q_gamma, const float* cs, float eps, const int* btab,
                                        int bshift, int max_blocks) {
    static std::atomic<bool> opted;
    if (const hipError_t e = opt_in_lds(opted, (const void*)k_prefill<kNormQ, kPaged, kEarlyK>, lds); e != hipSuccess)
        return e;
    k_prefill<kNormQ, kPaged, kEarlyK><<<grid, 64 * kSlots * kKS, lds, st>>>(q, q_stride, out, kc, vc, pos_dev, B, H, HKV, scale,
                                                                    ksplit, part_o, part_ml, q_gamma,
                                                                    reinterpret_cast<const float2*>(cs), eps, btab,
                                                                    bshift, max_blocks);
    return hipGetLastError();
}

hipError_t launch_prefill(hipStream_t st, const float* q, long q_stride, float* out, const float* kc,
                          const float* vc, const int* pos_dev, int B, int H, int HKV, float scale, int ksplit,
                          void* ws, const float* q_gamma, const float* cs, float eps, const int* block_table,
                          int block_shift, int max_blocks) {
    if (ksplit < 1) ksplit = 1;
    const unsigned grid = (unsigned)prefill_grid1(B, H, HKV) * ksplit;
    float* part_o = nullptr;
    float* part_ml = nullptr;
    if (ksplit > 1) {
        const size_t rows = (size_t)B * H;
        part_o = static_cast<float*>(ws);
        part_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + align256((size_t)ksplit * rows * kHeadDim * 4));
    }
    const size_t lds = (size_t)kLdsF * sizeof(float);  // > 64 KB: opt in once
    static_assert(kQStageF == kVBaseF && kQStageF <= kLdsF, "merge exchange below the staging area");
    static_assert(kLdsF * sizeof(float) <= 160 * 1024, "LDS budget");
    const bool nq = q_gamma != nullptr, pg = block_table != nullptr;
    hipError_t e;
    if (nq && pg) return hipErrorInvalidValue;  // not built: a paged step norms q in its prologue
    static const int early = [] {  // tuning aid: EI_PREFILL_EARLYK=0/1 forces the q-norm kernel's fetch order
        const char* v = std::getenv("EI_PREFILL_EARLYK");
        return v ? std::atoi(v) : -1;
    }();
    if (nq && (early == 1 || (early < 0 && ksplit > 1)))
        e = launch_prefill_kernel<true, false, true>(st, grid, lds, q, q_stride, out, kc, vc, pos_dev, B, H, HKV,
                                                     scale, ksplit, part_o, part_ml, q_gamma, cs, eps, nullptr, 0, 0);
    else if (nq)
        e = launch_prefill_kernel<true, false>(st, grid, lds, q, q_stride, out, kc, vc, pos_dev, B, H, HKV, scale,
                                               ksplit, part_o, part_ml, q_gamma, cs, eps, nullptr, 0, 0);
    else if (pg)
        e = launch_prefill_kernel<false, true>(st, grid, lds, q, q_stride, out, kc, vc, pos_dev, B, H, HKV, scale,
                                               ksplit, part_o, part_ml, nullptr, nullptr, 0.f, block_table,
                                               block_shift, max_blocks);
    else
        e = launch_prefill_kernel<false, false>(st, grid, lds, q, q_stride, out, kc, vc, pos_dev, B, H, HKV, scale,
                                                ksplit, part_o, part_ml, nullptr, nullptr, 0.f, nullptr, 0, 0);
    if (e != hipSuccess) return e;
    if (ksplit > 1) {
        const int rows = B * H;
        k_prefill_combine<<<(rows + 3) / 4, 128, 0, st>>>(part_o, part_ml, out, rows, ksplit, pos_dev, B, H, HKV);
    }
    return hipGetLastError();
}

}  // namespace ei

#ifdef EI_EXP_STAMPS
extern "C" __attribute__((visibility("default"))) int ei_diag_prefill_stamps(void* host, size_t n) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(ei::g_pstamps), n * 8, 0, hipMemcpyDeviceToHost);
}
#endif
