// decode.hip — split-K decode attention for gfx950 (one query token per sequence).
//
// Work decomposition: a 1-D grid of (sequence, KV head, key split) workgroups; 4 waves (long
// chunks, each wave a two-tile ring) or 8 waves (chunks of <= 128 keys, one tile per wave).
// A workgroup owns one KV head of one sequence and one chunk of keys, and serves all
// G = H/HKV query heads of that GQA group from the same K/V bytes (the reference re-reads K/V
// once per query head, src/cuda/model_cuda.cu:1051, :1066).  Inside the chunk, wave w owns the
// 16-key tiles w, w+NW, w+2NW, ... and runs its own online softmax over them; the waves merge
// once at the end.  There is no workgroup barrier between the DMA issue and the key loop.
// The split plan gives every (sequence, KV head) its own workgroup first and cuts keys only
// as far as it takes to reach about one workgroup per CU.
//
// Data movement: each wave streams its tiles HBM -> LDS with global_load_lds_dwordx4
// (gfx950 LDS DMA: 64 lanes x 16 B = one 1 KB instruction, no VGPRs spent on landing
// data, non-temporal: each byte is read once per step), through a private ring, so a
// workgroup keeps 128 KB of K/V in flight.  A 16-key tile is 16 rows x 512 B of K and the
// same of V; every instruction moves two whole rows (fully used 128-byte lines).  Within a
// row, 16-byte chunk q is stored at slot q ^ 8*(row & 1), which keeps both read patterns
// below free of LDS bank conflicts between neighbouring rows.  Cache rows come from a
// per-sequence offset (contiguous ranges) or from a block table (paged pools).
//
//   scores    lane (r = l/8, c = l%8) reads rows r and r+8 at d = 4c + 32i (i < 4) and
//             takes q for those d from registers (G <= 2) or from the workgroup's LDS
//             copy (more heads: register budget); the 8 lanes of a row hold partial dots for
//             (2 rows x G heads) and a transposing butterfly over lanes xor 1/2/4 leaves
//             one finished score per lane (7 exchanges for G = 4).
//   softmax   the tile max per head is a 4-step butterfly over the lanes holding that
//             head; p = 2^(s*scale*log2(e) - m) (one v_exp_f32) goes to a wave-private
//             LDS row.  The K rows of a tile are waited for first: scores and softmax
//             overlap the transfer of its V rows.
//   values    lane l owns d = 2l, 2l+1 of all 16 rows and accumulates p * v for the G
//             heads.
//
// Groups of 3, 5, 6 or 7 heads run on the kernel built for the next power of two, with the
// extra head slots idle (zero queries, never written out).
//
// Split combine: each workgroup writes its unnormalised partial (acc[G][128], and (m, l) in a
// one-line split record), merged as o = sum_s e^(m_s-M) acc_s / sum_s e^(m_s-M) l_s over the
// non-empty splits (src/cuda/model_cuda.cu:1097-1111 semantics).  Long chunks merge inside
// the launch: a unit's splits share one XCD and meet in its L2, and the workgroup that finds
// every split record published merges (merge_splits).  Short chunks merge in a second small
// launch (k_combine, one workgroup per query head).  A chunk covering all keys (nsplit = 1)
// writes o directly.
//
// Fused variant: the workgroup also applies QK-norm + RoPE to its G query heads, and the
// workgroup whose chunk holds the new position writes the normed K row and the V row to
// the cache and patches them into its LDS tile (the DMA may have read the old bytes).
// A sequence of length 0 (ragged or paged batches) produces zeros.
#include "common.h"
#include "launch.h"

#include <atomic>
#include <cstdlib>
#include <string>

namespace ei {

constexpr int kTile = 16;                          // keys per wave tile
constexpr int kTileFloats = 2 * kTile * kHeadDim;  // K rows then V rows
constexpr int kRingTiles = 8;                      // LDS ring: 8 tiles (128 KB) per workgroup
constexpr int kRec = 32;                           // uint32s per split record: one 128-byte line
constexpr int kCtrStride = 64;                     // uint32s between arrival counters (256 bytes)

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

// Copy nbytes (<= 1024, multiple of 16) of contiguous global memory into LDS; one
// instruction, lanes past the end idle.
__device__ __forceinline__ void dma_block(const float* g, uint32_t lds_base, int nbytes, int lane) {
    if (16 * lane < nbytes) dma16(g + 4 * lane, lds_base);
}

// Swizzled float offset of (row, 16-byte chunk) inside a tile's K or V half.
__device__ __forceinline__ int tile_off(int row, int chunk) {
    return row * kHeadDim + ((chunk ^ ((row & 1) << 3)) << 2);
}

// Issue the 16 DMA instructions of one tile: K rows t0..t0+15 then V rows (two rows per
// instruction), non-temporal: each byte of the cache is read once per step.  p0 is the cache
// row holding key t0; the tile's keys are consecutive rows from there (a paged block holds
// whole 16-key tiles).  Rows past t_end are clamped to the last visible row (valid memory; their
// scores are masked out).
// One half of a tile: the 16 K rows (which = 0) or the 16 V rows (which = 1), 8 instructions.
__device__ __forceinline__ void issue_half(const float* slot, const float* src, size_t KD, int t0, int t_end, int lane,
                                           size_t p0, int which) {
    const int half = lane >> 5, s = lane & 31;
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(slot)) + which * kTile * kHeadDim * 4;
#pragma unroll
    for (int t = 0; t < kTile / 2; ++t) {
        const int row = 2 * t + half;
        const int key = min(t0 + row, t_end - 1);
        const int chunk = s ^ ((row & 1) << 3);
        dma16_nt(src + (p0 + (size_t)(key - t0)) * KD + 4 * chunk, base + t * 1024);
    }
}

__device__ __forceinline__ void issue_tile(const float* slot, const float* kbase, const float* vbase, size_t KD,
                                           int t0, int t_end, int lane, size_t p0) {
    issue_half(slot, kbase, KD, t0, t_end, lane, p0, 0);
    issue_half(slot, vbase, KD, t0, t_end, lane, p0, 1);
}


// In-kernel split merge.  Loads miss the CU's L1 and read the XCD's L2 (buffer loads with
// sc0); the resource is based at one unit's partials, so 32-bit offsets always suffice.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufferDword3 = 0x00020000;  // raw 32-bit data, gfx9-family buffer resource word 3

__device__ __forceinline__ float4 ld_l2_f4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 1);
    return make_float4(__uint_as_float(x.x), __uint_as_float(x.y), __uint_as_float(x.z), __uint_as_float(x.w));
}
__device__ __forceinline__ float2 ld_l2_f2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 1);
    return make_float2(__uint_as_float(x.x), __uint_as_float(x.y));
}

__device__ __forceinline__ void fma4(float w, const float4 v, float4& acc) {
    acc.x = fmaf(w, v.x, acc.x);
    acc.y = fmaf(w, v.y, acc.y);
    acc.z = fmaf(w, v.z, acc.z);
    acc.w = fmaf(w, v.w, acc.w);
}

// Merge the S split partials of one unit (G head slots, the first Gr real) into out[Gr][128]:
// o = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s over the non-empty splits (m in log2
// units), the split-softmax combine of src/cuda/model_cuda.cu:1097-1111.
// Thread t owns float4 column t % (32 G) of splits t / (32 G), t / (32 G) + SG, ...; the
// first batch of its accumulator loads is in flight while each wave turns the (m, l) of its
// heads into weights (LDS); the SG column partials are summed in a fixed order, so the result
// does not depend on which workgroup merges.  `lds` is free LDS of >= G*256 + 64 +
// NT*4 floats.
template <int G, int NT>
__device__ __forceinline__ void merge_splits(const DecodeArgs& a, size_t head_slot, int S, int Gr, float* out,
                                             int tid, float* lds) {
    constexpr int D = kHeadDim, NCOLS = G * 32, SG = NT / NCOLS, NB = 8;
    static_assert(SG >= 1, "one thread per float4 column at least");
    const int col = tid % NCOLS, sg = tid / NCOLS, g = col >> 5, d4 = col & 31;
    const __amdgpu_buffer_rsrc_t racc = __builtin_amdgcn_make_buffer_rsrc(
        a.part_acc + head_slot * S * G * D, 0, S * G * D * 4, kBufferDword3);
    const __amdgpu_buffer_rsrc_t rml = __builtin_amdgcn_make_buffer_rsrc(
        a.rec + head_slot * S * kRec, 0, S * kRec * 4, kBufferDword3);
    float* wsh = lds;                                         // [G][256] split weights
    float* lsh = lds + G * kDecodeMaxSplits;                  // [G] weighted l sums
    float4* red = reinterpret_cast<float4*>(lsh + 64);        // [SG][NCOLS] column partials
    const uint32_t col_off = (uint32_t)(g * D + 4 * d4) * 4;  // bytes within one split's partial
    const uint32_t split_bytes = G * D * 4;
    float4 v[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) {  // out-of-range offsets read as zero (buffer bounds)
        const int s = sg + k * SG;
        v[k] = ld_l2_f4(racc, s < S ? (uint32_t)s * split_bytes + col_off : 0x80000000u);
    }
    const int lane = tid & 63;
    for (int hg = tid >> 6; hg < Gr; hg += NT / 64) {  // weights of head hg: one wave
        float mv[kDecodeMaxSplits / 64], lv[kDecodeMaxSplits / 64];
        float M = -INFINITY;
#pragma unroll
        for (int k = 0; k < kDecodeMaxSplits / 64; ++k) {
            const int s = lane + 64 * k;
            const float2 ml = s < S ? ld_l2_f2(rml, (uint32_t)(s * kRec + 2 + 2 * hg) * 4) : make_float2(-INFINITY, 0.f);
            mv[k] = ml.x;
            lv[k] = ml.y;
            M = fmaxf(M, ml.x);
        }
        M = wave_max(M);
        float L = 0.f;
#pragma unroll
        for (int k = 0; k < kDecodeMaxSplits / 64; ++k) {
            const int s = lane + 64 * k;
            const float wv = mv[k] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mv[k] - M);  // empty split: skipped
            if (s < S) wsh[hg * kDecodeMaxSplits + s] = wv;
            L = fmaf(wv, lv[k], L);
        }
        L = wave_sum(L);
        if (lane == 0) lsh[hg] = L;
    }
    __syncthreads();
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (g < Gr) {
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            const int s = sg + k * SG;
            if (s < S) fma4(wsh[g * kDecodeMaxSplits + s], v[k], acc);
        }
        for (int s0 = sg + NB * SG; s0 < S; s0 += NB * SG) {
#pragma unroll
            for (int k = 0; k < NB; ++k) {
                const int s = s0 + k * SG;
                v[k] = ld_l2_f4(racc, s < S ? (uint32_t)s * split_bytes + col_off : 0x80000000u);
            }
#pragma unroll
            for (int k = 0; k < NB; ++k) {
                const int s = s0 + k * SG;
                if (s < S) fma4(wsh[g * kDecodeMaxSplits + s], v[k], acc);
            }
        }
    }
    if (SG > 1) {
        red[sg * NCOLS + col] = acc;
        __syncthreads();
    }
    if (sg == 0 && g < Gr) {
#pragma unroll
        for (int j = 1; j < SG; ++j) {
            const float4 t = red[j * NCOLS + col];
            acc.x += t.x;
            acc.y += t.y;
            acc.z += t.z;
            acc.w += t.w;
        }
        const float L = lsh[g];
        const float4 o = L > 0.f ? make_float4(acc.x / L, acc.y / L, acc.z / L, acc.w / L)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);  // kv_len 0: zeros
        *reinterpret_cast<float4*>(out + (size_t)g * D + 4 * d4) = o;
    }
}

// NW waves per workgroup, each with a ring of kRingTiles/NW tile slots: 4 waves x 2 slots
// streams long chunks with one tile always in flight behind the one being scored; 8 waves
// x 1 slot gives short chunks (one tile per wave) two waves per SIMD to hide latency.
#ifdef EI_EXP_STAMPS
// Diagnostic build only.  Per workgroup of the last launch: [0] device realtime at start (100 MHz,
// common to all XCDs), [1] XCD, [2] realtime once this thread's partial (k_combine: output) store
// is acknowledged; k_combine's rows from 4096.  Per launch, block 0's start time in a ring of 1024
// ([0] k_decode, [1] k_combine).  Nothing is stored before the workgroup's end: a store issued
// early counts in vmcnt and would hold up the waits that follow it.
__device__ unsigned long long g_dstamps[8192 * 4];
__device__ unsigned long long g_dlaunch[2][1024];
__device__ unsigned g_dctr[2];
__device__ __forceinline__ unsigned long long rt_now() { return __builtin_amdgcn_s_memrealtime(); }
__device__ __forceinline__ unsigned long long xcc_now() {
    uint32_t x = 0;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x;
}
__device__ __forceinline__ void stamps_store(unsigned row, int kernel, unsigned long long t0, unsigned long long xcc) {
    wait_vmcnt<0>();
    const unsigned long long t1 = rt_now();
    if (threadIdx.x == 0) {
        g_dstamps[row * 4 + 0] = t0;
        g_dstamps[row * 4 + 1] = xcc;
        g_dstamps[row * 4 + 2] = t1;
        if (blockIdx.x == 0) g_dlaunch[kernel][atomicAdd(&g_dctr[kernel], 1u) & 1023u] = t0;
    }
}
#define STAMP_BEGIN const unsigned long long st_t0 = rt_now(), st_xcc = xcc_now()
#define STAMP_END(row, kernel) stamps_store((row), (kernel), st_t0, st_xcc)
#else
#define STAMP_BEGIN do { } while (0)
#define STAMP_END(row, kernel) do { } while (0)
#endif

template <int G, bool FUSED, int NW>
__global__ __launch_bounds__(64 * NW) void k_decode(const DecodeArgs a) {
    constexpr int kThreads = 64 * NW, kWaves = NW, kRing = kRingTiles / NW;
    constexpr int D = kHeadDim;
    constexpr int NV = 2 * G;                     // partial dots per lane in the score phase
    constexpr int NF = NV / 8 > 0 ? NV / 8 : 1;   // finished scores per lane after xreduce8
    constexpr int NCOL = G * 32;                  // float4 columns of the G output heads
    static_assert(kRing * kTileFloats >= G * kHeadDim, "a wave's ring slots hold its partial");
    STAMP_BEGIN;
    extern __shared__ __align__(16) float ring[];          // [kWaves][kRing][kTileFloats]; later scratch
    __shared__ __align__(16) float qs[G * D];
    __shared__ __align__(16) float pw[kWaves][kTile * G];  // per wave: p[row][g] of the current tile
    __shared__ __align__(16) float mw[kWaves][G];          // per wave: new running max per head
    __shared__ float wml[kWaves][2 * G];
    __shared__ __align__(16) float knew[4][D];             // fused: [0] K row (raw, then normed), [1] V row, [2] scratch
    __shared__ __align__(16) float stage[4 * D];           // fused: [0] q gamma, [1] k gamma, [2..3] RoPE row

    // Grid placement.  Workgroup b runs on XCD b % n_xcc.  With the in-kernel merge, every split
    // of one (sequence, KV head) unit sits on the same XCD, so the partials meet in its L2;
    // otherwise workgroup b takes split b % S of unit b / S, so an XCD streams the same key rows
    // of neighbouring KV heads (4 KB cache rows read by one XCD close together in time: ~2%
    // faster than a unit per XCD for short chunks).
    const int S = a.nsplit;
    int split, kvh, seq, unit;
    {
        const uint32_t b = blockIdx.x;
        if (a.merge_in_kernel) {
            const uint32_t nx = (uint32_t)a.n_xcc, x = b % nx, i = b / nx, lu = i / (uint32_t)S;
            split = (int)(i - lu * (uint32_t)S);
            unit = (int)(lu * nx + x);
        } else {
            unit = (int)(b / (uint32_t)S);
            split = (int)(b - (uint32_t)unit * S);
        }
        if (unit >= a.units) return;  // padding slot of the last XCD round
        seq = unit / a.HKV;
        kvh = unit - seq * a.HKV;
    }
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane >> 3, c = lane & 7;
    // this split's record line (its (m, l) per head slot; word 1: the XCD it ran on)
    uint32_t* unit_rec = a.rec + (size_t)unit * S * kRec;
    uint32_t* my_rec = unit_rec + split * kRec;
    const int len_in = a.kv_len ? a.kv_len[seq] : (*a.pos_dev + 1);
    const size_t KD = (size_t)a.HKV * D;
    const size_t row0 = a.kv_offset ? (size_t)a.kv_offset[seq] : 0;
    // cache row of this sequence's key t: contiguous from row0, or through the block table
    const int* btab = a.block_table ? a.block_table + (size_t)seq * a.max_blocks : nullptr;
    const int bshift = a.block_shift, bmask = (1 << bshift) - 1;
    // paged: keys past the table's blocks (a length outside the contract) are neither read nor
    // appended, so no table entry beyond max_blocks is ever loaded
    const int len = btab ? min(len_in, a.max_blocks << bshift) : len_in;
    auto phys = [&](int t) -> size_t {
        return btab ? ((size_t)btab[t >> bshift] << bshift) | (size_t)(t & bmask) : (size_t)t;
    };
    float* kbase = a.kc + row0 * KD + (size_t)kvh * D;
    float* vbase = a.vc + row0 * KD + (size_t)kvh * D;
    const int t_begin = split * a.chunk;
    // the last split takes every key past the plan (a kv_len above the planned max_kv is
    // still attended in full, and the fused step still finds the new row's owner)
    const int t_end = split == S - 1 ? len : min(len, t_begin + a.chunk);
    const int pos = len_in > 0 ? len_in - 1 : 0;  // a zero-length sequence has no new row; keep the table index valid
    const float* qrow = a.q + (size_t)seq * a.q_stride;
    const int Gr = a.H / a.HKV;  // heads of this KV head (<= G; heads Gr..G-1 are padding)
    const int h0 = kvh * Gr;
    float* wring = ring + w * (kRing * kTileFloats);


    // ---- prologue inputs first (wave 0: q rows, gammas, RoPE row; wave 1: the new K/V
    // row), then this wave's first two tiles, all as LDS DMA, so nothing waits on
    // anything before the whole workgroup's 128 KB is in flight
    const int tw0 = t_begin + kTile * w;
    constexpr int kStride = kTile * kWaves;  // distance between a wave's consecutive tiles
    // paged: lane i of lane_row holds the cache row of this wave's tile i, lane i of lane_row2
    // that of tile 64+i (the plan keeps <= 128 tiles per wave), read back with readlane: one or
    // two table loads per wave instead of one per tile
    int lane_row = 0, lane_row2 = 0;
    if (btab) {
        const int tl = max(t_end - 1, 0);
        const int t = min(tw0 + lane * kStride, tl);
        lane_row = (btab[t >> bshift] << bshift) | (t & bmask);
        if (tw0 + 64 * kStride < t_end) {
            const int t2 = min(tw0 + (lane + 64) * kStride, tl);
            lane_row2 = (btab[t2 >> bshift] << bshift) | (t2 & bmask);
        }
    }
    auto tile_row = [&](int t0) -> size_t {
        if (!btab) return (size_t)t0;
        const int i = (t0 - tw0) / kStride;
        if (i >= 128) return phys(t0);  // only a last split extended past the plan gets here
        return (size_t)(uint32_t)(i < 64 ? __builtin_amdgcn_readlane(lane_row, i)
                                         : __builtin_amdgcn_readlane(lane_row2, i - 64));
    };
    const bool owner = FUSED && t_begin <= pos && pos < t_end;  // pos >= t_end when len was capped
    const size_t pos_row = owner ? phys(pos) : 0;  // read before any DMA is in flight
    // The waves' DMA issue is back-pressured by the CU's request queue, so a wave spends most
    // of the stream waiting to get its instructions accepted.  Nothing waits at a workgroup
    // barrier behind that issue: wave 0 loads and norms q and publishes it (`q_ready`), and
    // each wave starts on its tiles as soon as q is ready and its own rows have landed.
    __shared__ int q_ready;
    if (tid == 0) q_ready = 0;
    __syncthreads();
    if (w == 0) {
        const uint32_t qa = __builtin_amdgcn_readfirstlane(lds_addr(qs));
#pragma unroll
        for (int i = 0; i < (G * D * 4 + 1023) / 1024; ++i)
            if (1024 * i < Gr * D * 4) dma_block(qrow + (size_t)h0 * D + 256 * i, qa + 1024 * i, Gr * D * 4 - 1024 * i, lane);
        if constexpr (FUSED) {
            dma_block(a.q_gamma, __builtin_amdgcn_readfirstlane(lds_addr(stage)), D * 4, lane);
            // the RoPE row: rope_dim*4 bytes, a multiple of 16 (the entry points require rope_dim % 4 == 0)
            dma_block(reinterpret_cast<const float*>(a.cs + (size_t)pos * (a.rope_dim >> 1)),
                      __builtin_amdgcn_readfirstlane(lds_addr(stage + 2 * D)), a.rope_dim * 4, lane);
            if (owner) {
                dma_block(qrow + (size_t)a.H * D + (size_t)kvh * D, __builtin_amdgcn_readfirstlane(lds_addr(knew[0])),
                          D * 4, lane);
                dma_block(qrow + (size_t)(a.H + a.HKV) * D + (size_t)kvh * D,
                          __builtin_amdgcn_readfirstlane(lds_addr(knew[1])), D * 4, lane);
                dma_block(a.k_gamma, __builtin_amdgcn_readfirstlane(lds_addr(stage + D)), D * 4, lane);
            }
        }
    }
    int ntiles0 = 0;
#pragma unroll
    for (int i = 0; i < kRing; ++i)
        if (tw0 + i * kStride < t_end) {
            issue_tile(wring + i * kTileFloats, kbase, vbase, KD, tw0 + i * kStride, t_end, lane,
                       tile_row(tw0 + i * kStride));
            ++ntiles0;
        }
    if (w == 0) {
        // the prologue DMA (older than this wave's tiles) has landed
        if (kRing == 2 && ntiles0 == 2) wait_vmcnt<2 * kTile>();
        else if (ntiles0 >= 1) wait_vmcnt<kTile>();
        else wait_vmcnt<0>();
        if (G > Gr)  // padding heads: zero queries (finite scores, never written out)
            for (int i = Gr * D + lane; i < G * D; i += 64) qs[i] = 0.f;
        if constexpr (FUSED) {
            const float2* cs_row = reinterpret_cast<const float2*>(stage + 2 * D);
            // in place: raw q -> normed, roped q; the G heads' norm factors together (padding
            // heads are zeros: a finite factor, never used)
            float x0[G], x1[G], inv[G];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                x0[g] = qs[g * D + lane];
                x1[g] = qs[g * D + lane + 64];
            }
            head_inv<G>(x0, x1, a.eps, inv, lane);
            const float qg0 = stage[lane], qg1 = stage[lane + 64];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                if (g >= Gr) break;
                float o0, o1;
                scale_rope_vals(x0[g], x1[g], inv[g], qg0, qg1, cs_row, a.rope_dim, knew[2], lane, &o0, &o1);
                qs[g * D + lane] = o0;
                qs[g * D + lane + 64] = o1;
            }
            if (owner) {
                float o0, o1;
                norm_rope_head(knew[0], stage + D, cs_row, a.rope_dim, a.eps, knew[2], lane, &o0, &o1);
                knew[0][lane] = o0;
                knew[0][lane + 64] = o1;
                __builtin_amdgcn_wave_barrier();
                // the new K row (lanes 0-31) and V row (lanes 32-63) to the cache, one float4 each
                float* dst = (lane < 32 ? kbase : vbase) + pos_row * KD + 4 * (lane & 31);
                *reinterpret_cast<float4*>(dst) = *reinterpret_cast<const float4*>(&knew[lane >> 5][4 * (lane & 31)]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): q (and the new K row) are in LDS
        __builtin_amdgcn_wave_barrier();
        if (lane == 0) __hip_atomic_store(&q_ready, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    } else {
        while (__hip_atomic_load(&q_ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 0)
            __builtin_amdgcn_s_sleep(1);
    }

    // q operand of the score phase: held in registers for up to 4 heads; 8 heads would take 128
    // VGPRs, so they are read from the LDS copy at each use (the 8 lanes of a chunk read one
    // address: broadcast reads)
    constexpr bool kQInRegs = G <= 2;
    float4 qreg[kQInRegs ? G : 1][4];
    if constexpr (kQInRegs)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) qreg[g][i] = *reinterpret_cast<const float4*>(qs + g * D + 4 * c + 32 * i);
    auto qv = [&](int g, int i) -> float4 {
        if constexpr (kQInRegs) return qreg[g][i];
        else return *reinterpret_cast<const float4*>(qs + g * D + 4 * c + 32 * i);
    };

    float m[G];         // running max per head (wave-uniform)
    float l[NF];        // per-lane partial denominators of this lane's (row, head) slots
    float2 acc[G];      // acc[g] at d = 2*lane, 2*lane+1
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        acc[g] = make_float2(0.f, 0.f);
    }
#pragma unroll
    for (int k = 0; k < NF; ++k) l[k] = 0.f;
    const int sidx = xreduce8_index<NV>(c);
    const float sl2 = a.scale * 1.44269504088896340736f;  // scores in log2 units: p = 2^(s - m)

    int slot_i = 0;
    for (int t0 = tw0; t0 < t_end; t0 += kStride, slot_i = (slot_i + 1) % kRing) {
        // this tile's K rows have landed (its 8 V instructions and the next tile may still
        // fly): the scores and softmax overlap the V transfer
        const bool next_flying = kRing == 2 && t0 + kStride < t_end;
        if (next_flying) wait_vmcnt<kTile + kTile / 2>();
        else wait_vmcnt<kTile / 2>();
        float* tk = wring + slot_i * kTileFloats;
        float* tv = tk + kTile * D;
        const int kr = pos - t0;  // fused: row of the new key in this tile, if any
        const bool patch = FUSED && owner && kr >= 0 && kr < kTile;
        if (patch) {  // the new row: overwrite what the DMA brought
            *reinterpret_cast<float2*>(tk + tile_off(kr, lane >> 1) + 2 * (lane & 1)) =
                *reinterpret_cast<const float2*>(&knew[0][2 * lane]);
            __builtin_amdgcn_wave_barrier();
        }

        // ---- scores: partial dots, 8-lane transposing reduction
        float part[NV];
#pragma unroll
        for (int x = 0; x < NV; ++x) part[x] = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 kv = *reinterpret_cast<const float4*>(tk + tile_off(8 * j + r, c + 8 * i));
#pragma unroll
                for (int g = 0; g < G; ++g) part[j * G + g] = dot4(qv(g, i), kv, part[j * G + g]);
            }
        xreduce8<NV>(part, c);

        // ---- online softmax over the tile, per head
#pragma unroll
        for (int k = 0; k < NF; ++k) {
            const int idx = sidx + k, j = idx / G, g = idx % G;
            const float sv = t0 + 8 * j + r < t_end ? part[k] * sl2 : -INFINITY;
            float mt = fmaxf(sv, lane_xor1(sv));  // lanes holding this head: xor 1, 8, 16, 32
            mt = fmaxf(mt, lane_xor8(mt));
            mt = fmaxf(mt, lane_xor16(mt));
            mt = fmaxf(mt, lane_xor32(mt));
            float mold = m[0];
#pragma unroll
            for (int gg = 1; gg < G; ++gg) mold = g == gg ? m[gg] : mold;
            const float mn = fmaxf(mold, mt);  // finite: the tile holds at least one visible key
            const float p = __builtin_amdgcn_exp2f(sv - mn);
            l[k] = l[k] * __builtin_amdgcn_exp2f(mold - mn) + p;
            pw[w][(8 * j + r) * G + g] = p;
            if (r == 0 && j == 0) mw[w][g] = mn;
        }
        __builtin_amdgcn_wave_barrier();
        if (t0 == tw0) {  // the wave's first tile: nothing accumulated yet, nothing to rescale
#pragma unroll
            for (int g = 0; g < G; ++g) m[g] = mw[w][g];
        } else {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float mn = mw[w][g];
                const float corr = __builtin_amdgcn_exp2f(m[g] - mn);
                m[g] = mn;
                acc[g].x *= corr;
                acc[g].y *= corr;
            }
        }
        // ---- values: acc[g][d] += p[row][g] * V[row][d], once the V rows have landed
        if (next_flying) wait_vmcnt<kTile>();
        else wait_vmcnt<0>();
        if (patch) {
            *reinterpret_cast<float2*>(tv + tile_off(kr, lane >> 1) + 2 * (lane & 1)) =
                *reinterpret_cast<const float2*>(&knew[1][2 * lane]);
            __builtin_amdgcn_wave_barrier();
        }
        const int voff = 2 * (lane & 1);
        // (8 heads: a partly unrolled loop keeps the row's p values and V pieces within the register budget)
#pragma unroll(G >= 4 ? 4 : kTile)
        for (int k = 0; k < kTile; ++k) {
            const float2 vv = *reinterpret_cast<const float2*>(tv + tile_off(k, lane >> 1) + voff);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float pv = pw[w][k * G + g];
                acc[g].x = fmaf(pv, vv.x, acc[g].x);
                acc[g].y = fmaf(pv, vv.y, acc[g].y);
            }
        }
        // reads of this slot have returned (their values were consumed above) before the
        // refill is issued into it
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
        if (t0 + kRing * kStride < t_end)
            issue_tile(tk, kbase, vbase, KD, t0 + kRing * kStride, t_end, lane, tile_row(t0 + kRing * kStride));
    }

    // ---- wave partial: l summed over the lanes holding each head; merge the waves in LDS
#pragma unroll
    for (int k = 0; k < NF; ++k) {
        float lv = l[k] + lane_xor1(l[k]);
        lv += lane_xor8(lv);
        lv += lane_xor16(lv);
        lv += lane_xor32(lv);
        const int idx = sidx + k, j = idx / G, g = idx % G;
        if (r == 0 && j == 0) {
            wml[w][g] = m[g];
            wml[w][G + g] = lv;
        }
    }
    // the wave's accumulator goes to its own ring slot: private to the wave, and every DMA
    // into it has landed (the key loop ends with a full wait), so one barrier suffices
#pragma unroll
    for (int g = 0; g < G; ++g) *reinterpret_cast<float2*>(&wring[g * D + 2 * lane]) = acc[g];
    __syncthreads();

    // thread t < NCOL merges float4 column (g, d4)
    const size_t head_slot = (size_t)seq * a.HKV + kvh;
    const size_t slot = head_slot * S + split;
    const int gcol = (tid % NCOL) / 32, d4 = (tid % NCOL) % 32;
    float Mw = -INFINITY, Lw = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tid < NCOL) {  // every wave wrote its (m, l, acc); a wave without keys has m = -inf, l = 0, acc = 0
        float mws[kWaves], lws[kWaves];
        float4 v[kWaves];
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) {
            mws[ww] = wml[ww][gcol];
            lws[ww] = wml[ww][G + gcol];
            v[ww] = *reinterpret_cast<const float4*>(&ring[ww * (kRing * kTileFloats) + gcol * D + 4 * d4]);
            Mw = fmaxf(Mw, mws[ww]);
        }
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) {
            const float wv = mws[ww] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mws[ww] - Mw);
            Lw = fmaf(wv, lws[ww], Lw);
            fma4(wv, v[ww], o);
        }
    }

    if (S == 1) {  // a single split is already the answer
        if (tid < NCOL && gcol < Gr) {
            if (Lw > 0.f) {
                o.x /= Lw;
                o.y /= Lw;
                o.z /= Lw;
                o.w /= Lw;
            }  // else no keys (kv_len 0): o is zeros
            *reinterpret_cast<float4*>(a.out + (size_t)seq * a.H * D + (size_t)(h0 + gcol) * D + 4 * d4) = o;
        }
        return;
    }

    // unnormalised partial of this split: acc rows, then the split's record line: for k_combine
    // the (m, l) pairs straight from the threads that hold them; for the in-kernel merge the
    // whole line by one instruction (valid in the L2 without a fill), with this XCD's id
    if (tid < NCOL && gcol < Gr) *reinterpret_cast<float4*>(a.part_acc + (slot * G + gcol) * D + 4 * d4) = o;
    const bool merging = a.merge_in_kernel;
    if (!merging) {  // k_combine merges in a second launch and reads only the (m, l) words of real heads
        if (tid < NCOL && d4 == 0 && gcol < Gr)
            *reinterpret_cast<float2*>(my_rec + 2 + 2 * gcol) = make_float2(Mw, Lw);
        STAMP_END(blockIdx.x, 0);
        return;
    }
    __shared__ float mlsh[2 * G];
    __shared__ int is_last;
    if (tid < NCOL && d4 == 0) {
        mlsh[2 * gcol] = Mw;
        mlsh[2 * gcol + 1] = Lw;
    }
    wait_vmcnt<0>();  // this thread's acc stores are in the L2 before the record is
    __syncthreads();
    if (w == 0) {
        uint32_t xcc = 0;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        if (lane < kRec)
            my_rec[lane] = lane == 1 ? xcc : lane >= 2 && lane < 2 + 2 * G ? __float_as_uint(mlsh[lane - 2]) : 0u;
        {
            // In-kernel merge.  Every split of the unit ran on this XCD, so the partials meet in
            // its L2: a store is acknowledged by the L2 (vmcnt), and loads that miss the CU's L1
            // read it there.  Once its partial and record are acknowledged, a workgroup counts
            // itself in on the unit's arrival counter (a line of its own); the one that brings
            // it to S merges and sets it back to zero for the next launch, whatever that
            // launch's plan.  No L2 write-back or invalidate (a device-wide fence costs more
            // than the whole decode on this part).
            wait_vmcnt<0>();  // the record is in the L2 before the count
            uint32_t old = 0;
            if (lane == 0) {
                uint32_t* ctr = a.ctr_top - (size_t)(unit + 1) * kCtrStride;
                old = atomicAdd(ctr, 1u);
                if (old == (uint32_t)S - 1) atomicSub(ctr, (uint32_t)S);
            }
            const bool last = __builtin_amdgcn_readfirstlane(old) == (uint32_t)S - 1;
            if (last) {  // the placement the protocol relies on (workgroups b and b + n_xcc share an
                         // XCD; the dispatcher's starting XCD may rotate between launches) held
                bool same_xcd = true;
                for (int s0 = 0; s0 < S; s0 += 64) {
                    const int sx = s0 + lane;
                    const uint32_t fx = sx < S ? __hip_atomic_load(unit_rec + sx * kRec + 1, __ATOMIC_RELAXED,
                                                                   __HIP_MEMORY_SCOPE_WORKGROUP)
                                               : xcc;
                    same_xcd = same_xcd && __builtin_amdgcn_ballot_w64(fx != xcc) == 0;
                }
                if (lane == 0 && !same_xcd) atomicOr(a.status, 1u);
            }
            if (lane == 0) is_last = last;
        }
    }
    __syncthreads();
    if (!is_last) return;
    merge_splits<G, kThreads>(a, head_slot, S, Gr, a.out + (size_t)seq * a.H * D + (size_t)h0 * D, tid, ring);
}

// Split combine as a separate launch: grid (n_seq * H), 128 threads (thread = d).  Wave 0
// issues the (m, l) loads of all S splits first, then every thread the accumulator loads of
// its first 32 splits, so the weights are computed while the partials are still in flight
// (loads return in issue order).  The weighted partials are summed in four interleaved
// chains (split s into chain s % 4), added in a fixed order at the end.  m is in log2 units
// (the decode kernel's exp2 domain).
template <int G>
__global__ __launch_bounds__(128) void k_combine(const DecodeArgs a) {
    constexpr int D = kHeadDim, B = 32, NA = 4, KM = kDecodeMaxSplits / 64;
    __shared__ float wsh[kDecodeMaxSplits];
    STAMP_BEGIN;
    __shared__ float Lsh;
    const int hq = blockIdx.x % a.H, seq = blockIdx.x / a.H;
    const int Gr = a.H / a.HKV;  // partials are laid out with G (>= Gr) head slots
    const int kvh = hq / Gr, g = hq % Gr;
    const int S = a.nsplit, tid = threadIdx.x;
    const size_t head_slot = (size_t)seq * a.HKV + kvh;
    const float* pml = reinterpret_cast<const float*>(a.rec + head_slot * S * kRec) + 2 + 2 * g;
    const float* pa = a.part_acc + (head_slot * S * G + g) * D + tid;
    float mv[KM], lv[KM];
    if (tid < 64) {
#pragma unroll
        for (int k = 0; k < KM; ++k) {
            const int s = tid + 64 * k;
            const float2 ml = s < S ? *reinterpret_cast<const float2*>(pml + (size_t)s * kRec)
                                    : make_float2(-INFINITY, 0.f);
            mv[k] = ml.x;
            lv[k] = ml.y;
        }
    }
    float acc[NA];
#pragma unroll
    for (int k = 0; k < NA; ++k) acc[k] = 0.f;
    for (int s0 = 0; s0 < S; s0 += B) {
        float v[B];
#pragma unroll
        for (int b = 0; b < B; ++b) v[b] = pa[(size_t)min(s0 + b, S - 1) * G * D];
        if (s0 == 0) {
            if (tid < 64) {  // weights: wave 0 reduces (m, l) over the splits
                float M = -INFINITY;
#pragma unroll
                for (int k = 0; k < KM; ++k) M = fmaxf(M, mv[k]);
                M = wave_max(M);
                float L = 0.f;
#pragma unroll
                for (int k = 0; k < KM; ++k) {
                    const int s = tid + 64 * k;
                    const float wv = mv[k] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mv[k] - M);  // empty split: skipped
                    if (s < S) wsh[s] = wv;
                    L = fmaf(wv, lv[k], L);
                }
                L = wave_sum(L);
                if (tid == 0) Lsh = L;
            }
            __syncthreads();
        }
#pragma unroll
        for (int b = 0; b < B; ++b)
            if (s0 + b < S) acc[b % NA] = fmaf(wsh[s0 + b], v[b], acc[b % NA]);
    }
    const float sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    a.out[(size_t)seq * a.H * D + (size_t)hq * D + tid] = Lsh > 0.f ? sum / Lsh : 0.f;  // kv_len 0: zeros
    STAMP_END(4096 + blockIdx.x, 1);
}

__global__ void k_ws_clear(uint32_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

// ------------------------------------------------------------------ host side
static int pow2_ceil(long x) {
    int p = 1;
    while (p < x && p < (1 << 30)) p <<= 1;
    return p;
}

DecodePlan decode_plan(int n_seq, int HKV, int max_kv, bool paged, bool capped) {
    // Keys are split as far as it takes to reach about one workgroup per CU (256): chunk =
    // max_kv / ceil(256 / (n_seq * HKV)), rounded up to a power of two >= 128 (128 fills every
    // wave's two-tile ring once), and at most 1024 keys: a batch of ragged sequences (the plan
    // sees only max_kv; the lengths are on the device) then spreads its long sequences over
    // many workgroups instead of leaving a few 8192-key units running alone at the end of the
    // launch (configs[4]-shaped batches, lengths U[256, 8192]: +1% to +10% over four length
    // draws, contiguous and paged alike).  Splits of a 1024-key chunk merge inside the launch,
    // so the cap adds no launch.  The split count stays within the combine's table.
    const long units = (long)n_seq * HKV;
    const long want = units >= 256 ? 1 : (256 + units - 1) / units;
    int chunk = pow2_ceil(((long)max_kv + want - 1) / want);
    if (chunk < 128) chunk = 128;
    if (capped && chunk > kDecodeMaxChunk) chunk = kDecodeMaxChunk;
    if (const char* env = std::getenv("EI_DECODE_CHUNK")) {  // tuning override (multiple of 64)
        const int v = std::atoi(env);
        if (v >= 64 && v % 64 == 0) chunk = v;
    }
    // paged: a wave keeps the cache rows of its tiles in two registers (<= 128 tiles, 4 waves)
    if (paged && chunk > kDecodePagedMaxChunk) chunk = kDecodePagedMaxChunk;
    while (((long)max_kv + chunk - 1) / chunk > kDecodeMaxSplits) chunk *= 2;
    DecodePlan p;
    p.chunk = chunk;
    p.nsplit = (max_kv + chunk - 1) / chunk;
    if (p.nsplit < 1) p.nsplit = 1;
    return p;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

DecodeWsLayout decode_ws_layout(int n_seq, int H, int HKV, int max_kv, bool capped) {
    // sized for the larger of the paged and contiguous plans, so one workspace serves both
    const DecodePlan p0 = decode_plan(n_seq, HKV, max_kv, false, capped);
    const DecodePlan p1 = decode_plan(n_seq, HKV, max_kv, true, capped);
    const DecodePlan p = p0.nsplit >= p1.nsplit ? p0 : p1;
    const size_t slots = (size_t)n_seq * HKV * p.nsplit;
    const int G = decode_group_slots(H / HKV);
    DecodeWsLayout l;
    l.rec = align256(slots * G * kHeadDim * 4);
    l.partials = l.rec + align256(slots * kRec * 4);
    l.units = (size_t)n_seq * HKV;
    return l;
}

size_t decode_ws_bytes(int n_seq, int H, int HKV, int max_kv) {
    const DecodeWsLayout l = decode_ws_layout(n_seq, H, HKV, max_kv);
    return ws_bytes_for(l.partials, l.units);
}

template <int G, int NW>
static hipError_t launch_gw(hipStream_t st, const DecodeArgs& a, int n_seq, bool fused) {
    // 1-D grid in XCD rounds: slot b runs on XCD b % n_xcc; the units of XCD x are x, x + n_xcc, ...
    // each with its nsplit workgroups (units past the end leave at once)
    const long rounds = ((long)a.units + a.n_xcc - 1) / a.n_xcc;
    const dim3 grid((unsigned)(rounds * a.n_xcc * a.nsplit));
    const size_t lds = (size_t)kRingTiles * kTileFloats * sizeof(float);  // 128 KB
    static std::atomic<bool> opted[2];
    const void* f = fused ? (const void*)k_decode<G, true, NW> : (const void*)k_decode<G, false, NW>;
    if (const hipError_t e = opt_in_lds(opted[fused], f, lds); e != hipSuccess) return e;
    if (fused) k_decode<G, true, NW><<<grid, 64 * NW, lds, st>>>(a);
    else k_decode<G, false, NW><<<grid, 64 * NW, lds, st>>>(a);
    if (a.nsplit > 1 && !a.merge_in_kernel)
        k_combine<G><<<(unsigned)(n_seq * a.H), 128, 0, st>>>(a);
    return hipGetLastError();
}

template <int G>
static hipError_t launch_g(hipStream_t st, const DecodeArgs& a, int n_seq, bool fused) {
    // one tile per wave with 8 waves when the chunk is short, else 4 waves streaming
    return a.chunk <= 8 * kTile ? launch_gw<G, 8>(st, a, n_seq, fused) : launch_gw<G, 4>(st, a, n_seq, fused);
}

int decode_group_slots(int g) { return g <= 1 ? 1 : g <= 2 ? 2 : g <= 4 ? 4 : g <= 8 ? 8 : 0; }

int device_xccs() {
    // XCDs of the current device (8 on an MI355X in SPX mode), queried once per device
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || v < 1 || v > 16) v = 1;
    cache[dev].store(v, std::memory_order_relaxed);
    return v;
}

bool decode_merge_in_kernel(int chunk, int n_xcc) {
    // Chunks of more than 128 keys (the 4-wave streaming kernel) merge in-kernel: configs[3]'s
    // 1024-key chunks run ~4.5% faster than with the second launch.  Short chunks (one tile per
    // wave, e.g. ctx 4096 over 32 splits) keep the second launch: there the partial stores are
    // acknowledged only once the memory queues drain after the stream (0.6-2 us, against
    // 0.18 us on an idle part), which costs more than the launch.  EI_DECODE_MERGE=launch or
    // =kernel forces either.  The protocol needs the splits of a unit on one XCD (one L2); that
    // workgroup b runs on XCD b % n_xcc was validated on MI355X in SPX mode (8 XCDs), and with
    // one XCD there is one L2.  Any other partition merges in the second launch.
    if (n_xcc != 8 && n_xcc != 1) return false;
    static const int forced = [] {
        const char* e = std::getenv("EI_DECODE_MERGE");
        if (!e) return -1;
        const std::string v(e);
        return v == "launch" ? 0 : v == "kernel" ? 1 : -1;
    }();
    return forced >= 0 ? forced == 1 : chunk > 8 * kTile;
}

hipError_t launch_decode(hipStream_t st, const DecodeArgs& a, int n_seq, bool fused) {
    // any group of 1..8 heads runs on the next kernel built for 1, 2, 4 or 8 heads
    switch (decode_group_slots(a.H / a.HKV)) {
        case 1: return launch_g<1>(st, a, n_seq, fused);
        case 2: return launch_g<2>(st, a, n_seq, fused);
        case 4: return launch_g<4>(st, a, n_seq, fused);
        case 8: return launch_g<8>(st, a, n_seq, fused);
        default: return hipErrorInvalidValue;
    }
}

// ------------------------------------------------------------------ stream ceiling
// The decode's memory traffic with no arithmetic: the same grid, waves, LDS-DMA instructions,
// tile order and cache policy as k_decode<G, false, NW> for one sequence of `len` keys, each
// wave waiting for its last tile and one lane per workgroup writing a word of it to `sink`.
// Its duration is the floor a decode launch of this plan can reach on this part.
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_stream_ceiling(const float* kc, const float* vc, int HKV, int len,
                                                            int chunk, int nsplit, float* sink) {
    constexpr int kRing = kRingTiles / NW, kStride = kTile * NW;
    extern __shared__ __align__(16) float ring[];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int unit = blockIdx.x / nsplit, split = blockIdx.x - unit * nsplit;
    if (unit >= HKV) return;
    const size_t KD = (size_t)HKV * kHeadDim;
    const float* kbase = kc + (size_t)unit * kHeadDim;
    const float* vbase = vc + (size_t)unit * kHeadDim;
    const int t_begin = split * chunk, t_end = min(len, t_begin + chunk);
    float* wring = ring + w * (kRing * kTileFloats);
    int slot = 0;
    for (int t0 = t_begin + kTile * w; t0 < t_end; t0 += kStride, slot = (slot + 1) % kRing) {
        if (t0 - (t_begin + kTile * w) >= kRing * kStride) wait_vmcnt<(kRing - 1) * kTile>();  // the slot's old tile
        issue_tile(wring + slot * kTileFloats, kbase, vbase, KD, t0, t_end, lane, (size_t)t0);
    }
    wait_vmcnt<0>();
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = ring[w * (kRing * kTileFloats)];
}

hipError_t launch_stream_ceiling(hipStream_t st, const float* kc, const float* vc, int HKV, int len, float* sink) {
    const DecodePlan p = decode_plan(1, HKV, len, false);
    const size_t lds = (size_t)kRingTiles * kTileFloats * sizeof(float);
    const dim3 grid((unsigned)(HKV * p.nsplit));
    if (p.chunk <= 8 * kTile) {
        static std::atomic<bool> opted;
        if (const hipError_t e = opt_in_lds(opted, (const void*)k_stream_ceiling<8>, lds); e != hipSuccess) return e;
        k_stream_ceiling<8><<<grid, 512, lds, st>>>(kc, vc, HKV, len, p.chunk, p.nsplit, sink);
    } else {
        static std::atomic<bool> opted;
        if (const hipError_t e = opt_in_lds(opted, (const void*)k_stream_ceiling<4>, lds); e != hipSuccess) return e;
        k_stream_ceiling<4><<<grid, 256, lds, st>>>(kc, vc, HKV, len, p.chunk, p.nsplit, sink);
    }
    return hipGetLastError();
}

// A plain streaming read: `bytes` (a multiple of 16) read once with non-temporal 16-byte global
// loads, consecutive lanes on consecutive 16-byte pieces, L loads per thread (L the smallest of
// 1, 2, 4, ..., 64 that covers the buffer with this grid; indices past the end are clamped to the
// last piece, so every load is unconditional).  kAll: every load of a thread is issued before any
// is used (a scheduling barrier; L x 4 registers); otherwise the compiler interleaves loads and
// uses, keeping fewer registers and more waves.  No LDS and no arithmetic beyond an XOR that keeps
// the loads; a workgroup writes to sink only if that XOR hits one fixed value.  Its duration is
// what a kernel reading this many bytes per launch with this grid can reach on this part.
template <int L, bool kAll>
__global__ __launch_bounds__(256) void k_read_ceiling(const u32x4* src, size_t n16, u32x4* sink) {
    const size_t nthr = (size_t)gridDim.x * 256, i = (size_t)blockIdx.x * 256 + threadIdx.x;
    u32x4 v[L];
#pragma unroll
    for (int k = 0; k < L; ++k) v[k] = __builtin_nontemporal_load(src + min(i + k * nthr, n16 - 1));
    if constexpr (kAll) __builtin_amdgcn_sched_barrier(0);
    u32x4 acc = v[0];
#pragma unroll
    for (int k = 1; k < L; ++k) acc ^= v[k];
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

template <bool kAll>
static hipError_t launch_read_ceiling_t(hipStream_t st, const u32x4* s, size_t n16, size_t per, int n_wg, u32x4* o) {
    if (per <= 1) k_read_ceiling<1, kAll><<<n_wg, 256, 0, st>>>(s, n16, o);
    else if (per <= 2) k_read_ceiling<2, kAll><<<n_wg, 256, 0, st>>>(s, n16, o);
    else if (per <= 4) k_read_ceiling<4, kAll><<<n_wg, 256, 0, st>>>(s, n16, o);
    else if (per <= 8) k_read_ceiling<8, kAll><<<n_wg, 256, 0, st>>>(s, n16, o);
    else if (per <= 16) k_read_ceiling<16, kAll><<<n_wg, 256, 0, st>>>(s, n16, o);
    else if (per <= 32) k_read_ceiling<32, kAll><<<n_wg, 256, 0, st>>>(s, n16, o);
    else if (per <= 64) k_read_ceiling<64, kAll><<<n_wg, 256, 0, st>>>(s, n16, o);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_read_ceiling(hipStream_t st, const void* src, size_t bytes, int n_wg, bool all_in_flight,
                               void* sink) {
    const size_t n16 = bytes / 16, nthr = (size_t)n_wg * 256, per = (n16 + nthr - 1) / nthr;
    const u32x4* s = static_cast<const u32x4*>(src);
    u32x4* o = static_cast<u32x4*>(sink);
    return all_in_flight ? launch_read_ceiling_t<true>(st, s, n16, per, n_wg, o)
                         : launch_read_ceiling_t<false>(st, s, n16, per, n_wg, o);
}

// ------------------------------------------------------------------ allocation-free scratch
// Device-resident scratch for ei_decode_step_noalloc: each GPU the library runs on holds its
// own copy until the process ends.  Host code never passes `scratch` itself (its host-side name
// is not a device address): decode_scratch() looks up this device's address once, with the
// device current, and callers use that pointer.
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

hipError_t decode_scratch(void** ptr) {
    constexpr int kMaxDevices = 64;
    static std::atomic<void*> addr[kMaxDevices];
    int dev = 0;
    if (const hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    void* p = addr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {  // first call on this device (concurrent first calls look up the same address)
        if (const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        addr[dev].store(p, std::memory_order_release);
    }
    *ptr = p;
    return hipSuccess;
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

#ifdef EI_EXP_STAMPS
extern "C" __attribute__((visibility("default"))) int ei_diag_decode_launches(void* host) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(ei::g_dlaunch), sizeof(ei::g_dlaunch), 0, hipMemcpyDeviceToHost);
}
extern "C" __attribute__((visibility("default"))) int ei_diag_decode_stamps(void* host, size_t n) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(ei::g_dstamps), n * 8, 0, hipMemcpyDeviceToHost);
}
#endif
