// Fused LoRA merge + rowwise weight requantization (gfx950).
//
//   W'[n][k]   = bf16(W[n][k] + bf16(lora_scale * sum_j B[n][j] A[j][k]))
//   w_scale[n] = max(max_k |W'[n][k]| / 448, 1e-12)
//   wq[n][k]   = e4m3(bf16(W'[n][k] / bf16(w_scale[n])))
//
// The reference merges in place on the bf16 weight (lora.py:91-92) and then
// quantizes it in eager torch (fp8_linear.py:262-267): several full passes over
// W plus the write-back of W'. Here W' is never stored unless asked for.
//
// Work split: the weight is cut into 256-column stripes and 64-row tiles. A
// workgroup (four waves, 16 rows each) owns one stripe and walks a set of its
// row tiles, so the stripe's slice of A is staged in LDS once per workgroup;
// the next tile's W and B are loaded into registers while the current tile is
// computed. Two such passes:
//   pass 1 (kRowMax)   W + delta in binary32 per element, the row maxima of
//                      |.| merged into w_scale (used as a uint32 max of bf16
//                      magnitude bits, zeroed first). Rounding to nearest is
//                      monotone and symmetric, so max |bf16(x)| = bf16(max |x|):
//                      the elements are not rounded in this pass.
//   pass 2 (kQuantize) W' recomputed (W re-read, largely from the last-level
//                      cache) and the codes written; the workgroups of stripe 0
//                      turn the row maxima into the reference's scales in place.
// Merge-only calls (no codes) run pass 2's body with the W' store alone.
//
// The rank-r update uses v_mfma_f32_16x16x32_bf16: MFMA row index = a column
// k of W, column index = a row n, reduction = rank. Products of bf16 are exact
// in fp32 and the accumulation is fp32, as the reference's fp32 matmul. The
// MFMA's k-side operand is A transposed, staged in LDS as one row per column
// k (rank contiguous, padded to rank + 8 elements). The staging permutes the
// columns (at_row) so that each lane's outputs over four MFMA tiles are 16
// consecutive columns of one row: W and W' move 32 bytes per lane and group,
// the codes 16.
#include <stdint.h>

#include <type_traits>

#include "vdn_common.h"

namespace vdn {
namespace {

constexpr int kRowsPerWave = 16;
constexpr int kWaves = 4;
constexpr int kLanes = 64;
constexpr int kThreads = kWaves * kLanes;
constexpr int kTileRows = kRowsPerWave * kWaves;   // 64
constexpr int kTileCols = 256;                      // one stripe
constexpr int kGroups = kTileCols / 64;             // per lane: 16 consecutive columns of each 64

enum Mode { kRowMax = 0, kQuantize = 1, kMergeOnly = 2, kQuantizeMerged = 3 };

// Byte offset past every buffer descriptor used here: a store sent there is dropped.
constexpr uint32_t kDropped = 0x80000000u;

typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x2_t u32x2(uint32_t a, uint32_t b) { return i32x2_t{(int)a, (int)b}; }
__device__ __forceinline__ i32x4_t u32x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d)
{
    return i32x4_t{(int)a, (int)b, (int)c, (int)d};
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct Args {
    const uint16_t* w;
    int64_t N, K, ldw;
    const uint16_t* a;   // [rank, K], 16-byte aligned
    const uint16_t* b;   // [N, rank]
    int64_t rank;
    int b_vec;           // rows of B are 16-byte aligned (rank % 8 == 0)
    float lora_scale;
    uint8_t* wq;
    int64_t ldq;
    float* w_scale;      // pass 1: the row maxima as uint32 bf16 magnitude bits
    uint16_t* w_merged;  // nullable, row stride ldw
    int wm16;            // w_merged rows are 16-byte aligned
    int stripes;         // ceil(K / 256); the grid is stripes x (tile walkers per stripe)
    int row_tiles;       // ceil(N / 64)
};

// LDS row of column k (0..255) of the stripe: MFMA tile t = 4 (k / 64) +
// (k % 16) / 4 holds, in its row i = 4 ((k % 64) / 16) + k % 4, column k. Lane
// (n, g) of tile t gets rows 4 g .. 4 g + 3, so over t = 4 c .. 4 c + 3 it gets
// columns 64 c + 16 g .. + 15.
__device__ __forceinline__ int at_row(int k)
{
    return 64 * (k >> 6) + 16 * ((k >> 2) & 3) + 4 * ((k >> 4) & 3) + (k & 3);
}

// Four bf16 values (two packed words) -> four codes: quotient by the bf16 scale,
// rounded to bf16 (two per conversion; opaque so the pair stays one
// instruction), then e4m3 straight from the packed bf16. Both operands are
// bf16, where RN_bf16(x * RN(1/s)) equals RN_bf16(x / s) for every pair
// (checked exhaustively): one multiply.
__device__ __forceinline__ uint32_t codes4(uint2 v, float r)
{
    uint32_t q01 = pack_bf16x2(bf16_lo(v.x) * r, bf16_hi(v.x) * r);
    uint32_t q23 = pack_bf16x2(bf16_lo(v.y) * r, bf16_hi(v.y) * r);
    asm volatile("" : "+v"(q01), "+v"(q23));
    return pack_e4m3x4_bf16(q01, q23);
}

__device__ __forceinline__ uint32_t codes4_exact(uint2 v, float s)
{
    return pack_e4m3x4(round_bf16(bf16_lo(v.x) / s), round_bf16(bf16_hi(v.x) / s),
                       round_bf16(bf16_lo(v.y) / s), round_bf16(bf16_hi(v.y) / s));
}

// Registers of one row tile: W (per group c, 16 columns in two 16-byte
// pieces), the B operand, and (pass 2) the row-maximum bits.
template <int RP>
struct TileRegs {
    uint4 w[2 * kGroups];
    bf16x8_t b[RP / 32];
    uint32_t mbits;
};

// B operand of rank step s for row nr of the tile based at row n0: lane holds
// B[n][32 s + 8 g .. +7] (zero beyond the rank), from 2-byte loads (any rank).
template <int RP>
__device__ __forceinline__ bf16x8_t b_operand_scalar(const Args& p, __amdgpu_buffer_rsrc_t br, int nr, int s, int g)
{
    const int j0 = 32 * s + 8 * g;
    uint32_t e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(br, (uint32_t)((nr * p.rank + j0 + 2 * i) * 2), 0, 0);
        const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(br, (uint32_t)((nr * p.rank + j0 + 2 * i + 1) * 2), 0, 0);
        e[i] = (lo & 0xffffu) | (hi << 16);
        const int j = j0 + 2 * i;
        if (j >= p.rank) e[i] = 0u;
        else if (j + 1 >= p.rank) e[i] &= 0xffffu;
    }
    return __builtin_bit_cast(bf16x8_t, make_uint4(e[0], e[1], e[2], e[3]));
}

// RP = rank padded to a multiple of 32. BVEC: rows of B 16-byte aligned and
// rank % 8 == 0, so B is prefetched with the tile's W by 16-byte loads.
template <int RP, int MODE, bool BVEC>
__global__ __launch_bounds__(kThreads) void k_lora_stripes(Args p)
{
    constexpr int kS = RP + 8;                       // LDS row (one column k) in elements
    constexpr bool kCodes = MODE == kQuantize || MODE == kQuantizeMerged;
    constexpr bool kMerged = MODE == kMergeOnly || MODE == kQuantizeMerged;
    __shared__ __attribute__((aligned(16))) uint16_t sAT[kTileCols * kS];

    const int tid = threadIdx.x, lane = tid & (kLanes - 1);
    const int wave = tid / kLanes;
    const int nl = lane & 15, g = lane >> 4;
    const int stripe = (int)(blockIdx.x % (unsigned)p.stripes);
    const int rstep = (int)(gridDim.x / (unsigned)p.stripes);
    const int64_t k0 = (int64_t)stripe * kTileCols;
    const int nr = wave * kRowsPerWave + nl;            // row within a tile

    // All loads go through buffer descriptors: rows past N and rank rows past
    // the LoRA rank read as zeros with no branch, so the loads stay in flight
    // together. Columns past K may read the next row's data; they only feed
    // outputs that are neither stored nor counted in a maximum.
    // A tile past the last one gets empty descriptors (every load reads zero
    // and touches no memory): the loads stay unconditional, so the compiler
    // counts them exactly and waits for a tile's loads only where it is used.
    auto load_tile = [&](int rt, TileRegs<RP>& t) {
        const int rtc = min(rt, p.row_tiles - 1);
        const int64_t n0 = (int64_t)rtc * kTileRows;
        const int64_t rows = rt < p.row_tiles ? min(p.N - n0, (int64_t)kTileRows) : 0;
        const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(p.w + n0 * p.ldw), 0, (int)(rows * p.ldw * 2), 0x00020000);
#pragma unroll
        for (int c = 0; c < kGroups; ++c) {
            const uint32_t off = (uint32_t)((nr * p.ldw + k0 + 64 * c + 16 * g) * 2);
            // pass 1 leaves W in the caches for pass 2, whose read is the last
            constexpr int pol = MODE == kRowMax ? 0 : kBufferLoadOnce;
            t.w[2 * c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, pol));
            t.w[2 * c + 1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, off + 16, 0, pol));
        }
        // B operand, raw (the rank mask applies when it is used, so that no
        // wait for these loads lands here)
        if (BVEC) {
            const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(p.b + n0 * p.rank), 0, (int)(rows * p.rank * 2), 0x00020000);
#pragma unroll
            for (int s = 0; s < RP / 32; ++s)
                t.b[s] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(
                    br, (uint32_t)((nr * p.rank + 32 * s + 8 * g) * 2), 0, 0));
        }
        t.mbits = 0u;
        if (kCodes) {
            const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(p.w_scale + n0), 0, (int)(rows * 4), 0x00020000);
            t.mbits = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(sr, (uint32_t)(nr * 4), 0, 0);
        }
    };

    // Stage A^T of the stripe: unit u covers rank rows j = 2 pr, 2 pr + 1 and
    // columns 8 kg .. 8 kg + 7; each column's pair is one dword at LDS row
    // at_row(column), element j. Rank rows past the rank read as zeros.
    {
        const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
            (void*)p.a, 0, (int)(p.rank * p.K * 2), 0x00020000);
        constexpr int kPairs = RP / 2, kUnits = kPairs * (kTileCols / 8);
        uint4 alo[kUnits / kThreads], ahi[kUnits / kThreads];
#pragma unroll
        for (int i = 0; i < kUnits / kThreads; ++i) {
            const int u = tid + i * kThreads;
            const int pr = u % kPairs, kg = u / kPairs;
            const int64_t j = 2 * pr, k = k0 + 8 * kg;
            alo[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ar, (uint32_t)((j * p.K + k) * 2), 0, 0));
            ahi[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ar, (uint32_t)(((j + 1) * p.K + k) * 2), 0, 0));
        }
#pragma unroll
        for (int i = 0; i < kUnits / kThreads; ++i) {
            const int u = tid + i * kThreads;
            const int pr = u % kPairs, kg = u / kPairs;
            const uint32_t l[4] = {alo[i].x, alo[i].y, alo[i].z, alo[i].w}, h[4] = {ahi[i].x, ahi[i].y, ahi[i].z, ahi[i].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t* d0 = reinterpret_cast<uint32_t*>(sAT + at_row(8 * kg + 2 * e) * kS + 2 * pr);
                uint32_t* d1 = reinterpret_cast<uint32_t*>(sAT + at_row(8 * kg + 2 * e + 1) * kS + 2 * pr);
                *d0 = (l[e] & 0xffffu) | (h[e] << 16);
                *d1 = (l[e] >> 16) | (h[e] & 0xffff0000u);
            }
        }
    }

    auto compute = [&](int rt, const TileRegs<RP>& t) {
        const int64_t n0 = (int64_t)rt * kTileRows;
        const int64_t rows = min(p.N - n0, (int64_t)kTileRows);
        const int64_t n = n0 + nr;
        const bool nvalid = n < p.N;
        // B operand: lane holds B[n][32 s + 8 g .. +7], zero beyond the rank
        // (rank % 8 == 0 on the vector path: all 8 or none)
        bf16x8_t bop[RP / 32];
        if (BVEC) {
#pragma unroll
            for (int s = 0; s < RP / 32; ++s)
                bop[s] = (32 * s + 8 * g < p.rank) ? t.b[s] : bf16x8_t{};
        } else {
            const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(p.b + n0 * p.rank), 0, (int)(rows * p.rank * 2), 0x00020000);
#pragma unroll
            for (int s = 0; s < RP / 32; ++s) bop[s] = b_operand_scalar<RP>(p, br, nr, s, g);
        }
        float sb = 0.0f, r = 0.0f;
        bool exact = false;   // some row of the wave has a non-finite scale
        if (kCodes) {
            // w_scale[n] holds either the row maximum's bf16 magnitude bits (below
            // 2^16) or, once a workgroup of stripe 0 has passed, the reference's
            // scale (binary32 bits of a value >= 1e-12 or NaN: above 2^16). Both
            // give the same scale; stripe 0 stores it, so racing readers agree.
            const float s32 = t.mbits < 0x10000u ? row_scale(bf16_to_f32((uint16_t)t.mbits)) : __uint_as_float(t.mbits);
            const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(p.w_scale + n0), 0, (int)(rows * 4), 0x00020000);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(s32), sr,
                                                  (stripe == 0 && g == 0) ? (uint32_t)(nr * 4) : kDropped, 0, 0);
            sb = round_bf16(s32);
            r = 1.0f / sb;
            exact = __builtin_amdgcn_ballot_w64(!__builtin_isfinite(sb)) != 0;
        }
        // Outputs go through buffer stores whose descriptors cover the tile's
        // rows; a lane whose columns lie past K sends its stores out of range
        // (dropped), so no store sits under a branch.
        const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(kCodes ? p.wq + n0 * p.ldq : nullptr), 0, kCodes ? (int)(rows * p.ldq) : 0, 0x00020000);
        const __amdgpu_buffer_rsrc_t mr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(kMerged ? p.w_merged + n0 * p.ldw : nullptr), 0, kMerged ? (int)(rows * p.ldw * 2) : 0, 0x00020000);
        float mx = 0.0f;
        auto group = [&](int c, auto exact_tag) {
            constexpr bool kExact = decltype(exact_tag)::value;
            const int64_t k = k0 + 64 * c + 16 * g;       // this lane's 16 columns k .. k + 15
            const bool in = nvalid && k < p.K;            // K % 16 == 0: all 16 or none
            f32x4_t acc[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                acc[m] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                const uint16_t* arow = sAT + (16 * (4 * c + m) + nl) * kS + 8 * g;
#pragma unroll
                for (int s = 0; s < RP / 32; ++s) {
                    const bf16x8_t aop = *reinterpret_cast<const bf16x8_t*>(arow + 32 * s);
                    acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, bop[s], acc[m], 0, 0, 0);
                }
            }
            // column 16 g + 4 m + e of the group <-> acc[m][e]; W word (m % 2) * 2 + e / 2
            // of piece m / 2, half e % 2
            float x[16];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const uint4 wp = t.w[2 * c + m / 2];
                const uint32_t ww[4] = {wp.x, wp.y, wp.z, wp.w};
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                    const uint32_t word = ww[(m % 2) * 2 + e / 2];
                    // delta.to(bf16) (two at a time), then the bf16 add: binary32 sum
                    // of the two bf16 values
                    uint32_t d = pack_bf16x2(acc[m][e] * p.lora_scale, acc[m][e + 1] * p.lora_scale);
                    // opaque: the compiler would otherwise split the pair back into
                    // two one-value conversions
                    asm volatile("" : "+v"(d));
                    x[4 * m + e] = bf16_lo(word) + bf16_lo(d);
                    x[4 * m + e + 1] = bf16_hi(word) + bf16_hi(d);
                }
            }
            if constexpr (MODE == kRowMax) {
                float gm = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; ++i) gm = __builtin_elementwise_maximum(gm, __builtin_fabsf(x[i]));
                mx = __builtin_elementwise_maximum(mx, in ? gm : 0.0f);
            } else {
            uint32_t wm[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                wm[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
                asm volatile("" : "+v"(wm[i]));
            }
            if constexpr (kMerged) {
                const uint32_t off = in ? (uint32_t)((nr * p.ldw + k) * 2) : kDropped;
                if (p.wm16) {
                    __builtin_amdgcn_raw_buffer_store_b128(u32x4(wm[0], wm[1], wm[2], wm[3]), mr, off, 0, 0);
                    __builtin_amdgcn_raw_buffer_store_b128(u32x4(wm[4], wm[5], wm[6], wm[7]), mr, off + 16, 0, 0);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        __builtin_amdgcn_raw_buffer_store_b64(u32x2(wm[2 * i], wm[2 * i + 1]), mr, off + 8 * i, 0, 0);
                }
            }
            if constexpr (kCodes) {
                uint32_t q[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint2 v = make_uint2(wm[2 * i], wm[2 * i + 1]);
                    q[i] = kExact ? codes4_exact(v, sb) : codes4(v, r);
                }
                const uint32_t off = in ? (uint32_t)(nr * p.ldq + k) : kDropped;
                __builtin_amdgcn_raw_buffer_store_b64(u32x2(q[0], q[1]), qr, off, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b64(u32x2(q[2], q[3]), qr, off + 8, 0, 0);
            }
            }
        };
        // One uniform branch per tile: the rows of a wave either all have finite
        // scales (one multiply per quotient) or take the IEEE division throughout
        // (the same codes where the scale is finite).
        // (Scheduling barriers between the groups keep the compiler from hoisting
        // several groups' work at once, which would cost occupancy.)
        if (kCodes && exact) {
#pragma unroll
            for (int c = 0; c < kGroups; ++c) {
                group(c, std::true_type{});
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
#pragma unroll
            for (int c = 0; c < kGroups; ++c) {
                group(c, std::false_type{});
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (MODE == kRowMax) {
            // the lanes sharing n differ in g (lane bits 4, 5)
            mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, 16, 64));
            mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, 32, 64));
            const uint32_t m = (pack_bf16x2(mx, 0.0f) & 0x7fffu);
            if (g == 0 && nvalid) atomicMax(reinterpret_cast<uint32_t*>(p.w_scale) + n, m);
        }
    };

    // Walk row tiles rt0, rt0 + rstep, ..., loading each tile's registers one
    // tile ahead (two register sets, alternating).
    int rt = (int)(blockIdx.x / (unsigned)p.stripes);
    TileRegs<RP> ta, tb;
    load_tile(rt, ta);
    __syncthreads();                                   // A^T staged
    while (rt < p.row_tiles) {
        const int r1 = rt + rstep;
        load_tile(r1, tb);
        __builtin_amdgcn_sched_barrier(0);
        compute(rt, ta);
        __builtin_amdgcn_sched_barrier(0);
        if (r1 >= p.row_tiles) break;
        const int r2 = r1 + rstep;
        load_tile(r2, ta);
        __builtin_amdgcn_sched_barrier(0);
        compute(r1, tb);
        __builtin_amdgcn_sched_barrier(0);
        rt = r2;
    }
}

__global__ void k_zero_u32(uint32_t* x, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = 0u;
}

// Workgroups of one kernel that fit on a CU at once (cached per kernel).
template <int RP, int MODE, bool BVEC>
int resident_per_cu()
{
    static int cached = 0;
    if (cached > 0) return cached;
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(&k_lora_stripes<RP, MODE, BVEC>),
                                                     kThreads, 0) != hipSuccess || nb < 1)
        nb = 1;
    cached = nb;
    return nb;
}

// Grid: stripes x walkers, walkers per stripe chosen so that every workgroup is
// resident at once (no second wave of workgroups) and no walker is idle.
template <int RP, int MODE, bool BVEC>
dim3 stripe_grid(const Args& p, int cus)
{
    const int64_t slots = (int64_t)cus * resident_per_cu<RP, MODE, BVEC>();
    const int64_t walkers = max((int64_t)1, min((int64_t)p.row_tiles, slots / p.stripes));
    return dim3((unsigned)(walkers * p.stripes));
}

template <int RP, bool BVEC>
void launch_rp(const Args& p, bool merge_only, int cus, hipStream_t st)
{
    const dim3 block(kThreads);
    if (merge_only) {
        const dim3 gm = stripe_grid<RP, kMergeOnly, BVEC>(p, cus);
        hipLaunchKernelGGL((k_lora_stripes<RP, kMergeOnly, BVEC>), gm, block, 0, st, p);
        return;
    }
    const dim3 vgrid((unsigned)((p.N + 255) / 256)), vblock(256);
    const dim3 g1 = stripe_grid<RP, kRowMax, BVEC>(p, cus);
    hipLaunchKernelGGL(k_zero_u32, vgrid, vblock, 0, st, reinterpret_cast<uint32_t*>(p.w_scale), p.N);
    hipLaunchKernelGGL((k_lora_stripes<RP, kRowMax, BVEC>), g1, block, 0, st, p);
    if (p.w_merged) {
        const dim3 g2 = stripe_grid<RP, kQuantizeMerged, BVEC>(p, cus);
        hipLaunchKernelGGL((k_lora_stripes<RP, kQuantizeMerged, BVEC>), g2, block, 0, st, p);
    } else {
        const dim3 g2 = stripe_grid<RP, kQuantize, BVEC>(p, cus);
        hipLaunchKernelGGL((k_lora_stripes<RP, kQuantize, BVEC>), g2, block, 0, st, p);
    }
}

}  // namespace

int launch_lora_requant(const uint16_t* w, int64_t N, int64_t K, int64_t ldw, const uint16_t* a,
                        const uint16_t* b, int64_t rank, float lora_scale, uint8_t* wq, int64_t ldq,
                        float* w_scale, uint16_t* w_merged, hipStream_t stream)
{
    if (rank < 1 || rank > 128)
        return set_error(VDN_FP8_EINVAL, "requantize_weight: LoRA rank %lld outside 1..128", (long long)rank);
    if (K % 16) return set_error(VDN_FP8_EINVAL, "requantize_weight: the LoRA path needs K %% 16 == 0 (K=%lld)", (long long)K);
    if ((uintptr_t)a % 16) return set_error(VDN_FP8_EINVAL, "requantize_weight: lora_a must be 16-byte aligned");
    if ((uintptr_t)b % 2) return set_error(VDN_FP8_EINVAL, "requantize_weight: lora_b must be 2-byte aligned");
    if (w_merged && ((uintptr_t)w_merged % 8)) return set_error(VDN_FP8_EINVAL, "requantize_weight: w_merged must be 8-byte aligned");
    if (wq && (((uintptr_t)wq % 8) || (ldq % 8))) return set_error(VDN_FP8_EINVAL, "requantize_weight: wq rows must be 8-byte aligned");
    if (w_scale && ((uintptr_t)w_scale % 4)) return set_error(VDN_FP8_EINVAL, "requantize_weight: w_scale must be 4-byte aligned");
    if ((int64_t)kTileRows * ldw * 2 > 0x7fffffffLL || (rank + 33) * K * 2 > 0x7fffffffLL ||
        (wq && (int64_t)kTileRows * ldq > 0x7fffffffLL))
        return set_error(VDN_FP8_EINVAL, "requantize_weight: rows too long for the LoRA path");
    if ((N + kTileRows - 1) / kTileRows > (1 << 24) || (K + kTileCols - 1) / kTileCols > (1 << 16))
        return set_error(VDN_FP8_EINVAL, "requantize_weight: shape [%lld, %lld] too large for the LoRA path",
                         (long long)N, (long long)K);
    const bool merge_only = wq == nullptr;
    const int b_vec = (rank % 8 == 0) && ((uintptr_t)b % 16 == 0);
    const int wm16 = w_merged && ((uintptr_t)w_merged % 16 == 0);
    const int cus = device_cus();
    if (cus <= 0) return set_error(VDN_FP8_ELAUNCH, "requantize_weight: cannot query the device's compute units");
    Args p{w, N, K, ldw, a, b, rank, b_vec, lora_scale, wq, ldq, w_scale, w_merged, wm16,
           (int)((K + kTileCols - 1) / kTileCols), (int)((N + kTileRows - 1) / kTileRows)};
    const int rp = (int)((rank + 31) / 32) * 32;
#define VDN_LORA_RP(R)                                                      \
    do {                                                                    \
        if (b_vec) launch_rp<R, true>(p, merge_only, cus, stream);          \
        else launch_rp<R, false>(p, merge_only, cus, stream);               \
    } while (0)
    switch (rp) {
        case 32: VDN_LORA_RP(32); break;
        case 64: VDN_LORA_RP(64); break;
        case 96: VDN_LORA_RP(96); break;
        default: VDN_LORA_RP(128); break;
    }
#undef VDN_LORA_RP
    return check_launch("requantize_weight (LoRA)");
}

}  // namespace vdn
