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
// Two kernels. k_lora_rows (further down; rank <= 64, K <= 5120, 16-byte rows)
// reads W once: a workgroup holds a group of whole rows of W' in registers
// until their maximum is known, then writes the codes. k_lora_stripes (first)
// serves everything else -- ranks up to 128, longer rows, unaligned operands,
// merge-only calls -- in two passes:
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

#include <algorithm>
#include <type_traits>
#include <utility>

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

// Bytes of `rows` rows of W (bf16, row stride ld elements) up to the end of the last
// row's K elements: the caller's W may end right after them, so no read range of a
// descriptor reaches past (ld - K) padding of the last row.
__device__ __forceinline__ int64_t w_span_bytes(int64_t rows, int64_t ld, int64_t K)
{
    return rows > 0 ? ((rows - 1) * ld + K) * 2 : 0;
}
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
            (void*)(p.w + n0 * p.ldw), 0, (int)w_span_bytes(rows, p.ldw, p.K), 0x00020000);
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
                    store_b128_settled<0>(u32x4(wm[4], wm[5], wm[6], wm[7]), mr, off + 16, 0);
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

// ---------------------------------------------------------------------------
// One pass: whole rows of W' held in registers (k_lora_rows)
// ---------------------------------------------------------------------------
// A workgroup of eight waves owns a group of 32 rows of W and every column. The
// columns advance in 256-wide chunks; wave w merges columns 32 w .. 32 w + 31 of
// each chunk for all 32 rows, so a lane (row n = lane % 32, half h = lane / 32)
// holds 16 consecutive columns of one row per chunk: all of its row's share of
// W' stays in VGPRs (8 words a chunk, 160 at K = 5120) until the row maximum is
// known, and W is read from HBM exactly once.
//
// The rank-r update is v_mfma_f32_32x32x16_bf16 with MFMA row i = a column of
// the chunk, MFMA column j = a row n of W, reduction = rank: the B operand
// (B[n][...]) stays in VGPRs for the whole group, the A operand comes from the
// chunk's slice of A, staged in LDS in its natural [rank][column] layout and
// read with ds_read_b64_tr_b16 (gfx950's transposing LDS read: lane i of each
// 16-lane group receives element i % 4 of the 8-byte row addressed by lane
// 4 j + i / 4, for j = 0..3), so no transposed copy of A is needed. MFMA row i
// stands for column 16 ((i / 4) % 2) + 4 (i / 8) + i % 4 of the wave's 32, which
// makes accumulator r of lane (n, h) column 16 h + r.
//
// Both streams reach LDS by global -> LDS copies: W (from HBM) through four
// 16 KiB stages, A (from L2) through three; every wave issues its share of both
// (2 W and RP / 16 A copies of 1 KiB per chunk, spread over the previous
// chunk's merge). A wave's memory counter orders its operations as issued, so
// slice c of A is requested after chunk c of W and before chunk c + 1: one
// exact wait for slice c then covers both, while W of chunks c + 1 and c + 2
// stays in flight (chunk c + 3 goes out after it), and the merge of chunk c
// runs meanwhile. After the last chunk the row maxima meet in LDS; the next
// group's first four W chunks are requested, and the codes leave through LDS
// (the A stages' space, two alternating buffers) as whole 1 KiB row pieces,
// four chunks at a time, while those chunks stream in; then the next group's
// first A slices and B rows. The grid is persistent, one workgroup per CU, the
// rows spread evenly over its groups (up to 32 rows each).
namespace rows {
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kLanes;   // 512
constexpr int kRows = 32;                   // rows of W per group (at most)
constexpr int kChunk = 256;                 // columns per chunk (32 per wave)
constexpr int kMaxChunks = 20;              // K <= 5120
constexpr int kWStages = 4;                 // W chunks in LDS (16 KiB each)
constexpr int kAStages = 3;                 // A slices in LDS (RP x 512 bytes each)
constexpr int kRowB = kChunk * 2;           // bytes of one row of a chunk (W) or one rank row of a slice (A)
constexpr int kWStage = kRows * kRowB;      // 16 KiB

// Memory operations a wave has issued after slice c of A by the time it waits
// for chunk c (wc W copies and ac A copies per chunk, nb B loads per group).
// Order: in the first group W0 A0 W1 A1 W2 A2 W3; in later groups, requested
// while the previous group's codes went out, W0-W3, the code stores, A0-A2,
// the B loads; then, after the wait of each chunk k >= 1, A(k + 2) and W(k + 3).
constexpr int ops_after_a(int c, bool first, int nch, int wc, int ac, int nb)
{
    int count = 0;
    bool seen = false;
    auto op = [&](bool is_a, int idx, int n) {
        if (seen) count += n;
        if (is_a && idx == c) seen = true;
    };
    if (first) {
        for (int k = 0; k < kWStages && k < nch; ++k) {
            op(false, k, wc);
            if (k < kAStages) op(true, k, ac);
        }
    } else {
        for (int k = 0; k < kAStages && k < nch; ++k) op(true, k, ac);
        op(false, -1, nb);
    }
    for (int k = 1; k < c; ++k) {
        if (k + kAStages - 1 < nch) op(true, k + kAStages - 1, ac);
        if (k + kWStages - 1 < nch) op(false, k + kWStages - 1, wc);
    }
    return count;
}
}  // namespace rows

struct RowArgs {
    const uint16_t* w;
    int64_t N, K, ldw;
    const uint16_t* a;   // [rank, K], rows K elements apart
    const uint16_t* b;   // [N, rank]
    int64_t rank;
    float lora_scale;
    uint8_t* wq;         // rows ldq bytes apart, 16-byte aligned
    int64_t ldq;
    float* w_scale;
    uint16_t* w_merged;  // MERGED only: rows ldw apart, 16-byte aligned
    int nch;             // ceil(K / 256)
    int rows_pg;         // rows of W per group (<= 32; fewer so that the groups fill every CU)
    int groups;          // ceil(N / rows_pg)
};

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// One wave-wide global -> LDS copy of 16 bytes per lane: lane L's bytes at
// buffer offset voff + soff (soff wave-uniform) land at LDS byte lds + 16 L.
// Inline assembly, so that the compiler does not make every later LDS read wait
// for it; the kernel waits on vmcnt itself. M0 carries the LDS address (restored
// afterwards); s_nop covers the M0-write -> LDS-DMA hazard. kNT: non-temporal
// (data read exactly once, such as the weight).
template <bool kNT = false>
__device__ __forceinline__ void copy16_to_lds(i32x4_t rsrc, uint32_t lds, uint32_t voff, uint32_t soff)
{
    uint32_t saved;
    if constexpr (kNT)
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %1\n\t"
            "s_nop 0\n\t"
            "buffer_load_dwordx4 %2, %3, %4 offen nt lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
            : "memory");
    else
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %1\n\t"
            "s_nop 0\n\t"
            "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
            : "memory");
}

__device__ __forceinline__ i32x4_t rsrc_words(const void* base, int64_t bytes)
{
    const uint64_t a = (uint64_t)base;
    bytes = max(min(bytes, (int64_t)0x7fffffff), (int64_t)0);
    return i32x4_t{__builtin_amdgcn_readfirstlane((int)(a & 0xffffffffu)),
                   __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffffu)),
                   __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
}

// s_waitcnt with vmcnt = VM (63: no condition on memory operations) and
// lgkmcnt = 0 (this wave's LDS accesses done).
template <int VM>
__device__ __forceinline__ void wait_vm_lgkm()
{
    __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (0 << 8) | ((VM >> 4) << 14));
}

// The wait, then all waves meet. The scheduling barriers keep the compiler from
// moving instructions across.
template <int VM>
__device__ __forceinline__ void rows_sync()
{
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_lgkm<VM>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// f(std::integral_constant<int, i>) for i = 0 .. N - 1, unrolled at compile time
// (the chunk index is then a constant expression, e.g. for a wait's count).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>)
{
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f)
{
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int RP, int NCH, bool BVEC, bool MERGED>
__global__ __launch_bounds__(rows::kThreads) void k_lora_rows(RowArgs p)
{
    using namespace rows;
    constexpr int kSteps = RP / 16;                  // rank steps of 16 (one MFMA each)
    constexpr int kAStage = RP * kRowB;
    constexpr int kWCopies = kWStage / 1024 / rows::kWaves;  // 1 KiB W copies per wave per chunk (2)
    constexpr int kACopies = kAStage / 1024 / rows::kWaves;  // 1 KiB A copies per wave per chunk (RP / 16)
    static_assert(kACopies + kWCopies <= 8, "a chunk's copies are spread over the eight words of a merge");
    constexpr int kWArea = kWStages * kWStage;
    constexpr int kAArea = kAStages * kAStage;
    // The codes leave in parts of kPartC chunks (kPartC x 256 bytes of every row),
    // staged by rows in the A area in two alternating buffers (rows padded by 16
    // bytes: the 16 rows one 16-byte write of a quarter-wave covers fall on 16
    // different bank quads); the last KiB of the A area holds the row maxima.
    constexpr int kRedOff = kWArea + kAArea - 1024;
    constexpr int kPartC = (2 * kRows * (4 * kChunk + 16) <= kAArea - 1024) ? 4
                           : (2 * kRows * (2 * kChunk + 16) <= kAArea - 1024) ? 2 : 1;
    constexpr int kParts = NCH / kPartC;
    constexpr int kCRow = kPartC * kChunk + 16;
    constexpr int kCBuf = kRows * kCRow;
    static_assert(NCH % kPartC == 0 && 2 * kCBuf <= kAArea - 1024, "codes staging exceeds the A area");
    // One 1 KiB store covers kRowsPerStore rows of a part; a wave stores kPartC of them
    // per part, one while each chunk of the next part is formed.
    constexpr int kRowsPerStore = 1024 / (kPartC * kChunk);
    static_assert(kRows / kRowsPerStore == kPartC * rows::kWaves, "one store per wave and chunk");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kWArea + kAArea];
    uint32_t* const red = reinterpret_cast<uint32_t*>(smem + kRedOff);

    const int tid = threadIdx.x, lane = tid & (kLanes - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nl = lane & 31, h = lane >> 5;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_void_t*)smem;
    const int64_t rpg = p.rows_pg;   // rows of a group (rows past it read as zeros, store nothing)

    // Copy i of a wave's W share moves rows 2 d and 2 d + 1 (d = 2 wave + i) of a chunk; lane L
    // fills row 2 d + L / 32, 16-byte piece L % 32, which holds the row's logical
    // piece (L % 32) ^ (row % 16): the 16 rows a quarter-wave reads at one column
    // fall on 16 different bank quads. Copy i of its A share moves rank rows 2 d and
    // 2 d + 1 (d = kACopies wave + i) of a slice, piece (L % 32) ^ (4 (row % 4)): the
    // four rank rows of one transposing read sit in four different 64-byte windows.
    // The row of copy i is 2 d + h with 2 d even, so the piece a lane fetches is
    // ((L % 32) ^ h) ^ ((2 d) % 16) for W and ((L % 32) ^ 4 h) ^ 4 ((2 d) % 4) for A:
    // a lane part held in registers (h rows down, that piece), xor'ed with a
    // per-copy constant, and a uniform part (rows 2 d, the chunk) carried by the
    // instruction's scalar offset.
    const i32x4_t arsrc = rsrc_words(p.a, p.rank * p.K * 2);
    const uint32_t ldw2 = (uint32_t)(p.ldw * 2), k2 = (uint32_t)(p.K * 2);
    const uint32_t w_lrow = (uint32_t)h * ldw2, w_lpc = (uint32_t)((nl ^ h) << 4);
    const uint32_t a_lrow = (uint32_t)h * k2, a_lpc = (uint32_t)((nl ^ (4 * h)) << 4);
    // W is read once (non-temporal copies); the codes are stored non-temporally too
    // (read by later GEMMs, not by the next kernel): [15360, 5120] rank 64 with W from
    // HBM 52.9 us against 57.6 us with both cached
    auto copy_w1 = [&](i32x4_t wrs, int c, int st, int i) {
        const int d = kWCopies * wave + i;
        uint32_t so = (uint32_t)(2 * d) * ldw2;
        asm volatile("" : "+s"(so));   // the chunk's part added here, not kept per chunk
        copy16_to_lds<true>(wrs, lds_base + (uint32_t)(st * kWStage + d * 1024),
                      (w_lpc ^ (uint32_t)(((2 * d) & 15) << 4)) + w_lrow, so + (uint32_t)(c * kRowB));
    };
    auto copy_a1 = [&](int c, int st, int i) {
        const int d = kACopies * wave + i;
        uint32_t so = (uint32_t)(2 * d) * k2;
        asm volatile("" : "+s"(so));
        copy16_to_lds(arsrc, lds_base + (uint32_t)(kWArea + st * kAStage + d * 1024),
                      (a_lpc ^ (uint32_t)(((2 * d) & 3) << 6)) + a_lrow, so + (uint32_t)(c * kRowB));
    };
    auto copy_w = [&](i32x4_t wrs, int c, int st) {
#pragma unroll
        for (int i = 0; i < kWCopies; ++i) copy_w1(wrs, c, st, i);
    };
    auto copy_a = [&](int c, int st) {
#pragma unroll
        for (int i = 0; i < kACopies; ++i) copy_a1(c, st, i);
    };
    // W descriptor of a group (empty past the last group: reads zeros, touches no memory)
    auto w_rsrc = [&](int64_t n0) {
        const int64_t rows = n0 < p.N ? min(p.N - n0, rpg) : 0;
        return rsrc_words(p.w + n0 * p.ldw, w_span_bytes(rows, p.ldw, p.K));
    };
    // Transposing reads: lane (group G = lane / 16, j = (lane / 4) % 4, q = lane % 4)
    // addresses rank row 8 h + j (+ 16 s + 4 half) at the four columns MFMA rows
    // 16 (G % 2) + 4 q .. + 3 stand for: 32 wave + 16 (q % 2) + 8 (G % 2) + 4 (q / 2).
    const int tj = (lane >> 2) & 3, tq = lane & 3, tg = (lane >> 4) & 1;
    const uint32_t tr_off = (uint32_t)((8 * h + tj) * kRowB +
                                       (((4 * wave + 2 * (tq & 1) + tg) ^ (4 * tj)) << 4) + 8 * (tq >> 1));
    // This lane's W pieces in a stage: row n, logical pieces 4 wave + 2 h + e.
    // (piece 4 wave + 2 h + 1 sits at the other 16 bytes of the pair: 4 wave + 2 h is even)
    const uint32_t wrd0 = (uint32_t)(nl * kRowB + (((4 * wave + 2 * h) ^ (nl & 15)) << 4));

    const int lcol = 32 * wave + 16 * h;                       // first column of the lane in a chunk
    const int nvalid = (int)((p.K - lcol + kChunk - 1) / kChunk);   // chunks with this lane's columns < K
    auto col_in = [&](int c) {
        int nv = nvalid;
        asm volatile("" : "+v"(nv));
        return c < nv;
    };
    auto voff_at = [&](uint32_t base, int c) {
        asm volatile("" : "+v"(base));
        return col_in(c) ? base : kDropped;
    };

    // B operand of rank step s: B[n][16 s + 8 h .. + 7], zero beyond the rank; the
    // raw 16-byte loads are masked where they are first used.
    bf16x8_t braw[kSteps];
    auto load_b = [&](int64_t n0) {
        const int64_t rows = n0 < p.N ? min(p.N - n0, rpg) : 0;
        const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(p.b + n0 * p.rank), 0, (int)(rows * p.rank * 2), 0x00020000);
#pragma unroll
        for (int s = 0; s < kSteps; ++s)
            braw[s] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(
                br, (uint32_t)((nl * p.rank + 16 * s + 8 * h) * 2), 0, 0));
    };

    int g = blockIdx.x;
    if (g >= p.groups) return;
    // Prologue of the first group: B, then W0 A0 W1 A1 W2 A2 W3.
    load_b((int64_t)g * rpg);
    {
        const i32x4_t wrs = w_rsrc((int64_t)g * rpg);
#pragma unroll
        for (int c = 0; c < kWStages && c < NCH; ++c) {
            copy_w(wrs, c, c);
            if (c < kAStages) copy_a(c, c);
        }
    }

    uint32_t wr[NCH][8];
    bool first = true;
    for (; g < p.groups; g += gridDim.x) {
        const int64_t n0 = (int64_t)g * rpg;
        const int64_t rows = min(p.N - n0, rpg);
        const i32x4_t wrs = w_rsrc(n0);
        bf16x8_t bop[kSteps];

        // Merge: W' = bf16(W + bf16(scale * B A)) per chunk, into wr[c]; mx keeps the
        // magnitude maximum of the valid columns' binary32 sums before their rounding
        // (rounding to nearest is monotone and symmetric, so the row maximum of |W'| is
        // that maximum rounded; v_maximum3_f32 takes two magnitudes an instruction and
        // propagates NaN). Software-pipelined by one
        // chunk: chunk c's LDS reads go out, then chunk c - 1's VALU work (its MFMAs
        // have had a chunk's time to finish) hides their latency, then chunk c's MFMAs
        // run while the next chunk waits for its data.
        float mx = 0.0f;
        f32x16_t acc;   // chunk c's sums, read by back(c) before mfmas(c + 1) rewrites them
        auto front = [&](int c) {
            if (c == 0) {
                // (masked past the first wait: the B loads are long done by then)
#pragma unroll
                for (int s = 0; s < kSteps; ++s)
                    bop[s] = (!BVEC || 16 * s + 8 * h < p.rank) ? braw[s] : bf16x8_t{};
            }
        };
        auto reads_w = [&](int c) {
            const uint8_t* ws = smem + (c % kWStages) * kWStage;
            const uint4 x = *reinterpret_cast<const uint4*>(ws + wrd0);
            const uint4 y = *reinterpret_cast<const uint4*>(ws + (wrd0 ^ 16u));
            wr[c][0] = x.x; wr[c][1] = x.y; wr[c][2] = x.z; wr[c][3] = x.w;
            wr[c][4] = y.x; wr[c][5] = y.y; wr[c][6] = y.z; wr[c][7] = y.w;
        };
        // the A operand of rank steps s0 .. s1 - 1
        auto reads_a = [&](int c, bf16x8_t (&aop)[kSteps], int s0, int s1) {
            const uint8_t* st = smem + kWArea + (c % kAStages) * kAStage + tr_off;
#pragma unroll
            for (int s = 0; s < kSteps; ++s) {
                if (s < s0 || s >= s1) continue;
                typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
                const lds_s16x4_t* p0 = (const lds_s16x4_t*)(lds_void_t*)(st + (16 * s) * kRowB);
                const lds_s16x4_t* p1 = (const lds_s16x4_t*)(lds_void_t*)(st + (16 * s + 4) * kRowB);
                const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_s16x4_t*>(p0));
                const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_s16x4_t*>(p1));
                aop[s] = __builtin_bit_cast(bf16x8_t, (short __attribute__((ext_vector_type(8)))){
                    lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
            }
        };
        auto mfmas = [&](int, const bf16x8_t (&aop)[kSteps]) {
            f32x16_t a = f32x16_t{};
#pragma unroll
            for (int s = 0; s < kSteps; ++s) a = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aop[s], bop[s], a, 0, 0, 0);
            acc = a;
        };
        // Copy j (0 .. kACopies + kWCopies - 1) of chunk c: every wave is past chunk
        // c - 1, so its stages can take slice c + kAStages - 1 (A, copies j < kACopies)
        // and chunk c + kWStages - 1 (W, the others), requested in that order.
        auto copy_j = [&](int c, int j) {
            if (j < kACopies) {
                if (c >= 1 && c + kAStages - 1 < NCH) copy_a1(c + kAStages - 1, (c + kAStages - 1) % kAStages, j);
            } else if (j < kACopies + kWCopies) {
                if (c >= 1 && c + kWStages - 1 < NCH) copy_w1(wrs, c + kWStages - 1, (c + kWStages - 1) % kWStages, j - kACopies);
            }
        };
        // back(c, cn): chunk c's merge, with chunk cn's copies spread over it (one after
        // each of the first words), so the copy path works while the VALU does.
        auto back = [&](int c, int cn) {
            const f32x16_t& a = acc;
            float gm = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                if (cn >= 0) {
                    __builtin_amdgcn_sched_barrier(0);
                    copy_j(cn, d);
                    __builtin_amdgcn_sched_barrier(0);
                }
                // bf16(delta) as binary32, one conversion per value (its operand the
                // scale multiply, not the accumulator itself)
                const float dlo = round_bf16_hi(a[2 * d] * p.lora_scale), dhi = round_bf16_hi(a[2 * d + 1] * p.lora_scale);
                const float lo = bf16_lo(wr[c][d]) + dlo, hi = bf16_hi(wr[c][d]) + dhi;
                uint32_t m = pack_bf16x2(lo, hi);
                asm volatile("" : "+v"(m));
                wr[c][d] = m;
                gm = __builtin_elementwise_maximum(gm, __builtin_elementwise_maximum(__builtin_fabsf(lo), __builtin_fabsf(hi)));
            }
            mx = col_in(c) ? __builtin_elementwise_maximum(mx, gm) : mx;
        };
        static_for<NCH>([&](auto ic) {
            constexpr int c = decltype(ic)::value;
            // Slice c (and with it chunk c, requested before it) has landed once only
            // the operations issued after it may be pending.
            constexpr int kFirst = ops_after_a(c, true, NCH, kWCopies, kACopies, kSteps);
            constexpr int kLater = ops_after_a(c, false, NCH, kWCopies, kACopies, kSteps);
            if (first) rows_sync<(kFirst > 63 ? 63 : kFirst)>();
            else rows_sync<(kLater > 63 ? 63 : kLater)>();
            front(c);
            // (half of the A operand before the VALU work, half after: all of it held
            // across that work would cost registers the rows of W' need)
            bf16x8_t aop[kSteps];
            reads_w(c);
            reads_a(c, aop, 0, kSteps / 2);
            __builtin_amdgcn_sched_barrier(0);
            if (c >= 1) back(c - 1, c);
            __builtin_amdgcn_sched_barrier(0);
            reads_a(c, aop, kSteps / 2, kSteps);
            mfmas(c, aop);
            __builtin_amdgcn_sched_barrier(0);
        });
        back(NCH - 1, -1);

        // Row maxima: the two halves of each lane's words, the two lanes of a row,
        // then the eight waves through LDS (in the last KiB of the A area: written
        // once every wave is done with the last chunk).
        uint32_t m16 = pack_bf16x2(mx, 0.0f) & 0x7fffu;   // bf16 magnitude bits (NaN above inf)
        m16 = max(m16, (uint32_t)__shfl_xor((int)m16, 32, 64));
        rows_sync<63>();
        if (h == 0) red[wave * kRows + nl] = m16;
        rows_sync<63>();
        uint32_t mbits = 0u;
#pragma unroll
        for (int w8 = 0; w8 < rows::kWaves; ++w8) mbits = max(mbits, red[w8 * kRows + nl]);
        const float s32 = row_scale(bf16_to_f32((uint16_t)mbits));
        {
            const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(p.w_scale + n0), 0, (int)(rows * 4), 0x00020000);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(s32), sr,
                                                  (wave == 0 && h == 0) ? (uint32_t)(nl * 4) : kDropped, 0, 0);
        }
        const float sb = round_bf16(s32);
        const float r = 1.0f / sb;
        // every wave holds the same 32 rows: the branch is uniform over the workgroup
        const bool exact = __builtin_amdgcn_ballot_w64(!__builtin_isfinite(sb)) != 0;

        // The next group's first W chunks (the W stages are free: every wave has read
        // its last chunk), then the codes, part by part.
        const int gn = g + (int)gridDim.x;
        const bool more = gn < p.groups;
        const i32x4_t nrs = w_rsrc((int64_t)gn * rpg);
#pragma unroll
        for (int c = 0; c < kWStages && c < NCH; ++c) copy_w(nrs, c, c);
        const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(p.wq + n0 * p.ldq), 0, (int)(rows * p.ldq), 0x00020000);
        const __amdgpu_buffer_rsrc_t mr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(MERGED ? p.w_merged + n0 * p.ldw : nullptr), 0, MERGED ? (int)(rows * p.ldw * 2) : 0, 0x00020000);
        // (one uniform branch per chunk around the quotients only)
        auto codes_chunk = [&](int c, int c0, uint8_t* cst) {
            uint32_t q[4];
            if (exact) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint2 v = make_uint2(wr[c][2 * i], wr[c][2 * i + 1]);
                    // opaque, so that the compiler does not unpack every word once for
                    // both paths ahead of the branch
                    asm volatile("" : "+v"(v.x), "+v"(v.y));
                    q[i] = codes4_exact(v, sb);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) q[i] = codes4(make_uint2(wr[c][2 * i], wr[c][2 * i + 1]), r);
            }
            *reinterpret_cast<uint4*>(cst + nl * kCRow + (c - c0) * kChunk + lcol) = make_uint4(q[0], q[1], q[2], q[3]);
            if (MERGED) {
                const uint32_t wv = (uint32_t)((nl * p.ldw + lcol) * 2);
                const uint32_t off = voff_at(wv, c);
                store_b128_settled<0>(u32x4(wr[c][0], wr[c][1], wr[c][2], wr[c][3]), mr, off, c * kRowB);
                store_b128_settled<0>(u32x4(wr[c][4], wr[c][5], wr[c][6], wr[c][7]), mr, off + 16, c * kRowB);
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        // Store j of a wave in a part: rows kRowsPerStore (kPartC wave + j) .., lane L at
        // row + L / (16 kPartC), bytes 16 (L % (16 kPartC)) of the part's kPartC x 256.
        // Columns past K and rows past the group go out of range.
        constexpr int kLanesPerRow = 16 * kPartC;
        const int srow = lane / kLanesPerRow, sbyte = 16 * (lane % kLanesPerRow);
        uint4 pend[kPartC];
        auto read_part = [&](const uint8_t* cst) {
#pragma unroll
            for (int j = 0; j < kPartC; ++j) {
                const int row = kRowsPerStore * (kPartC * wave + j) + srow;
                pend[j] = *reinterpret_cast<const uint4*>(cst + row * kCRow + sbyte);
            }
        };
        auto store_piece = [&](int c0, int j) {
            const int row = kRowsPerStore * (kPartC * wave + j) + srow;
            const uint32_t off = ((int64_t)c0 * kChunk + sbyte < p.K) ? (uint32_t)(row * p.ldq + sbyte) : kDropped;
            store_b128_settled<kBufferLoadOnce>(__builtin_bit_cast(i32x4_t, pend[j]), qr, off, c0 * kChunk);
        };
        // Part q's codes go to buffer q % 2 while part q - 1's pieces are stored; then
        // (all of part q in LDS, every wave past its reads of part q - 1) part q's pieces
        // are read. The buffer part q + 1 overwrites is part q - 1's, read before that.
        static_for<kParts>([&](auto iq) {
            constexpr int q = decltype(iq)::value;
            uint8_t* const cst = smem + kWArea + (q % 2) * kCBuf;
#pragma unroll
            for (int j = 0; j < kPartC; ++j) {
                codes_chunk(q * kPartC + j, q * kPartC, cst);
                if (q >= 1) store_piece((q - 1) * kPartC, j);
            }
            rows_sync<63>();
            read_part(cst);
        });
        // every wave's reads of the last part are done before the A stages are refilled
        rows_sync<63>();
#pragma unroll
        for (int j = 0; j < kPartC; ++j) store_piece((kParts - 1) * kPartC, j);
        // The next group's first A slices (the A area is free again) and B rows.
        if (more) {
#pragma unroll
            for (int c = 0; c < kAStages && c < NCH; ++c) copy_a(c, c);
        }
        load_b((int64_t)gn * rpg);
        first = false;
    }
    // No copy may still be writing LDS when the workgroup ends.
    wait_vm_lgkm<0>();
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
    // One pass with the rows in registers: codes wanted, rank <= 64 with 16-byte B
    // rows, K <= 5120, 16-byte rows everywhere.
    const bool one_pass = !merge_only && rank <= 64 && b_vec && K <= (int64_t)rows::kChunk * rows::kMaxChunks &&
                          aligned(w, 16) && ldw % 8 == 0 && aligned(wq, 16) && ldq % 16 == 0 &&
                          (!w_merged || aligned(w_merged, 16)) && (int64_t)rows::kRows * ldw * 2 <= 0x7fffffffLL &&
                          (int64_t)rows::kRows * ldq <= 0x7fffffffLL && rank * K * 2 <= 0x7fffffffLL;
    if (one_pass) {
        // persistent grid, one workgroup per CU: as many rounds of groups as 32-row
        // groups would need, then the rows spread evenly over rounds x CUs groups
        // ([15360, *] on 256 CUs: 512 groups of 30 rows, two per workgroup)
        const int64_t rounds = (N + (int64_t)rows::kRows * cus - 1) / ((int64_t)rows::kRows * cus);
        const int rows_pg = (int)((N + rounds * cus - 1) / (rounds * cus));
        RowArgs r{w, N, K, ldw, a, b, rank, lora_scale, wq, ldq, w_scale, w_merged,
                  (int)((K + rows::kChunk - 1) / rows::kChunk), rows_pg, (int)((N + rows_pg - 1) / rows_pg)};
        const dim3 grid((unsigned)min((int64_t)r.groups, (int64_t)cus)), block(rows::kThreads);
        // chunk-count instances: 8 (K <= 2048), 16 (K <= 4096), 20 (K <= 5120); chunks past
        // K read nothing and store nothing
#define VDN_LORA_ROWS(R, C)                                                                            \
    do {                                                                                               \
        if (w_merged) hipLaunchKernelGGL((k_lora_rows<R, C, true, true>), grid, block, 0, stream, r);  \
        else hipLaunchKernelGGL((k_lora_rows<R, C, true, false>), grid, block, 0, stream, r);          \
    } while (0)
#define VDN_LORA_ROWS_RP(R)                              \
    do {                                                 \
        if (r.nch <= 8) VDN_LORA_ROWS(R, 8);             \
        else if (r.nch <= 16) VDN_LORA_ROWS(R, 16);      \
        else VDN_LORA_ROWS(R, 20);                       \
    } while (0)
        if (rank <= 32) VDN_LORA_ROWS_RP(32);
        else VDN_LORA_ROWS_RP(64);
#undef VDN_LORA_ROWS_RP
#undef VDN_LORA_ROWS
        return check_launch("requantize_weight (LoRA, one pass)");
    }
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
