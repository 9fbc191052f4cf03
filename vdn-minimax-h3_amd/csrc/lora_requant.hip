// Fused LoRA merge + rowwise weight requantization (gfx950).
//
//   W'[n][k]   = bf16(W[n][k] + bf16(lora_scale * sum_j B[n][j] A[j][k]))
//   w_scale[n] = max(max_k |W'[n][k]| / 448, 1e-12)
//   wq[n][k]   = e4m3(bf16(W'[n][k] / bf16(w_scale[n])))
//
// The reference merges in place on the bf16 weight (lora.py:91-92) and then
// quantizes it in eager torch (fp8_linear.py:262-267): three full passes over
// W. Here one workgroup owns 16 rows of W: it computes the rank-r update with
// bf16 MFMA (products of bf16 values are exact in fp32, accumulation is fp32,
// as in the reference's fp32 matmul), adds it to W as it streams W in, keeps
// W' in VGPRs while the row maxima are reduced, then writes the e4m3 codes.
// HBM traffic is W once (2 B/elt) plus the codes (1 B/elt); A and B (a few
// hundred KiB) stay in L2. Rows wider than the register-resident limit
// recompute the update in a second sweep instead (W is re-read from L2/MALL).
//
// MFMA orientation: v_mfma_f32_16x16x32_bf16 with the MFMA row index = k
// (16 columns of W), column index = n (16 rows of W), reduction = rank. Its
// result leaves each lane with 4 consecutive k of one row n, so W and W' move
// 8 bytes per lane and the codes 4 bytes per lane.
#include <stdint.h>

#include "vdn_common.h"

namespace vdn {
namespace {

constexpr int kRows = 16;             // rows of W per workgroup
constexpr int kWaves = 16;            // 1024 threads
constexpr int kLanes = 64;
constexpr int kChunk = kWaves * 16;   // columns per sweep step (one 16x16 tile per wave)
constexpr int kPad = 4;               // LDS row padding (elements) against bank conflicts
constexpr int kStride = kChunk + kPad;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct Args {
    const uint16_t* w;
    int64_t N, K, ldw;
    const uint16_t* a;   // [rank, K]
    const uint16_t* b;   // [N, rank]
    int64_t rank;
    float lora_scale;
    uint8_t* wq;
    int64_t ldq;
    float* w_scale;
    uint16_t* w_merged;  // nullable, row stride ldw
};

// A[:, k0 : k0 + kChunk] (rows j < RP, zero beyond rank and K) travels to LDS in
// two halves, so the global loads of the next step can be in flight while the
// current step computes: load_a fills this thread's pieces, store_a writes them.
template <int RP>
struct APieces {
    static constexpr int kPieces = RP * (kChunk / 4);               // 8-byte pieces
    static constexpr int kPerThread = kPieces / (kWaves * kLanes);  // RP / 16
    uint2 v[kPerThread];
};

template <int RP>
__device__ __forceinline__ void load_a(const Args& p, APieces<RP>& a, int64_t k0)
{
#pragma unroll
    for (int i = 0; i < APieces<RP>::kPerThread; ++i) {
        const int q = (int)threadIdx.x + i * kWaves * kLanes;
        const int j = q / (kChunk / 4), c4 = (q % (kChunk / 4)) * 4;
        const int64_t k = k0 + c4;
        a.v[i] = make_uint2(0u, 0u);
        if (j < p.rank && k < p.K) a.v[i] = *reinterpret_cast<const uint2*>(p.a + (int64_t)j * p.K + k);
    }
}

template <int RP>
__device__ __forceinline__ void store_a(const APieces<RP>& a, uint16_t* sA)
{
#pragma unroll
    for (int i = 0; i < APieces<RP>::kPerThread; ++i) {
        const int q = (int)threadIdx.x + i * kWaves * kLanes;
        const int j = q / (kChunk / 4), c4 = (q % (kChunk / 4)) * 4;
        *reinterpret_cast<uint2*>(sA + j * kStride + c4) = a.v[i];
    }
}

template <int RP>
__device__ __forceinline__ void stage_a(const Args& p, uint16_t* sA, int64_t k0)
{
    APieces<RP> a;
    load_a<RP>(p, a, k0);
    store_a<RP>(a, sA);
}

// One 16x16 tile of W' for this wave: columns kt .. kt+15 of rows n0 .. n0+15.
// Returns the lane's 4 values (k = kt + 4*(lane/16) + i, n = n0 + lane%16)
// packed as bf16 pairs.
template <int RP>
__device__ __forceinline__ uint2 merged_tile(const Args& p, const uint16_t* sA, int col, uint2 w4,
                                             const bf16x8_t* bop)
{
    const int lane = threadIdx.x & (kLanes - 1);
    const int nl = lane & 15, g = lane >> 4;
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < RP / 32; ++s) {
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int j = 32 * s + 8 * g + 2 * e;
            const uint32_t lo = sA[j * kStride + col + nl];
            const uint32_t hi = sA[(j + 1) * kStride + col + nl];
            pk[e] = lo | (hi << 16);
        }
        const bf16x8_t aop = __builtin_bit_cast(bf16x8_t, make_uint4(pk[0], pk[1], pk[2], pk[3]));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, bop[s], acc, 0, 0, 0);
    }
    // delta.to(bf16), then the bf16 add: binary32 add of the two bf16 values, rounded.
    const float d0 = round_bf16(acc[0] * p.lora_scale), d1 = round_bf16(acc[1] * p.lora_scale);
    const float d2 = round_bf16(acc[2] * p.lora_scale), d3 = round_bf16(acc[3] * p.lora_scale);
    uint2 out;
    out.x = pack_bf16x2(bf16_lo(w4.x) + d0, bf16_hi(w4.x) + d1);
    out.y = pack_bf16x2(bf16_lo(w4.y) + d2, bf16_hi(w4.y) + d3);
    return out;
}

__device__ __forceinline__ uint32_t codes4(uint2 v, float s, float r)
{
    return pack_e4m3x4(round_bf16(div_by_scale(bf16_lo(v.x), s, r)), round_bf16(div_by_scale(bf16_hi(v.x), s, r)),
                       round_bf16(div_by_scale(bf16_lo(v.y), s, r)), round_bf16(div_by_scale(bf16_hi(v.y), s, r)));
}

__device__ __forceinline__ uint32_t codes4_exact(uint2 v, float s)
{
    return pack_e4m3x4(round_bf16(bf16_lo(v.x) / s), round_bf16(bf16_hi(v.x) / s),
                       round_bf16(bf16_lo(v.y) / s), round_bf16(bf16_hi(v.y) / s));
}

// RP = rank padded to a multiple of 32; NRES = sweep steps whose W' tiles stay
// in VGPRs (0: recompute in a second sweep).
template <int RP, int NRES>
__global__ __launch_bounds__(kWaves * kLanes) void k_lora_requant(Args p)
{
    __shared__ uint16_t sA[2][RP * kStride];
    __shared__ uint32_t sMax[kWaves][kRows];

    const int wave = threadIdx.x / kLanes, lane = threadIdx.x & (kLanes - 1);
    const int nl = lane & 15, g = lane >> 4;
    const int64_t n = (int64_t)blockIdx.x * kRows + nl;
    const bool nvalid = n < p.N;
    const int64_t steps = (p.K + kChunk - 1) / kChunk;

    // B operand: lane holds B[n][32 s + 8 g + e], e < 8 (zero beyond rank).
    bf16x8_t bop[RP / 32];
#pragma unroll
    for (int s = 0; s < RP / 32; ++s) {
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t j = 32 * s + 8 * g + 2 * e;
            uint32_t lo = 0, hi = 0;
            if (nvalid && j < p.rank) lo = p.b[n * p.rank + j];
            if (nvalid && j + 1 < p.rank) hi = p.b[n * p.rank + j + 1];
            pk[e] = lo | (hi << 16);
        }
        bop[s] = __builtin_bit_cast(bf16x8_t, make_uint4(pk[0], pk[1], pk[2], pk[3]));
    }

    // This lane's W values (rows n, columns step*kChunk + wave*16 + 4g .. +3) for
    // every step are loaded up front when they fit in registers, so no step
    // waits on HBM; A goes through two LDS buffers, the next step's global
    // loads in flight while the current step computes.
    const bool merge_only = p.wq == nullptr;
    auto w_at = [&](int64_t step) {
        const int64_t kt = step * kChunk + wave * 16;
        uint2 w4 = make_uint2(0u, 0u);
        if (nvalid && kt < p.K) w4 = *reinterpret_cast<const uint2*>(p.w + n * p.ldw + kt + 4 * g);
        return w4;
    };
    uint2 res[NRES > 0 ? NRES : 1];
    if constexpr (NRES > 0) {
#pragma unroll
        for (int i = 0; i < NRES; ++i)
            if (i < steps) res[i] = w_at(i);
    }
    uint32_t m2 = 0;
    stage_a<RP>(p, sA[0], 0);
    __syncthreads();
    for (int64_t step = 0; step < steps; ++step) {
        APieces<RP> next;
        const bool more = step + 1 < steps;
        if (more) load_a<RP>(p, next, (step + 1) * kChunk);
        const int64_t kt = step * kChunk + wave * 16;
        uint2 w4 = make_uint2(0u, 0u);
        if constexpr (NRES > 0) {
#pragma unroll
            for (int i = 0; i < NRES; ++i)
                if (i == step) w4 = res[i];
        } else {
            w4 = w_at(step);
        }
        uint2 t = make_uint2(0u, 0u);
        if (kt < p.K) t = merged_tile<RP>(p, sA[step & 1], wave * 16, w4, bop);
        if (merge_only) {
            if (kt < p.K && nvalid) *reinterpret_cast<uint2*>(p.w_merged + n * p.ldw + kt + 4 * g) = t;
        } else {
            m2 = absmax_bf16x2(m2, t.x);
            m2 = absmax_bf16x2(m2, t.y);
            if constexpr (NRES > 0) {
#pragma unroll
                for (int i = 0; i < NRES; ++i)
                    if (i == step) res[i] = t;
            }
        }
        if (more) store_a<RP>(next, sA[(step + 1) & 1]);
        __syncthreads();
    }
    if (merge_only) return;

    // Row maxima: the lanes sharing n differ in g (lane bits 4, 5), then waves.
    uint32_t m = max(m2 & 0xffffu, m2 >> 16);
    m = max(m, (uint32_t)__shfl_xor((int)m, 16, 64));
    m = max(m, (uint32_t)__shfl_xor((int)m, 32, 64));
    if (g == 0) sMax[wave][nl] = m;
    __syncthreads();
    m = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) m = max(m, sMax[w][nl]);
    const float scale = row_scale(bf16_to_f32((uint16_t)m));
    if (wave == 0 && g == 0 && nvalid) p.w_scale[n] = scale;
    const float sb = round_bf16(scale);
    const float r = 1.0f / sb;
    const bool finite = __builtin_isfinite(sb);

    for (int64_t step = 0; step < steps; ++step) {
        const int64_t kt = step * kChunk + wave * 16;
        uint2 t = make_uint2(0u, 0u);
        if constexpr (NRES > 0) {
#pragma unroll
            for (int i = 0; i < NRES; ++i)
                if (i == step) t = res[i];
        } else {
            stage_a<RP>(p, sA[0], step * kChunk);
            __syncthreads();
            if (kt < p.K) t = merged_tile<RP>(p, sA[0], wave * 16, w_at(step), bop);
            __syncthreads();
        }
        if (kt < p.K && nvalid) {
            *reinterpret_cast<uint32_t*>(p.wq + n * p.ldq + kt + 4 * g) = finite ? codes4(t, sb, r) : codes4_exact(t, sb);
            if (p.w_merged) *reinterpret_cast<uint2*>(p.w_merged + n * p.ldw + kt + 4 * g) = t;
        }
    }
}

template <int RP>
void launch_rp(const Args& p, dim3 grid, hipStream_t st)
{
    const dim3 block(kWaves * kLanes);
    const int64_t steps = (p.K + kChunk - 1) / kChunk;
    // W' stays in registers for up to kMaxRes steps (what fits in the 128 VGPRs
    // of a 1024-thread workgroup next to the rank-RP operand); wider rows recompute.
    constexpr int kMaxRes = RP >= 96 ? 12 : 20;
    if (steps <= 8) hipLaunchKernelGGL((k_lora_requant<RP, 8>), grid, block, 0, st, p);
    else if (steps <= 12) hipLaunchKernelGGL((k_lora_requant<RP, 12>), grid, block, 0, st, p);
    else if (steps <= 16 && kMaxRes >= 16) hipLaunchKernelGGL((k_lora_requant<RP, (kMaxRes >= 16 ? 16 : 0)>), grid, block, 0, st, p);
    else if (steps <= 20 && kMaxRes >= 20) hipLaunchKernelGGL((k_lora_requant<RP, (kMaxRes >= 20 ? 20 : 0)>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((k_lora_requant<RP, 0>), grid, block, 0, st, p);
}

}  // namespace

int launch_lora_requant(const uint16_t* w, int64_t N, int64_t K, int64_t ldw, const uint16_t* a,
                        const uint16_t* b, int64_t rank, float lora_scale, uint8_t* wq, int64_t ldq,
                        float* w_scale, uint16_t* w_merged, hipStream_t stream)
{
    if (rank < 1 || rank > 128)
        return set_error(VDN_FP8_EINVAL, "requantize_weight: LoRA rank %lld outside 1..128", (long long)rank);
    if (K % 16) return set_error(VDN_FP8_EINVAL, "requantize_weight: the LoRA path needs K %% 16 == 0 (K=%lld)", (long long)K);
    if (((uintptr_t)a % 8) || (K % 4)) return set_error(VDN_FP8_EINVAL, "requantize_weight: lora_a must be 8-byte aligned");
    if (w_merged && ((uintptr_t)w_merged % 8)) return set_error(VDN_FP8_EINVAL, "requantize_weight: w_merged must be 8-byte aligned");
    if (wq && (((uintptr_t)wq % 4) || (ldq % 4))) return set_error(VDN_FP8_EINVAL, "requantize_weight: wq rows must be 4-byte aligned");
    Args p{w, N, K, ldw, a, b, rank, lora_scale, wq, ldq, w_scale, w_merged};
    const dim3 grid((unsigned)((N + kRows - 1) / kRows));
    const int rp = (int)((rank + 31) / 32) * 32;
    switch (rp) {
        case 32: launch_rp<32>(p, grid, stream); break;
        case 64: launch_rp<64>(p, grid, stream); break;
        case 96: launch_rp<96>(p, grid, stream); break;
        default: launch_rp<128>(p, grid, stream); break;
    }
    return check_launch("requantize_weight (LoRA)");
}

}  // namespace vdn
