// Fused LoRA merge + rowwise weight requantization (gfx950).
//
//   W'[n][k]   = bf16(W[n][k] + bf16(lora_scale * sum_j B[n][j] A[j][k]))
//   w_scale[n] = max(max_k |W'[n][k]| / 448, 1e-12)
//   wq[n][k]   = e4m3(bf16(W'[n][k] / bf16(w_scale[n])))
//
// The reference merges in place on the bf16 weight (lora.py:91-92) and then
// quantizes it in eager torch (fp8_linear.py:262-267): several full passes over
// W plus the write-back of W'. Here W' is never stored unless asked for. The
// weight is cut into 64-row x 256-column tiles, each a workgroup of four
// waves (16 rows each), so the work is spread over thousands of independent
// workgroups:
//   pass 1 (k_lora_tiles<.., kRowMax>)   W' of the tile in registers, its row
//                                        maxima merged into w_scale (used as a
//                                        uint32 max, zeroed first);
//   pass 2 (k_lora_tiles<.., kQuantize>) W' recomputed (W re-read, mostly from
//                                        the last-level cache), the codes written;
//   k_rowmax_to_scale                    w_scale[n] = the reference's scale.
// Merge-only calls (no codes) run pass 2's body with the W' store alone.
//
// The rank-r update uses v_mfma_f32_16x16x32_bf16: MFMA row index = k (16
// columns of W), column index = n (16 rows of W), reduction = rank. Products of
// bf16 are exact in fp32 and the accumulation is fp32, as the reference's fp32
// matmul. The MFMA's k-side operand is A transposed, so each workgroup stages
// A[:, k0 : k0 + 256] in LDS as rows of k (the rank contiguous, rows padded to
// rank + 8 elements: the 16-row reads and the staging writes are both
// conflict-free at rank 64). Each lane ends with 4 consecutive k of one row n,
// so W and W' move 8 bytes per lane and the codes 4 bytes per lane.
#include <stdint.h>

#include "vdn_common.h"

namespace vdn {
namespace {

constexpr int kRowsPerWave = 16;
constexpr int kWaves = 4;
constexpr int kLanes = 64;
constexpr int kTileRows = kRowsPerWave * kWaves;   // 64
constexpr int kTileCols = 256;                      // 16 MFMA tiles of 16 columns
constexpr int kSub = kTileCols / 16;

enum Mode { kRowMax = 0, kQuantize = 1, kMergeOnly = 2 };

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
};

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

// RP = rank padded to a multiple of 32.
template <int RP, int MODE>
__global__ __launch_bounds__(kWaves * kLanes) void k_lora_tiles(Args p)
{
    constexpr int kS = RP + 8;                       // LDS row (one k) in elements
    __shared__ __attribute__((aligned(16))) uint16_t sAT[kTileCols * kS];

    const int tid = threadIdx.x, lane = tid & (kLanes - 1);
    const int wave = tid / kLanes;
    const int nl = lane & 15, g = lane >> 4;
    const int64_t k0 = (int64_t)blockIdx.x * kTileCols;
    const int64_t n = (int64_t)blockIdx.y * kTileRows + wave * kRowsPerWave + nl;
    const bool nvalid = n < p.N;

    // All loads go through buffer descriptors: rows past N and rank rows past
    // the LoRA rank read as zeros with no branch, so the loads stay in flight
    // together (a load under a divergent branch makes the compiler wait for it).
    // Columns past K may read the next row's data; they only feed outputs that
    // are never stored.
    const int64_t n0 = (int64_t)blockIdx.y * kTileRows;
    const int64_t rows = min(p.N - n0, (int64_t)kTileRows);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.w + n0 * p.ldw), 0, (int)(rows * p.ldw * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.b + n0 * p.rank), 0, (int)(rows * p.rank * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
        (void*)p.a, 0, (int)(p.rank * p.K * 2), 0x00020000);
    const int nr = wave * kRowsPerWave + nl;            // row within the tile

    // This lane's W values: row n, columns k0 + 16 t + 4 g .. +3 (K % 16 == 0,
    // so a 16-column tile is wholly inside or outside the matrix).
    uint2 w4[kSub];
#pragma unroll
    for (int t = 0; t < kSub; ++t) {
        const uint32_t off = (uint32_t)((nr * p.ldw + k0 + 16 * t + 4 * g) * 2);
        w4[t] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wr, off, 0, 0));
    }
    // B operand: lane holds B[n][32 s + 8 g .. +7], zero beyond the rank.
    bf16x8_t bop[RP / 32];
#pragma unroll
    for (int s = 0; s < RP / 32; ++s) {
        const int j0 = 32 * s + 8 * g;
        uint32_t e[4];
        if (p.b_vec) {
            const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                br, (uint32_t)((nr * p.rank + j0) * 2), 0, 0));
            e[0] = v.x; e[1] = v.y; e[2] = v.z; e[3] = v.w;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(br, (uint32_t)((nr * p.rank + j0 + 2 * i) * 2), 0, 0);
                const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(br, (uint32_t)((nr * p.rank + j0 + 2 * i + 1) * 2), 0, 0);
                e[i] = (lo & 0xffffu) | (hi << 16);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = j0 + 2 * i;
            if (j >= p.rank) e[i] = 0u;
            else if (j + 1 >= p.rank) e[i] &= 0xffffu;
        }
        bop[s] = __builtin_bit_cast(bf16x8_t, make_uint4(e[0], e[1], e[2], e[3]));
    }
    // Stage A^T: unit u covers rows j = 2p, 2p+1 and columns 8 kg .. 8 kg + 7;
    // the pair is written as one dword per column at sAT[k][j]. Rows past the
    // rank read as zeros.
    constexpr int kPairs = RP / 2, kUnits = kPairs * (kTileCols / 8);
    uint4 alo[kUnits / (kWaves * kLanes)], ahi[kUnits / (kWaves * kLanes)];
#pragma unroll
    for (int i = 0; i < kUnits / (kWaves * kLanes); ++i) {
        const int u = tid + i * kWaves * kLanes;
        const int pr = u % kPairs, kg = u / kPairs;
        const int64_t j = 2 * pr, k = k0 + 8 * kg;
        alo[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ar, (uint32_t)((j * p.K + k) * 2), 0, 0));
        ahi[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ar, (uint32_t)(((j + 1) * p.K + k) * 2), 0, 0));
    }
#pragma unroll
    for (int i = 0; i < kUnits / (kWaves * kLanes); ++i) {
        const int u = tid + i * kWaves * kLanes;
        const int pr = u % kPairs, kg = u / kPairs;
        const uint32_t l[4] = {alo[i].x, alo[i].y, alo[i].z, alo[i].w}, h[4] = {ahi[i].x, ahi[i].y, ahi[i].z, ahi[i].w};
        uint32_t* dst = reinterpret_cast<uint32_t*>(sAT + (8 * kg) * kS + 2 * pr);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            dst[(2 * e) * (kS / 2)] = (l[e] & 0xffffu) | (h[e] << 16);
            dst[(2 * e + 1) * (kS / 2)] = (l[e] >> 16) | (h[e] & 0xffff0000u);
        }
    }
    __syncthreads();

    float sb = 0.0f, r = 0.0f;
    bool finite = true;
    if (MODE == kQuantize && nvalid) {
        const uint32_t mbits = reinterpret_cast<const uint32_t*>(p.w_scale)[n];
        sb = round_bf16(row_scale(bf16_to_f32((uint16_t)mbits)));
        r = 1.0f / sb;
        finite = __builtin_isfinite(sb);
    }
    uint32_t m2 = 0;
#pragma unroll
    for (int t = 0; t < kSub; ++t) {
        const int64_t k = k0 + 16 * t + 4 * g;
        f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
        const uint16_t* arow = sAT + (16 * t + nl) * kS + 8 * g;
#pragma unroll
        for (int s = 0; s < RP / 32; ++s) {
            const bf16x8_t aop = *reinterpret_cast<const bf16x8_t*>(arow + 32 * s);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, bop[s], acc, 0, 0, 0);
        }
        // delta.to(bf16), then the bf16 add: binary32 add of the two bf16 values, rounded.
        const float d0 = round_bf16(acc[0] * p.lora_scale), d1 = round_bf16(acc[1] * p.lora_scale);
        const float d2 = round_bf16(acc[2] * p.lora_scale), d3 = round_bf16(acc[3] * p.lora_scale);
        uint2 wm;
        wm.x = pack_bf16x2(bf16_lo(w4[t].x) + d0, bf16_hi(w4[t].x) + d1);
        wm.y = pack_bf16x2(bf16_lo(w4[t].y) + d2, bf16_hi(w4[t].y) + d3);
        const bool in = nvalid && k < p.K;
        if (MODE == kRowMax) {
            if (in) {
                m2 = absmax_bf16x2(m2, wm.x);
                m2 = absmax_bf16x2(m2, wm.y);
            }
        } else {
            if (in && p.w_merged) *reinterpret_cast<uint2*>(p.w_merged + n * p.ldw + k) = wm;
            if (MODE == kQuantize && in)
                *reinterpret_cast<uint32_t*>(p.wq + n * p.ldq + k) = finite ? codes4(wm, sb, r) : codes4_exact(wm, sb);
        }
    }
    if (MODE == kRowMax) {
        // the lanes sharing n differ in g (lane bits 4, 5)
        uint32_t m = max(m2 & 0xffffu, m2 >> 16);
        m = max(m, (uint32_t)__shfl_xor((int)m, 16, 64));
        m = max(m, (uint32_t)__shfl_xor((int)m, 32, 64));
        if (g == 0 && nvalid) atomicMax(reinterpret_cast<uint32_t*>(p.w_scale) + n, m);
    }
}

__global__ void k_zero_u32(uint32_t* x, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = 0u;
}

// The row maxima (bf16 magnitude bits) -> the reference's fp32 scale, in place.
__global__ void k_rowmax_to_scale(float* w_scale, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const uint32_t m = reinterpret_cast<const uint32_t*>(w_scale)[i];
        w_scale[i] = row_scale(bf16_to_f32((uint16_t)m));
    }
}

template <int RP>
void launch_rp(const Args& p, bool merge_only, hipStream_t st)
{
    const dim3 grid((unsigned)((p.K + kTileCols - 1) / kTileCols), (unsigned)((p.N + kTileRows - 1) / kTileRows));
    const dim3 block(kWaves * kLanes);
    if (merge_only) {
        hipLaunchKernelGGL((k_lora_tiles<RP, kMergeOnly>), grid, block, 0, st, p);
        return;
    }
    const dim3 vgrid((unsigned)((p.N + 255) / 256)), vblock(256);
    hipLaunchKernelGGL(k_zero_u32, vgrid, vblock, 0, st, reinterpret_cast<uint32_t*>(p.w_scale), p.N);
    hipLaunchKernelGGL((k_lora_tiles<RP, kRowMax>), grid, block, 0, st, p);
    hipLaunchKernelGGL((k_lora_tiles<RP, kQuantize>), grid, block, 0, st, p);
    hipLaunchKernelGGL(k_rowmax_to_scale, vgrid, vblock, 0, st, p.w_scale, p.N);
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
    if (wq && (((uintptr_t)wq % 4) || (ldq % 4))) return set_error(VDN_FP8_EINVAL, "requantize_weight: wq rows must be 4-byte aligned");
    if (w_scale && ((uintptr_t)w_scale % 4)) return set_error(VDN_FP8_EINVAL, "requantize_weight: w_scale must be 4-byte aligned");
    if ((int64_t)kTileRows * ldw * 2 > 0x7fffffffLL || (rank + 33) * K * 2 > 0x7fffffffLL)
        return set_error(VDN_FP8_EINVAL, "requantize_weight: rows too long for the LoRA path");
    if ((N + kTileRows - 1) / kTileRows > 65535)
        return set_error(VDN_FP8_EINVAL, "requantize_weight: N=%lld above the LoRA path's 4194240 rows", (long long)N);
    const bool merge_only = wq == nullptr;
    const int b_vec = (rank % 8 == 0) && ((uintptr_t)b % 16 == 0);
    Args p{w, N, K, ldw, a, b, rank, b_vec, lora_scale, wq, ldq, w_scale, w_merged};
    const int rp = (int)((rank + 31) / 32) * 32;
    switch (rp) {
        case 32: launch_rp<32>(p, merge_only, stream); break;
        case 64: launch_rp<64>(p, merge_only, stream); break;
        case 96: launch_rp<96>(p, merge_only, stream); break;
        default: launch_rp<128>(p, merge_only, stream); break;
    }
    return check_launch("requantize_weight (LoRA)");
}

}  // namespace vdn
