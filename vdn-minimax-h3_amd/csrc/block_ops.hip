// The DiT block's gated residual add as one pass (the compiled `post` of the
// reference, src/models/ops/fused_block.py:47-49,101-110):
//
//   out[m][n] = bf16(residual[m][n] + gate[i][n] * branch[m][n]),   i = gate_index[m]
//
// in binary32 with one rounding (the product of two bf16 values is exact in
// binary32, so the only roundings are the sum's and the store's). The same
// arithmetic as the GEMM's gate epilogue, for a branch whose last op is not one
// of this library's GEMMs (the attention sub-layer).
//
// Layout: one workgroup per 2048-element piece of a row (256 threads x 8
// elements, 16-byte loads and stores); the grid is rows x pieces.
#include <stdint.h>

#include "vdn_common.h"

namespace vdn {
namespace {

constexpr int kThreads = 256;
constexpr int kPiece = kThreads * 8;

__global__ __launch_bounds__(kThreads) void k_gated_residual(
    const uint16_t* __restrict__ residual, int64_t ldr, const uint16_t* __restrict__ gate, int64_t ldgate,
    const int32_t* __restrict__ gate_index, int64_t gate_rows, const uint16_t* __restrict__ branch, int64_t ldb,
    uint16_t* out, int64_t ldo, int64_t N)
{
    const int64_t m = blockIdx.x;
    const int64_t n = (int64_t)blockIdx.y * kPiece + 8 * threadIdx.x;
    if (n >= N) return;
    int64_t gi = 0;
    if (gate_index) gi = min(max((int64_t)gate_index[m], (int64_t)0), gate_rows - 1);
    const uint4 r = *reinterpret_cast<const uint4*>(residual + m * ldr + n);
    const uint4 g = *reinterpret_cast<const uint4*>(gate + gi * ldgate + n);
    const uint4 b = *reinterpret_cast<const uint4*>(branch + m * ldb + n);
    const uint32_t rw[4] = {r.x, r.y, r.z, r.w}, gw[4] = {g.x, g.y, g.z, g.w}, bw[4] = {b.x, b.y, b.z, b.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float lo = bf16_lo(rw[e]) + bf16_lo(gw[e]) * bf16_lo(bw[e]);
        const float hi = bf16_hi(rw[e]) + bf16_hi(gw[e]) * bf16_hi(bw[e]);
        o[e] = pack_bf16x2(lo, hi);
    }
    *reinterpret_cast<uint4*>(out + m * ldo + n) = make_uint4(o[0], o[1], o[2], o[3]);
}

bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

}  // namespace
}  // namespace vdn

using namespace vdn;

extern "C" int vdn_fp8_gated_residual(const void* residual, int64_t ldr, const void* gate, int64_t ldgate,
                                      const int32_t* gate_index, int64_t gate_rows, const void* branch,
                                      int64_t ldb, void* out, int64_t ldo, int64_t M, int64_t N,
                                      hipStream_t stream)
{
    if (M < 0 || N < 0) return set_error(VDN_FP8_EINVAL, "gated_residual: negative shape");
    if (M == 0 || N == 0) return VDN_FP8_OK;
    if (!residual || !gate || !branch || !out) return set_error(VDN_FP8_EINVAL, "gated_residual: null pointer");
    if (N % 8 || ldr % 8 || ldgate % 8 || ldb % 8 || ldo % 8 || ldr < N || ldb < N || ldo < N ||
        (gate_rows > 1 && ldgate < N) || gate_rows < 1)
        return set_error(VDN_FP8_EINVAL, "gated_residual: need N and the row strides multiples of 8 and >= N, "
                                         "and a gate table of >= 1 row");
    if (!aligned16(residual) || !aligned16(gate) || !aligned16(branch) || !aligned16(out) ||
        (gate_index && ((uintptr_t)gate_index % 4)))
        return set_error(VDN_FP8_EINVAL, "gated_residual: misaligned pointer (residual, gate, branch, out 16 B)");
    if (M > 0x7fffffffLL) return set_error(VDN_FP8_EINVAL, "gated_residual: too many rows");
    const int64_t pieces = (N + kPiece - 1) / kPiece;
    if (pieces > 65535) return set_error(VDN_FP8_EINVAL, "gated_residual: rows too long");
    const dim3 grid((unsigned)M, (unsigned)pieces), block(kThreads);
    hipLaunchKernelGGL(k_gated_residual, grid, block, 0, stream, (const uint16_t*)residual, ldr,
                       (const uint16_t*)gate, ldgate, gate_index, gate_rows, (const uint16_t*)branch, ldb,
                       (uint16_t*)out, ldo, N);
    return check_launch("gated_residual");
}
