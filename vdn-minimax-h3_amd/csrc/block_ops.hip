// The DiT block's gated residual add as one pass (the compiled `post` of the
// reference, src/models/ops/fused_block.py:47-49,101-110):
//
//   out[m][n] = bf16(residual[m][n] + gate[i][n] * branch[m][n]),   i = gate_index[m]
//   out[m][n] = bf16(gate[i][n] * branch[m][n])                       (no residual)
//
// in binary32 with one rounding (the product of two bf16 values is exact in
// binary32, so the only roundings are the sum's and the store's). The same
// arithmetic as the GEMM's gate epilogue, for a branch whose last op is not one
// of this library's GEMMs (the attention sub-layer).
//
// Layout: one wave per row (four rows per workgroup); lane L takes the row's
// 16-byte chunks L, L + 64, ..., four at a time with all their loads issued
// before any is used.
#include <stdint.h>

#include "vdn_common.h"

namespace vdn {
namespace {

constexpr int kLanes = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kBatch = 4;            // chunks per lane in flight
// Outputs of at least this many bytes are stored non-temporally: beyond what the
// 256 MB last-level cache holds, cached stores only evict each other ([32760, 5120]:
// 0.180 ms against 0.193 ms).
constexpr int64_t kNtStoreBytes = 256ll << 20;
typedef int i32x4_t __attribute__((ext_vector_type(4)));
constexpr int kStoreOnce = 2;        // cache policy of a non-temporal buffer store

template <bool RES, bool NT>
__global__ __launch_bounds__(kWavesPerBlock * kLanes) void k_gated_residual(
    const uint16_t* residual, int64_t ldr, const uint16_t* __restrict__ gate, int64_t ldgate,
    const int32_t* __restrict__ gate_index, int64_t gate_rows, const uint16_t* branch, int64_t ldb,
    uint16_t* out, int64_t ldo, int64_t M, int64_t N)   // out may alias residual or branch
{
    const int lane = threadIdx.x & (kLanes - 1);
    // One wave per (row, span of kBatch * 64 chunks): every wave issues all its loads
    // at once and makes one round trip. The unit as a uniform value: the row's gate
    // index is read by a scalar load.
    const int nch = (int)(N >> 3);
    const int64_t spans = (nch + kBatch * kLanes - 1) / (kBatch * kLanes);
    const int64_t unit = (int64_t)blockIdx.x * kWavesPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x / kLanes);
    const int64_t m = unit / spans;
    if (m >= M) return;
    // Buffer loads and stores over the row (16-byte chunks past N fall outside the
    // descriptors: zeros read, stores dropped), so nothing sits under a branch and
    // the stores go out back to back.
    const int rowbytes = nch * 16;
    const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(RES ? residual + m * ldr : branch), 0, RES ? rowbytes : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc((void*)(branch + m * ldb), 0, rowbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc((void*)(out + m * ldo), 0, rowbytes, 0x00020000);
    const uint32_t c0 = (uint32_t)(unit - m * spans) * kBatch * kLanes + lane;
    uint4 r[kBatch], g[kBatch], b[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
        const uint32_t off = (c0 + j * kLanes) * 16u;
        r[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rrs, off, 0, kBufferLoadOnce));
        b[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(brs, off, 0, kBufferLoadOnce));
    }
    // the gate row's index is read after the row's own loads are issued (the gate
    // addresses wait for it; the residual and branch loads need not)
    __builtin_amdgcn_sched_barrier(0);
    int64_t gi = 0;
    if (gate_index) gi = min(max((int64_t)gate_index[m], (int64_t)0), gate_rows - 1);
    const __amdgpu_buffer_rsrc_t grs = __builtin_amdgcn_make_buffer_rsrc((void*)(gate + gi * ldgate), 0, rowbytes, 0x00020000);
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
        g[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(grs, (c0 + j * kLanes) * 16u, 0, 0));
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
        const uint32_t rw[4] = {r[j].x, r[j].y, r[j].z, r[j].w}, gw[4] = {g[j].x, g[j].y, g[j].z, g[j].w},
                       bw[4] = {b[j].x, b[j].y, b[j].z, b[j].w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // without a residual the product is stored as it is (no + 0: that would turn -0 into +0)
            float lo = bf16_lo(gw[e]) * bf16_lo(bw[e]);
            float hi = bf16_hi(gw[e]) * bf16_hi(bw[e]);
            if (RES) { lo = bf16_lo(rw[e]) + lo; hi = bf16_hi(rw[e]) + hi; }
            o[e] = pack_bf16x2(lo, hi);
        }
        store_b128_settled<NT ? kStoreOnce : 0>(i32x4_t{(int)o[0], (int)o[1], (int)o[2], (int)o[3]}, ors,
                                                (c0 + j * kLanes) * 16u, 0);
    }
}

}  // namespace

// Launch without argument checks (the callers have made them): also the second
// pass of the GEMM's per-row gate / residual epilogue, in place on its output.
int launch_gated_residual(const uint16_t* residual, int64_t ldr, const uint16_t* gate, int64_t ldgate,
                          const int32_t* gate_index, int64_t gate_rows, const uint16_t* branch, int64_t ldb,
                          uint16_t* out, int64_t ldo, int64_t M, int64_t N, hipStream_t stream)
{
    const int64_t spans = (N / 8 + kBatch * kLanes - 1) / (kBatch * kLanes);   // waves per row
    const dim3 grid((unsigned)((M * spans + kWavesPerBlock - 1) / kWavesPerBlock)), block(kWavesPerBlock * kLanes);
    const bool nt = M * N * 2 >= kNtStoreBytes;
#define VDN_GR(R, T)                                                                                         \
    hipLaunchKernelGGL((k_gated_residual<R, T>), grid, block, 0, stream, residual, ldr, gate, ldgate, gate_index, \
                       gate_rows, branch, ldb, out, ldo, M, N)
    if (residual) {
        if (nt) VDN_GR(true, true); else VDN_GR(true, false);
    } else {
        if (nt) VDN_GR(false, true); else VDN_GR(false, false);
    }
#undef VDN_GR
    return check_launch("gated_residual");
}

}  // namespace vdn

using namespace vdn;

extern "C" int vdn_fp8_gated_residual(const void* residual, int64_t ldr, const void* gate, int64_t ldgate,
                                      const int32_t* gate_index, int64_t gate_rows, const void* branch,
                                      int64_t ldb, void* out, int64_t ldo, int64_t M, int64_t N,
                                      hipStream_t stream)
{
    if (M < 0 || N < 0) return set_error(VDN_FP8_EINVAL, "gated_residual: negative shape");
    if (M == 0 || N == 0) return VDN_FP8_OK;
    if (!gate || !branch || !out) return set_error(VDN_FP8_EINVAL, "gated_residual: null pointer");
    if (N % 8 || (residual && (ldr % 8 || ldr < N)) || ldgate % 8 || ldb % 8 || ldo % 8 || ldb < N || ldo < N ||
        (gate_rows > 1 && ldgate < N) || gate_rows < 1)
        return set_error(VDN_FP8_EINVAL, "gated_residual: need N and the row strides multiples of 8 and >= N, "
                                         "and a gate table of >= 1 row");
    if ((residual && !aligned(residual, 16)) || !aligned(gate, 16) || !aligned(branch, 16) || !aligned(out, 16) ||
        (gate_index && ((uintptr_t)gate_index % 4)))
        return set_error(VDN_FP8_EINVAL, "gated_residual: misaligned pointer (residual, gate, branch, out 16 B)");
    if (M * (N / 8 / (kBatch * kLanes) + 1) / kWavesPerBlock >= 0x7fffffffLL || N >= 0x40000000LL)
        return set_error(VDN_FP8_EINVAL, "gated_residual: problem too large");
    return launch_gated_residual((const uint16_t*)residual, ldr, (const uint16_t*)gate, ldgate, gate_index, gate_rows,
                                 (const uint16_t*)branch, ldb, (uint16_t*)out, ldo, M, N, stream);
}
