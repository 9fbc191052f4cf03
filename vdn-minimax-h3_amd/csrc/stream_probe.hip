// Bare read + write stream for measurement: the rate the memory system gives a
// kernel that only moves bytes, as a ceiling to set the row kernels' rates
// against. Not part of the product's C ABI (libvdnprobe.so, loaded by bench.py
// only).
//
// Each wave takes units of KR 1 KiB read pieces and KW 1 KiB write pieces
// (consecutive units to consecutive waves, then strided by the grid), with
// 16-byte non-temporal buffer loads and 16-byte buffer stores, non-temporal or
// cached, the row kernels' access forms. The stored values depend on the loaded
// ones, so no load is dead.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int i32x4_t __attribute__((ext_vector_type(4)));
constexpr int kLanes = 64;
constexpr int kWaves = 4;   // waves per workgroup
constexpr int kLoadNT = 2;  // cache policy: non-temporal

template <int KR, int KW, bool NT_STORE>
__global__ __launch_bounds__(kWaves * kLanes) void k_stream(const uint8_t* __restrict__ src, int64_t units,
                                                            uint8_t* __restrict__ dst)
{
    const int lane = threadIdx.x & (kLanes - 1);
    const int64_t first = (int64_t)blockIdx.x * kWaves + threadIdx.x / kLanes;
    const int64_t step = (int64_t)gridDim.x * kWaves;
    for (int64_t u = first; u < units; u += step) {
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc((void*)(src + u * KR * 1024), 0, KR * 1024, 0x00020000);
        const __amdgpu_buffer_rsrc_t ws =
            __builtin_amdgcn_make_buffer_rsrc((void*)(dst + u * KW * 1024), 0, KW * 1024, 0x00020000);
        i32x4_t v[KR];
#pragma unroll
        for (int c = 0; c < KR; ++c)
            v[c] = __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)((c * kLanes + lane) * 16), 0, kLoadNT);
        i32x4_t x = v[0];
#pragma unroll
        for (int c = 1; c < KR; ++c) x ^= v[c];
#pragma unroll
        for (int c = 0; c < KW; ++c)
            __builtin_amdgcn_raw_buffer_store_b128(x + c, ws, (uint32_t)((c * kLanes + lane) * 16), 0,
                                                   NT_STORE ? kLoadNT : 0);
    }
}

}  // namespace

// Reads units * kr KiB from src and writes units * kw KiB to dst with `grid`
// workgroups of four waves. (kr, kw) in {(1, 1), (2, 1), (4, 1)}; nt_store selects
// non-temporal stores. Returns 0, EINVAL for another shape or a bad argument, or the
// launch's HIP error.
extern "C" int vdn_stream_probe(int kr, int kw, int nt_store, const void* src, int64_t units, void* dst, int grid,
                                hipStream_t stream)
{
    if (!src || !dst || units <= 0 || grid <= 0) return 22;
    const dim3 g((unsigned)grid), b(kWaves * kLanes);
    const uint8_t* s = static_cast<const uint8_t*>(src);
    uint8_t* d = static_cast<uint8_t*>(dst);
#define VDN_PROBE(R, W)                                                                                \
    if (kr == R && kw == W) {                                                                          \
        if (nt_store) hipLaunchKernelGGL((k_stream<R, W, true>), g, b, 0, stream, s, units, d);        \
        else hipLaunchKernelGGL((k_stream<R, W, false>), g, b, 0, stream, s, units, d);                \
        return (int)hipGetLastError();                                                                 \
    }
    VDN_PROBE(1, 1)
    VDN_PROBE(2, 1)
    VDN_PROBE(4, 1)
#undef VDN_PROBE
    return 22;
}
