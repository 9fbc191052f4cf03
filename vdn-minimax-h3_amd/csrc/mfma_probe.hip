// Bare fp8 matrix-core loop for measurement: the rate the MFMA units sustain on
// a given kind of operand data when nothing else runs -- no global -> LDS copy
// stream, no epilogue, no output -- as a ceiling to set the GEMM's rate against.
// Not part of the product's C ABI (libvdnprobe.so, loaded by bench.py only).
//
// The GEMM's grid: one workgroup of four waves per CU (one wave per SIMD), each
// wave a 128 x 128 quadrant. Modes 0-2: 4 x 4 v_mfma_f32_32x32x64_f8f6f4
// accumulators, a block of 128 K bytes consumed as two half-steps of 16 MFMAs
// whose operand fragments are read from LDS (16-byte reads of swizzled 128-byte
// rows) while the previous half-step's MFMAs run. Modes 3-5: the 16 x 16 x 128
// form the GEMM uses (k_mfma_probe16 below). The LDS stage is filled once from the caller's e4m3 codes (a
// 256-row tile of X and one of W, at a per-workgroup offset), so the MFMAs see
// the same operand bits a GEMM over those matrices sees, block after block.
// mode 0: those codes; mode 1: every code e4m3 1.0 (0x38, no multiplier bits
// toggle); mode 2: the codes, fragments read once and then held in registers
// (no LDS reads in the loop: the matrix core alone).
// Modes 3-5: the same three for the 16 x 16 x 128 instruction (the GEMM's).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kRows = 256;                 // rows of the X tile and of the W tile
constexpr int kBK = 128;                   // K bytes per block
constexpr int kStage = 2 * kRows * kBK;    // 64 KiB: X tile, then W tile

__device__ __forceinline__ int lds_off(int row, int chunk) { return row * kBK + ((chunk ^ ((row >> 1) & 7)) << 4); }

template <int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_mfma_probe(const uint8_t* __restrict__ xq, const uint8_t* __restrict__ wq, int64_t ld, int64_t tiles,
                  int blocks, float* __restrict__ out)
{
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kStage];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wm = wave >> 1;

    // fill: thread t moves 16-byte chunks (row, chunk) = ((t + 256 i) / 8, (t + 256 i) % 8)
    const int64_t tile = blockIdx.x % tiles;
    for (int i = 0; i < kStage / 16 / kThreads; ++i) {
        const int q = tid + kThreads * i;
        const int row = (q >> 3) & (kRows - 1), chunk = q & 7;
        const bool is_w = q >= kRows * 8;
        uint4 v;
        if (MODE == 1) {
            v = make_uint4(0x38383838u, 0x38383838u, 0x38383838u, 0x38383838u);
        } else {
            const uint8_t* src = (is_w ? wq : xq) + (tile * kRows + row) * ld + chunk * 16;
            v = *reinterpret_cast<const uint4*>(src);
        }
        *reinterpret_cast<uint4*>(smem + (is_w ? kRows * kBK : 0) + lds_off(row, chunk)) = v;
    }
    __syncthreads();

    const int frow = lane & 31, fh = lane >> 5;
    auto read_frag = [&](int h, int f) -> i32x8_t {
        const uint8_t* s = smem + (f < 4 ? kRows * kBK : 0);
        const int row = (f < 4 ? wn * 128 + 32 * f : wm * 128 + 32 * (f - 4)) + frow;
        const uint4 lo = *reinterpret_cast<const uint4*>(s + lds_off(row, 4 * h + 2 * fh));
        const uint4 hi = *reinterpret_cast<const uint4*>(s + lds_off(row, 4 * h + 2 * fh + 1));
        return i32x8_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    };
    i32x8_t w0[4], x0[4], w1[4], x1[4];
    auto read_into = [&](int h, int f, i32x8_t* wf, i32x8_t* xf) {
        if (f < 4) wf[f] = read_frag(h, f);
        else xf[f - 4] = read_frag(h, f);
    };
    f32x16_t acc[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[t][u] = f32x16_t{};
    auto mfma = [&](const i32x8_t* wf, const i32x8_t* xf, int q) {
        const int t = q & 3, u = q >> 2;
        acc[t][u] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[t], xf[u], acc[t][u], 0, 0, 0, 0, 0, 0);
    };
#pragma unroll
    for (int f = 0; f < 8; ++f) read_into(0, f, w0, x0);
    if (MODE == 2) {
#pragma unroll
        for (int f = 0; f < 8; ++f) read_into(1, f, w1, x1);
    }
    for (int j = 0; j < blocks; ++j) {
        // half 0: its MFMAs, reading half 1's fragments during the first four
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            mfma(w0, x0, q);
            __builtin_amdgcn_sched_barrier(0);
            if (MODE != 2 && q < 4) {
                read_into(1, 2 * q, w1, x1);
                read_into(1, 2 * q + 1, w1, x1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // half 1: its MFMAs, reading the next block's half-0 fragments during MFMAs 8-15
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            mfma(w1, x1, q);
            __builtin_amdgcn_sched_barrier(0);
            if (MODE != 2 && q >= 8) read_into(0, q - 8, w0, x0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // every accumulator feeds the output, so no MFMA is dead
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r) s += acc[t][u][r];
    out[(int64_t)blockIdx.x * kThreads + tid] = s;
}

// The same measurement for v_mfma_f32_16x16x128_f8f6f4, the GEMM's instruction: per
// 128-byte block 8 groups of 8 MFMAs, group j multiplying X fragment j (16 rows x 128
// bytes, read from LDS before the group) by the wave's 8 W fragments (read after the
// block's last group), the rows in the GEMM's LDS layout for this instruction (chunk c of
// row r at c ^ s16(r)). mode 3: the caller's codes; 4: every code 1.0; 5: fragments read
// once and then held in registers.
__device__ __forceinline__ int lds_off16(int row, int chunk)
{
    const int s = ((row >> 1) & 1) | ((row & 1) << 1) | (row & 4);
    return row * kBK + ((chunk ^ s) << 4);
}

template <int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_mfma_probe16(const uint8_t* __restrict__ xq, const uint8_t* __restrict__ wq, int64_t ld, int64_t tiles,
                    int blocks, float* __restrict__ out)
{
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kStage];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wm = wave >> 1;
    const int64_t tile = blockIdx.x % tiles;
    for (int i = 0; i < kStage / 16 / kThreads; ++i) {
        const int q = tid + kThreads * i;
        const int row = (q >> 3) & (kRows - 1), chunk = q & 7;
        const bool is_w = q >= kRows * 8;
        uint4 v;
        if (MODE == 4) {
            v = make_uint4(0x38383838u, 0x38383838u, 0x38383838u, 0x38383838u);
        } else {
            const uint8_t* src = (is_w ? wq : xq) + (tile * kRows + row) * ld + chunk * 16;
            v = *reinterpret_cast<const uint4*>(src);
        }
        *reinterpret_cast<uint4*>(smem + (is_w ? kRows * kBK : 0) + lds_off16(row, chunk)) = v;
    }
    __syncthreads();
    const int fr = lane & 15, fg = lane >> 4;
    auto read_frag = [&](bool w, int f) -> i32x8_t {
        const uint8_t* s = smem + (w ? kRows * kBK : 0);
        const int row = (w ? wn * 128 : wm * 128) + 16 * f + fr;
        const uint4 lo = *reinterpret_cast<const uint4*>(s + lds_off16(row, 2 * fg));
        const uint4 hi = *reinterpret_cast<const uint4*>(s + lds_off16(row, 2 * fg + 1));
        return i32x8_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    };
    typedef float f32x4_t __attribute__((ext_vector_type(4)));
    f32x4_t acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{};
    i32x8_t wf[8], xr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) wf[i] = read_frag(true, i);
    if (MODE == 5) {
#pragma unroll
        for (int j = 0; j < 8; ++j) xr[j] = read_frag(false, j);
    }
    for (int b = 0; b < blocks; ++b) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const i32x8_t xf = MODE == 5 ? xr[j] : read_frag(false, j);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[i], xf, acc[i][j], 0, 0, 0, 0, 0, 0);
            if (MODE != 5 && j == 7) {
#pragma unroll
                for (int i = 0; i < 8; ++i) wf[i] = read_frag(true, i);
            }
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) s += acc[i][j][r];
    out[(int64_t)blockIdx.x * kThreads + tid] = s;
}

}  // namespace

// Runs `grid` workgroups (one per CU for the GEMM's shape), each wave issuing
// blocks x 32 MFMAs of 32 x 32 x 64 (modes 0-2) or blocks x 64 of 16 x 16 x 128 (modes
// 3-5): the same FLOP. xq and wq: e4m3 codes with row stride ld,
// at least tiles x 256 rows each (workgroup b uses tile b % tiles of both, the
// first 128 bytes of each row); out: grid x 256 floats. Modes as above.
// Returns 0, 22 for a bad argument, or the launch's HIP error.
extern "C" int vdn_mfma_probe(int mode, const void* xq, const void* wq, int64_t ld, int64_t tiles, int blocks,
                              int grid, float* out, hipStream_t stream)
{
    if (!out || grid <= 0 || blocks <= 0 || tiles <= 0 || (mode != 1 && mode != 4 && (!xq || !wq || ld < kBK || ld % 16)))
        return 22;
    const dim3 g((unsigned)grid), b(kThreads);
    const uint8_t* x = static_cast<const uint8_t*>(xq);
    const uint8_t* w = static_cast<const uint8_t*>(wq);
    if (mode == 0) hipLaunchKernelGGL(k_mfma_probe<0>, g, b, 0, stream, x, w, ld, tiles, blocks, out);
    else if (mode == 1) hipLaunchKernelGGL(k_mfma_probe<1>, g, b, 0, stream, x, w, ld, tiles, blocks, out);
    else if (mode == 2) hipLaunchKernelGGL(k_mfma_probe<2>, g, b, 0, stream, x, w, ld, tiles, blocks, out);
    else if (mode == 3) hipLaunchKernelGGL(k_mfma_probe16<3>, g, b, 0, stream, x, w, ld, tiles, blocks, out);
    else if (mode == 4) hipLaunchKernelGGL(k_mfma_probe16<4>, g, b, 0, stream, x, w, ld, tiles, blocks, out);
    else if (mode == 5) hipLaunchKernelGGL(k_mfma_probe16<5>, g, b, 0, stream, x, w, ld, tiles, blocks, out);
    else return 22;
    return (int)hipGetLastError();
}
