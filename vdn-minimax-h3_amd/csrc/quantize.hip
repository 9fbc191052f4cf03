// Row quantizers for the fp8 linear path (gfx950):
//   - per-token activation quantization      (vdn_fp8_quantize_rows)
//   - fused SwiGLU + per-token quantization  (vdn_fp8_swiglu_quantize_rows)
//   - fused RMSNorm + AdaLN affine + per-token quantization (vdn_fp8_norm_quantize_rows)
//   - rowwise weight quantization, no LoRA   (vdn_fp8_requantize_weight)
//
// All three are HBM-bound: 2 bytes in and 1 byte out per element plus 4 bytes
// of scale per row. One wavefront owns one row and keeps the whole row in
// VGPRs between the absmax sweep and the scaled cast, so every input byte is
// read from HBM exactly once (the reference's Triton kernel reads each row
// twice, fp8_linear.py:21-23,70-78). Loads are 16 bytes per lane and
// consecutive lanes read consecutive 16-byte chunks (a wave reads 1 KiB
// contiguous per instruction); stores are 8 bytes per lane, likewise
// contiguous.
#include <stdint.h>

#include <type_traits>

#include "vdn_common.h"

namespace vdn {
namespace {

constexpr int kWavesPerBlock = 4;  // waves per workgroup

// Outputs (codes, normed rows) of at least this many bytes are stored
// non-temporally: beyond what the 256 MB last-level cache holds the cached stores
// only evict each other ([32760, 13824] codes: 0.229 ms against 0.251 ms), while
// smaller outputs stay in that cache for the kernel that reads them next
// ([32760, 5120] codes: 0.084 ms cached, 0.086 ms non-temporal).
constexpr int64_t kNtStoreBytes = 256ll << 20;

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
template <bool NT>
__device__ __forceinline__ void store_normed(uint4* p, uint4 v)
{
    if (NT) __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t*>(p));
    else *p = v;
}

template <bool NT>
__device__ __forceinline__ void store_codes(uint2* p, uint2 v)
{
    if (NT) __builtin_nontemporal_store(u32x2_t{v.x, v.y}, reinterpret_cast<u32x2_t*>(p));
    else *p = v;
}
constexpr int kLanes = 64;

// Quotient of the activation quantizer. kExact uses the IEEE division, for the
// rows whose scale is not finite (a row holding inf or NaN), where the
// reciprocal form does not apply.
template <bool kExact>
__device__ __forceinline__ float quotient(float x, float s, float r)
{
    return kExact ? x / s : div_by_scale(x, s, r);
}

// Converts one 16-byte chunk (8 bf16) to 8 codes. The weight path rounds the
// binary32 quotient by bf16(scale) to bf16 first (the reference's bf16 divide);
// there both operands are bf16, and RN_bf16(x * RN(1/s)) equals RN_bf16(x / s)
// for every such pair (checked exhaustively), so one multiply replaces the
// division, two quotients share one bf16 conversion, and the codes are converted
// from the packed bf16 quotients.
template <bool kWeight, bool kExact>
__device__ __forceinline__ uint2 quantize_chunk(uint4 v, float s, float r)
{
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint2 out;
    if (kWeight && !kExact) {
        uint32_t p[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] = pack_bf16x2(bf16_lo(w[e]) * r, bf16_hi(w[e]) * r);
        asm volatile("" : "+v"(p[0]), "+v"(p[1]), "+v"(p[2]), "+v"(p[3]));   // keep each pair in one conversion
        out.x = pack_e4m3x4_bf16(p[0], p[1]);
        out.y = pack_e4m3x4_bf16(p[2], p[3]);
        return out;
    }
    float q[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        q[2 * e] = quotient<kExact>(bf16_lo(w[e]), s, r);
        q[2 * e + 1] = quotient<kExact>(bf16_hi(w[e]), s, r);
        if (kWeight) { q[2 * e] = round_bf16(q[2 * e]); q[2 * e + 1] = round_bf16(q[2 * e + 1]); }
    }
    out.x = pack_e4m3x4(q[0], q[1], q[2], q[3]);
    out.y = pack_e4m3x4(q[4], q[5], q[6], q[7]);
    return out;
}

// WPR waves share a row (1, 2 or 4); CPL = 16-byte chunks held per lane, with
// CPL*64*WPR >= K/8. Wave part p of a row holds chunks p*64 + lane + 64*WPR*c,
// so the waves of a row read interleaved 1 KiB blocks; their row maxima meet in
// LDS. More waves per row cut the registers per wave and multiply the
// workgroups: [32760, 5120] activations in 0.075 ms with two against 0.077 ms with
// one (non-temporal loads in both), 76.3 against 77.3 us with four against two.
// GELU: the row is first replaced by bf16(gelu_tanh(x)) of each element (the GEMM
// epilogue's GELU of its bf16 output, so the codes are those of that epilogue's output
// quantized by this kernel).
template <int CPL, bool kWeight, int WPR, bool NT, bool GELU = false>
__global__ __launch_bounds__(kWavesPerBlock * kLanes) void k_rowquant(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, int64_t ldx,
    uint8_t* __restrict__ y, int64_t ldy, float* __restrict__ scale_out)
{
    static_assert(WPR == 1 || WPR == 2 || WPR == 4, "one, two or four waves per row");
    __shared__ uint32_t smax[kWavesPerBlock];
    const int lane = threadIdx.x & (kLanes - 1), wave = threadIdx.x / kLanes;
    const int part = wave % WPR;
    const int64_t row = (int64_t)blockIdx.x * (kWavesPerBlock / WPR) + wave / WPR;
    if (WPR == 1 && row >= M) return;
    // (with two waves per row every wave reaches the barrier below)
    const bool valid = row < M;
    const int nch = (int)(K >> 3);
    const uint4* xr = reinterpret_cast<const uint4*>(x + (valid ? row : 0) * ldx);

    uint4 v[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int idx = part * kLanes + lane + kLanes * WPR * c;
        v[c] = (valid && idx < nch) ? load_once(xr + idx) : make_uint4(0u, 0u, 0u, 0u);
    }
    if constexpr (GELU) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            uint32_t w4[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) w4[e] = pack_bf16x2(gelu_tanh(bf16_lo(w4[e])), gelu_tanh(bf16_hi(w4[e])));
            v[c] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
    }
    uint32_t m2 = 0;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        m2 = absmax_bf16x2(m2, v[c].x);
        m2 = absmax_bf16x2(m2, v[c].y);
        m2 = absmax_bf16x2(m2, v[c].z);
        m2 = absmax_bf16x2(m2, v[c].w);
    }
    uint32_t mbits = wave_max_u32(max(m2 & 0xffffu, m2 >> 16));
    if (WPR > 1) {
        if (lane == 0) smax[wave] = mbits;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < WPR; ++w) mbits = max(mbits, smax[(wave / WPR) * WPR + w]);
    }
    const float scale = row_scale(bf16_to_f32((uint16_t)mbits));
    if (valid && part == 0 && lane == 0) scale_out[row] = scale;
    const float sdiv = kWeight ? round_bf16(scale) : scale;
    const float r = 1.0f / sdiv;

    uint2* yr = reinterpret_cast<uint2*>(y + (valid ? row : 0) * ldy);
    if (__builtin_isfinite(sdiv)) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int idx = part * kLanes + lane + kLanes * WPR * c;
            if (valid && idx < nch) store_codes<NT>(yr + idx, quantize_chunk<kWeight, false>(v[c], sdiv, r));
        }
    } else {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int idx = part * kLanes + lane + kLanes * WPR * c;
            if (valid && idx < nch) store_codes<NT>(yr + idx, quantize_chunk<kWeight, true>(v[c], sdiv, r));
        }
    }
}

// Rows wider than 64*32 chunks (K > 16384): two sweeps, the second re-reads
// the row (from L2 for all but the widest rows).
template <bool kWeight>
__global__ __launch_bounds__(kWavesPerBlock * kLanes) void k_rowquant_wide(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, int64_t ldx,
    uint8_t* __restrict__ y, int64_t ldy, float* __restrict__ scale_out)
{
    const int lane = threadIdx.x & (kLanes - 1);
    const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x / kLanes);
    if (row >= M) return;
    const int64_t nch = K >> 3;
    const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
    uint32_t m2 = 0;
    for (int64_t idx = lane; idx < nch; idx += kLanes) {
        uint4 v = xr[idx];
        m2 = absmax_bf16x2(m2, v.x);
        m2 = absmax_bf16x2(m2, v.y);
        m2 = absmax_bf16x2(m2, v.z);
        m2 = absmax_bf16x2(m2, v.w);
    }
    const uint32_t mbits = wave_max_u32(max(m2 & 0xffffu, m2 >> 16));
    const float scale = row_scale(bf16_to_f32((uint16_t)mbits));
    if (lane == 0) scale_out[row] = scale;
    const float sdiv = kWeight ? round_bf16(scale) : scale;
    const float r = 1.0f / sdiv;
    uint2* yr = reinterpret_cast<uint2*>(y + row * ldy);
    if (__builtin_isfinite(sdiv)) {
        for (int64_t idx = lane; idx < nch; idx += kLanes) yr[idx] = quantize_chunk<kWeight, false>(xr[idx], sdiv, r);
    } else {
        for (int64_t idx = lane; idx < nch; idx += kLanes) yr[idx] = quantize_chunk<kWeight, true>(xr[idx], sdiv, r);
    }
}

// ---------------------------------------------------------------------------
// SwiGLU + quantize
// ---------------------------------------------------------------------------

// a * g * sigmoid(g) in binary32 (the reference's Triton body, fp8_linear.py:88,96).
__device__ __forceinline__ float swiglu(float a, float g)
{
    return a * g * __fdividef(1.0f, 1.0f + __expf(-g));
}

template <int CPL>
__global__ __launch_bounds__(kWavesPerBlock * kLanes) void k_swiglu_quant(
    const uint16_t* __restrict__ h, int64_t M, int64_t K, int64_t ldh,
    uint8_t* __restrict__ y, int64_t ldy, float* __restrict__ scale_out)
{
    const int lane = threadIdx.x & (kLanes - 1);
    const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x / kLanes);
    if (row >= M) return;
    const int nch = (int)(K >> 3);
    const uint4* ar = reinterpret_cast<const uint4*>(h + row * ldh);
    const uint4* gr = reinterpret_cast<const uint4*>(h + row * ldh + K);

    float act[CPL][8];
    float amax = 0.0f;
    bool nan_seen = false;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int idx = lane + kLanes * c;
        uint4 a = make_uint4(0u, 0u, 0u, 0u), g = a;
        if (idx < nch) { a = load_once(ar + idx); g = load_once(gr + idx); }
        const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, gw[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            act[c][2 * j] = swiglu(bf16_lo(aw[j]), bf16_lo(gw[j]));
            act[c][2 * j + 1] = swiglu(bf16_hi(aw[j]), bf16_hi(gw[j]));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            nan_seen |= __builtin_isnan(act[c][j]);
            amax = fmaxf(amax, fabsf(act[c][j]));
        }
    }
    // Magnitudes are non-negative, so their binary32 patterns order like
    // unsigned integers; a NaN anywhere in the row makes the scale NaN.
    uint32_t mbits = wave_max_u32(nan_seen ? 0x7fc00000u : __float_as_uint(amax));
    const float scale = row_scale(__uint_as_float(mbits));
    if (lane == 0) scale_out[row] = scale;
    const float r = 1.0f / scale;
    const bool finite = __builtin_isfinite(scale);

    uint2* yr = reinterpret_cast<uint2*>(y + row * ldy);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int idx = lane + kLanes * c;
        if (idx >= nch) continue;
        float q[8];
        if (finite) {
#pragma unroll
            for (int j = 0; j < 8; ++j) q[j] = quotient<false>(act[c][j], scale, r);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) q[j] = quotient<true>(act[c][j], scale, r);
        }
        yr[idx] = make_uint2(pack_e4m3x4(q[0], q[1], q[2], q[3]), pack_e4m3x4(q[4], q[5], q[6], q[7]));
    }
}

// ---------------------------------------------------------------------------
// binary32 and binary16 rows (the reference's quantizers load any float type
// and compute in binary32, fp8_linear.py:72,77,89-90; its weight branch
// divides in the weight's own type, fp8_linear.py:264-265). A path for
// models that do not run in bf16: one wave per row and two sweeps (the row
// maximum, then the codes, the second reading the row again), IEEE division.
// ---------------------------------------------------------------------------

// torch's cast to e4m3fn does not saturate: a magnitude above 464 (halfway
// between 448 and the NaN pattern) becomes NaN, as inf and NaN do.
__device__ __forceinline__ float e4m3_domain(float q)
{
    return __builtin_fabsf(q) > 464.0f ? __builtin_copysignf(__builtin_nanf(""), q) : q;
}

// 16 bytes of a row as binary32 values (4 binary32 or 8 binary16 ones), and a
// rounding to the row's own type.
template <typename T> struct FloatRow;
template <> struct FloatRow<float> {
    static constexpr int kPer = 4;
    __device__ static void unpack(uint4 v, float (&o)[8])
    {
        o[0] = __uint_as_float(v.x); o[1] = __uint_as_float(v.y);
        o[2] = __uint_as_float(v.z); o[3] = __uint_as_float(v.w);
    }
    __device__ static float round(float v) { return v; }
};
template <> struct FloatRow<_Float16> {
    static constexpr int kPer = 8;
    __device__ static void unpack(uint4 v, float (&o)[8])
    {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            o[2 * e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[e] & 0xffffu));
            o[2 * e + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[e] >> 16));
        }
    }
    __device__ static float round(float v) { return (float)(_Float16)v; }
};

// The row maximum of binary32 magnitudes over the wave (NaN anywhere: NaN), then
// the scale max(amax / 448, 1e-12) as quantize_rows forms it.
__device__ __forceinline__ float float_row_scale(float amax, bool nan_seen)
{
    // non-negative binary32 patterns order like unsigned integers (NaN above inf)
    return row_scale(__uint_as_float(wave_max_u32(nan_seen ? 0x7fc00000u : __float_as_uint(amax))));
}

// Codes of up to 8 quotients: 4 (binary32 rows) or 8 bytes at byte offset kPer c.
template <int kPer>
__device__ __forceinline__ void store_float_codes(uint8_t* yr, int64_t c, const float (&q)[8])
{
    if (kPer == 4) *reinterpret_cast<uint32_t*>(yr + 4 * c) = pack_e4m3x4(q[0], q[1], q[2], q[3]);
    else *reinterpret_cast<uint2*>(yr + 8 * c) = make_uint2(pack_e4m3x4(q[0], q[1], q[2], q[3]),
                                                            pack_e4m3x4(q[4], q[5], q[6], q[7]));
}

//   scale[m] = max(max_k |x[m][k]| / 448, 1e-12)
//   y[m][k]  = e4m3(x[m][k] / scale[m])                    (activations)
//   y[m][k]  = e4m3(T(x[m][k] / T(scale[m])))              (kWeight: the weight's own type)
template <typename T, bool kWeight>
__global__ __launch_bounds__(kWavesPerBlock * kLanes) void k_rowquant_float(
    const T* __restrict__ x, int64_t M, int64_t K, int64_t ldx,
    uint8_t* __restrict__ y, int64_t ldy, float* __restrict__ scale_out)
{
    using R = FloatRow<T>;
    const int lane = threadIdx.x & (kLanes - 1);
    const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x / kLanes);
    if (row >= M) return;
    const int64_t nch = K / R::kPer;
    const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
    float amax = 0.0f;
    bool nan_seen = false;
    for (int64_t c = lane; c < nch; c += kLanes) {
        float v[8];
        R::unpack(xr[c], v);
#pragma unroll
        for (int e = 0; e < R::kPer; ++e) {
            nan_seen |= __builtin_isnan(v[e]);
            amax = fmaxf(amax, fabsf(v[e]));
        }
    }
    const float scale = float_row_scale(amax, nan_seen);
    if (lane == 0) scale_out[row] = scale;
    const float sdiv = kWeight ? R::round(scale) : scale;
    uint8_t* yr = y + row * ldy;
    for (int64_t c = lane; c < nch; c += kLanes) {
        float v[8], q[8];
        R::unpack(xr[c], v);
#pragma unroll
        for (int e = 0; e < R::kPer; ++e) {
            const float t = v[e] / sdiv;
            q[e] = e4m3_domain(kWeight ? R::round(t) : t);
        }
        store_float_codes<R::kPer>(yr, c, q);
    }
}

// SwiGLU + quantize of binary32 / binary16 rows h [M, 2K] (value half, then gate
// half): act = a * g * sigmoid(g) in binary32 as k_swiglu_quant forms it, formed
// again in the second sweep.
template <typename T>
__global__ __launch_bounds__(kWavesPerBlock * kLanes) void k_swiglu_quant_float(
    const T* __restrict__ h, int64_t M, int64_t K, int64_t ldh,
    uint8_t* __restrict__ y, int64_t ldy, float* __restrict__ scale_out)
{
    using R = FloatRow<T>;
    const int lane = threadIdx.x & (kLanes - 1);
    const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x / kLanes);
    if (row >= M) return;
    const int64_t nch = K / R::kPer;
    const uint4* ar = reinterpret_cast<const uint4*>(h + row * ldh);
    const uint4* gr = reinterpret_cast<const uint4*>(h + row * ldh + K);
    auto acts = [&](int64_t c, float (&o)[8]) {
        float a[8], g[8];
        R::unpack(ar[c], a);
        R::unpack(gr[c], g);
#pragma unroll
        for (int e = 0; e < R::kPer; ++e) o[e] = swiglu(a[e], g[e]);
    };
    float amax = 0.0f;
    bool nan_seen = false;
    for (int64_t c = lane; c < nch; c += kLanes) {
        float v[8];
        acts(c, v);
#pragma unroll
        for (int e = 0; e < R::kPer; ++e) {
            nan_seen |= __builtin_isnan(v[e]);
            amax = fmaxf(amax, fabsf(v[e]));
        }
    }
    const float scale = float_row_scale(amax, nan_seen);
    if (lane == 0) scale_out[row] = scale;
    uint8_t* yr = y + row * ldy;
    for (int64_t c = lane; c < nch; c += kLanes) {
        float v[8], q[8];
        acts(c, v);
#pragma unroll
        for (int e = 0; e < R::kPer; ++e) q[e] = e4m3_domain(v[e] / scale);
        store_float_codes<R::kPer>(yr, c, q);
    }
}

// ---------------------------------------------------------------------------
// RMSNorm + AdaLN affine + quantize
// ---------------------------------------------------------------------------

struct NormArgs {
    const uint16_t* x;
    int64_t M, K, ldx;
    const uint16_t* weight;   // [K] or NULL
    float eps;
    const uint16_t* mod_scale;  // [T, K] or NULL (then mod_shift is NULL too)
    const uint16_t* mod_shift;
    int64_t ldmod;
    const int32_t* mod_index;   // [M] or NULL (row 0)
    int64_t mod_rows;
    uint8_t* y;
    int64_t ldy;
    float* y_scale;
    uint16_t* normed;           // [M, K] or NULL
    int64_t ldn;
};

__device__ __forceinline__ float wave_sum_f32(float v)
{
    // pairwise within the rows (both lanes of each exchange form the same sum), then
    // (row 0 + row 1) + (row 2 + row 3), wave-uniform
    v += __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(v)));
    v += __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(v)));
    v += __uint_as_float(dpp_u32<kDppHalfMirror>(__float_as_uint(v)));
    v += __uint_as_float(dpp_u32<kDppMirror>(__float_as_uint(v)));
    const uint32_t u = __float_as_uint(v);
    const float r0 = __uint_as_float(__builtin_amdgcn_readlane(u, 0)), r1 = __uint_as_float(__builtin_amdgcn_readlane(u, 16)),
                r2 = __uint_as_float(__builtin_amdgcn_readlane(u, 32)), r3 = __uint_as_float(__builtin_amdgcn_readlane(u, 48));
    return (r0 + r1) + (r2 + r3);
}

// The block's pre-norm fused with the per-token quantization:
//   rstd   = rsqrt(sum_k x^2 / K + eps)     (binary32, v_rsq_f32: within 1 ulp, as rms_norm's rsqrt)
//   n[k]   = bf16(fma(x[k] * rstd, f[k], shift[i][k]))   f = w (1 + scale[i]),
//                                                         (x[k] * rstd) * w[k] without a table
//   y, s   = the quantize_rows arithmetic on n
// with i = mod_index[row] (clamped into the table). The affine's association
// differs from the compiled `pre`'s ((x rstd) w)(1 + scale) + shift (its fp32
// operation order is unspecified); the normed values stay within one bf16
// rounding of the float64 restatement. The codes follow from the bf16 n exactly
// as quantize_rows' do. Without codes (QUANT false) the call is the pre-norm
// alone, with the same n, so the fused and unfused forms of a block give the
// same bits.
// WPR waves share a row (1, 2 or 4): wave part p holds chunks p*64 + lane +
// 64*WPR*c; the partial sums of squares and the row maxima meet in LDS (summed
// in part order, so every wave of the row gets the same rstd). Each group of
// WPR waves walks a contiguous block of `rb` rows, the next row's loads in
// flight while the current one is computed. The per-column factors f and the
// shift (binary32) stay in VGPRs and are formed again only when the table row
// changes (a frame of tokens shares one), so a row costs its own bytes and
// three binary32 operations per element before the rounding. Up to five chunks
// per lane, the waves-per-EU bound holds the kernel to 168 VGPRs, so three waves
// share each SIMD (wider rows need more registers and run two).
template <int CPL, int WPR, bool NT, bool AFFINE, bool QUANT>
__global__ __launch_bounds__(WPR * kLanes) __attribute__((amdgpu_waves_per_eu(CPL <= 5 ? 3 : 1))) void k_norm_quant_blocks(NormArgs p, int64_t rb)
{
    // one group of WPR waves (one row at a time) per workgroup: the barriers that
    // combine a row's partial sums hold up only the waves of that row
    // The partial sums of squares alternate between two slots by row parity: the
    // norm-only form meets one barrier per row, so a wave may write the next row's
    // sum while another still reads this row's.
    __shared__ float ssum[2][WPR];
    __shared__ uint32_t smax[WPR];
    const int lane = threadIdx.x & (kLanes - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kLanes);
    const int part = wave % WPR;
    const int64_t gid = (int64_t)blockIdx.x;
    const int64_t row0 = gid * rb;
    const int64_t row_end = min(p.M, row0 + rb);
    const int nch = (int)(p.K >> 3);
    const int rowbytes = nch * 16;
    auto chunk_off = [&](int c) { return (uint32_t)(part * kLanes + lane + kLanes * WPR * c) * 16u; };
    // Rows and row addresses as wave-uniform values (scalar registers): the buffer
    // descriptors built from them need no per-lane loop.
    auto uniform = [](int64_t v) -> int64_t {
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
        return (int64_t)(((uint64_t)hi << 32) | lo);
    };
    // Buffer loads: chunks past K (and every chunk of a row past the block) fall
    // outside the descriptor's range and read as zeros, with no branch.
    auto load_row = [&](int64_t row, uint4 (&v)[CPL]) {
        const bool valid = row < row_end;
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)uniform((int64_t)(p.x + (valid ? row : 0) * p.ldx)), 0, valid ? rowbytes : 0, 0x00020000);
#pragma unroll
        for (int c = 0; c < CPL; ++c)
            v[c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xrs, chunk_off(c), 0, kBufferLoadOnce));
    };
    float f[CPL][8], h[CPL][8];
    auto load_factors = [&](int64_t ti) {
        const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(p.weight ? p.weight : p.x), 0, p.weight ? rowbytes : 0, 0x00020000);
        const __amdgpu_buffer_rsrc_t scs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(AFFINE ? p.mod_scale + ti * p.ldmod : p.x), 0, AFFINE ? rowbytes : 0, 0x00020000);
        const __amdgpu_buffer_rsrc_t shs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(AFFINE ? p.mod_shift + ti * p.ldmod : p.x), 0, AFFINE ? rowbytes : 0, 0x00020000);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint4 wv = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wrs, chunk_off(c), 0, 0));
            const uint4 sc = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(scs, chunk_off(c), 0, 0));
            const uint4 sh = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(shs, chunk_off(c), 0, 0));
            const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w}, sw[4] = {sc.x, sc.y, sc.z, sc.w},
                           hw[4] = {sh.x, sh.y, sh.z, sh.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float w0 = p.weight ? bf16_lo(ww[e]) : 1.0f, w1 = p.weight ? bf16_hi(ww[e]) : 1.0f;
                f[c][2 * e] = AFFINE ? w0 * (1.0f + bf16_lo(sw[e])) : w0;
                f[c][2 * e + 1] = AFFINE ? w1 * (1.0f + bf16_hi(sw[e])) : w1;
                h[c][2 * e] = AFFINE ? bf16_lo(hw[e]) : 0.0f;
                h[c][2 * e + 1] = AFFINE ? bf16_hi(hw[e]) : 0.0f;
            }
        }
    };
    auto table_row = [&](int64_t row) -> int64_t {
        if (!AFFINE || !p.mod_index || row >= row_end) return 0;
        // wave-uniform (one row per wave group): kept in scalar registers, so the
        // table descriptors are too
        const int32_t ti = __builtin_amdgcn_readfirstlane(p.mod_index[row]);
        return min(max((int64_t)ti, (int64_t)0), p.mod_rows - 1);
    };

    uint4 va[CPL], vb[CPL];
    load_row(row0, va);
    int64_t cur_ti = table_row(row0);
    load_factors(cur_ti);
    auto one_row = [&](int64_t row_in, uint4 (&v)[CPL], uint4 (&vn)[CPL], int par) {
        const int64_t row = uniform(row_in);
        load_row(row + 1, vn);                       // the next row, in flight meanwhile
        __builtin_amdgcn_sched_barrier(0);
        const bool valid = row < row_end;
        if (AFFINE && p.mod_index) {
            const int64_t ti = table_row(row);
            if (ti != cur_ti) {                      // wave-uniform: a new frame's table row
                cur_ti = ti;
                load_factors(ti);
            }
        }
        // sum of squares straight from the packed bf16 pairs (v_dot2c_f32_bf16: no
        // unpacking), four partial sums to keep the chains short
        float ssp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t w4[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                ssp[e] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w4[e]),
                                                         __builtin_bit_cast(bf16x2_t, w4[e]), ssp[e], false);
        }
        float ss = wave_sum_f32((ssp[0] + ssp[1]) + (ssp[2] + ssp[3]));
        if (WPR > 1) {
            if (lane == 0) ssum[par][wave] = ss;
            __syncthreads();
            ss = ssum[par][0];
#pragma unroll
            for (int w = 1; w < WPR; ++w) ss += ssum[par][w];
        }
        const float rstd = __builtin_amdgcn_rsqf(ss / (float)p.K + p.eps);   // v_rsq_f32 (1 ulp)
        float mf = 0.0f;                             // row maximum of |n| (binary32)
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t xw[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float a = bf16_lo(xw[e]) * rstd, b = bf16_hi(xw[e]) * rstd;
                if (AFFINE) {
                    a = __builtin_fmaf(a, f[c][2 * e], h[c][2 * e]);
                    b = __builtin_fmaf(b, f[c][2 * e + 1], h[c][2 * e + 1]);
                } else {
                    a *= f[c][2 * e];
                    b *= f[c][2 * e + 1];
                }
                o[e] = pack_bf16x2(a, b);
                // max(|a|, |b|, mf) in one v_maximum3_f32 (NaN propagates)
                mf = __builtin_elementwise_maximum(
                    mf, __builtin_elementwise_maximum(__builtin_fabsf(a), __builtin_fabsf(b)));
            }
            // chunks past K hold zeros (x = 0, f = 0, shift = 0): nothing to the maximum
            v[c] = make_uint4(o[0], o[1], o[2], o[3]);
        }
        const __amdgpu_buffer_rsrc_t nrs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)uniform((int64_t)(p.normed ? p.normed + (valid ? row : 0) * p.ldn : nullptr)), 0,
            (valid && p.normed) ? rowbytes : 0, 0x00020000);
        if (!QUANT) {                                // the pre-norm alone (bf16 out)
#pragma unroll
            for (int c = 0; c < CPL; ++c)
                store_b128_settled<NT ? kBufferLoadOnce : 0>(__builtin_bit_cast(i32x4_t, v[c]), nrs, chunk_off(c), 0);
            return;
        }
        // bf16 rounding is monotone and odd, so the bf16 of the binary32 maximum of |n|
        // is the maximum of the rounded |n| quantize_rows takes (NaN stays NaN)
        uint32_t mbits = wave_max_u32(pack_bf16x2(mf, 0.0f) & 0x7fffu);
        if (WPR > 1) {
            if (lane == 0) smax[wave] = mbits;
            __syncthreads();
#pragma unroll
            for (int w = 0; w < WPR; ++w) mbits = max(mbits, smax[w]);
        }
        const float scale = row_scale(bf16_to_f32((uint16_t)mbits));
        if (valid && part == 0 && lane == 0) p.y_scale[row] = scale;
        const float r = 1.0f / scale;
        const bool finite = __builtin_isfinite(scale);
        const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)uniform((int64_t)(p.y + (valid ? row : 0) * p.ldy)), 0, valid ? nch * 8 : 0, 0x00020000);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t off = chunk_off(c);
            if (p.normed)
                store_b128_settled<NT ? kBufferLoadOnce : 0>(__builtin_bit_cast(i32x4_t, v[c]), nrs, off, 0);
            const uint2 q = finite ? quantize_chunk<false, false>(v[c], scale, r) : quantize_chunk<false, true>(v[c], scale, r);
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2_t, q), yrs, off / 2, 0, 0);
        }
    };
    for (int64_t i = 0; i < rb; i += 2) {
        one_row(row0 + i, va, vb, 0);
        if (i + 1 < rb) one_row(row0 + i + 1, vb, va, 1);
    }
}

// The per-column factors of the pre-norm for one 16-byte chunk q of table row ti:
// f = w (1 + scale[ti]) and the shift (w alone and zero without a table); chunks
// past K read as zeros.
template <bool AFFINE>
__device__ __forceinline__ void norm_factors(const NormArgs& p, int64_t ti, int q, int rowbytes, float (&f)[8],
                                             float (&h)[8])
{
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.weight ? p.weight : p.x), 0, p.weight ? rowbytes : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t scs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(AFFINE ? p.mod_scale + ti * p.ldmod : p.x), 0, AFFINE ? rowbytes : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t shs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(AFFINE ? p.mod_shift + ti * p.ldmod : p.x), 0, AFFINE ? rowbytes : 0, 0x00020000);
    const uint32_t off = (uint32_t)q * 16u;
    const uint4 wv = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 0));
    const uint4 sc = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(scs, off, 0, 0));
    const uint4 sh = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(shs, off, 0, 0));
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w}, sw[4] = {sc.x, sc.y, sc.z, sc.w}, hw[4] = {sh.x, sh.y, sh.z, sh.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float w0 = p.weight ? bf16_lo(ww[e]) : 1.0f, w1 = p.weight ? bf16_hi(ww[e]) : 1.0f;
        f[2 * e] = AFFINE ? w0 * (1.0f + bf16_lo(sw[e])) : w0;
        f[2 * e + 1] = AFFINE ? w1 * (1.0f + bf16_hi(sw[e])) : w1;
        h[2 * e] = AFFINE ? bf16_lo(hw[e]) : 0.0f;
        h[2 * e + 1] = AFFINE ? bf16_hi(hw[e]) : 0.0f;
    }
}

// The same pre-norm + quantization, one wave per row, for rows of up to 64 CPL
// chunks (CPL <= 14: the DiT's 5120 and H3's 5376 and 7168). One workgroup of W
// waves per CU walks a contiguous block of rows, wave w taking rows w, w + W, ..
// of it, the next one's loads in flight while a row is computed. The per-column factors sit in LDS for two table
// rows -- those of the block's first and last rows, so every row of a block that
// spans at most two frames of tokens finds its own; any other row forms its
// factors from the tables itself -- so the registers hold only the rows, and a
// row needs no exchange with another wave: its sum of squares and maximum are
// wave reductions. Chunk q of a row is lane q % 64's chunk q / 64; the factor
// slots keep the low and high four values of each chunk apart, so the 64 lanes'
// 16-byte reads cover consecutive addresses.
// Waves per workgroup: three per SIMD while the two row buffers leave room (168
// VGPRs), two for rows of more than 512 chunks -- except with the table (the affine
// form) at 640 and 704 chunks, where twelve fit once the next row's loads go out after
// the row's normalization instead of before (0.0880 against 0.0907 ms with eight waves
// and the early loads at 640; H3's 5376-wide rows, 672 chunks, as 11 per lane:
// [13107, 5376] 0.0428 against 0.0471 ms with eight waves and 12 per lane). With the late
// loads, the next row's first kNormEarlyChunks chunks per lane still go out before the
// normalization (the registers hold that much beside it): [13107, 5376] 41.2 against
// 42.5 us (0, 2, 3, 4 and 6 early chunks: 42.6, 41.9, 41.3, 41.2, 41.3 us; the
// [32760, 5120] rows 88.3 against 88.6 us).
constexpr int norm_row_waves(int cpl, bool affine) { return cpl <= 8 || ((cpl == 10 || cpl == 11) && affine) ? 12 : 8; }
constexpr bool norm_row_late_load(int cpl, bool affine) { return cpl > 8 && norm_row_waves(cpl, affine) == 12; }
constexpr int kNormEarlyChunks = 4;
// Rows in flight per wave besides the one computed (two, in the registers two waves
// per SIMD leave at 64 chunks x 10, measured 0.0911 ms against 0.0891 ms with one).
constexpr int norm_row_lookahead(int) { return 1; }
template <int CPL, bool NT, bool AFFINE, bool QUANT>
__global__ __launch_bounds__(norm_row_waves(CPL, AFFINE) * kLanes) void k_norm_quant_rows(NormArgs p, int64_t rb)
{
    constexpr int kNormRowWaves = norm_row_waves(CPL, AFFINE), LA = norm_row_lookahead(CPL);
    constexpr bool kLate = norm_row_late_load(CPL, AFFINE);
    constexpr int NQ = CPL * kLanes;
    __shared__ float4 sf[2][2][NQ], sh[2][2][NQ];
    const int lane = threadIdx.x & (kLanes - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kLanes);
    const int64_t row0 = (int64_t)blockIdx.x * rb;
    const int64_t row_end = min(p.M, row0 + rb);
    const int nch = (int)(p.K >> 3);
    const int rowbytes = nch * 16;
    // the lane's part of every row offset; the chunk's part (a multiple of 1 KiB) goes
    // in the instructions' scalar offset
    const uint32_t lane16 = (uint32_t)lane * 16u;
    auto uniform = [](int64_t v) -> int64_t {
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
        return (int64_t)(((uint64_t)hi << 32) | lo);
    };
    // chunks c0 .. c1 - 1 of a row (per lane)
    auto load_part = [&](int64_t row, uint4 (&v)[CPL], int c0, int c1) {
        const bool valid = row < row_end;
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)uniform((int64_t)(p.x + (valid ? row : 0) * p.ldx)), 0, valid ? rowbytes : 0, 0x00020000);
#pragma unroll
        for (int c = 0; c < CPL; ++c)
            if (c >= c0 && c < c1)
                v[c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xrs, lane16, c * kLanes * 16,
                                                                                      kBufferLoadOnce));
    };
    auto load_row = [&](int64_t row, uint4 (&v)[CPL]) { load_part(row, v, 0, CPL); };
    auto table_row = [&](int64_t row) -> int64_t {
        if (!AFFINE || !p.mod_index || row >= row_end) return 0;
        const int32_t ti = __builtin_amdgcn_readfirstlane(p.mod_index[row]);
        return min(max((int64_t)ti, (int64_t)0), p.mod_rows - 1);
    };
    constexpr int kEarly = kLate ? kNormEarlyChunks : CPL;   // chunks of the next row loaded before the normalization

    uint4 vbuf[LA + 1][CPL];                         // buffer j: rows j, j + LA + 1, .. of this wave
#pragma unroll
    for (int j = 0; j < LA; ++j) load_row(row0 + wave + j * kNormRowWaves, vbuf[j]);   // in flight while the slots fill
    const int64_t t0 = table_row(row0), t1 = table_row(row_end - 1);
    for (int q = threadIdx.x; q < NQ; q += kNormRowWaves * kLanes) {
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) {
            if (sl == 1 && t1 == t0) break;          // one table row: slot 1 is never chosen
            float f[8], h[8];
            norm_factors<AFFINE>(p, sl ? t1 : t0, q, rowbytes, f, h);
            sf[sl][0][q] = make_float4(f[0], f[1], f[2], f[3]);
            sf[sl][1][q] = make_float4(f[4], f[5], f[6], f[7]);
            sh[sl][0][q] = make_float4(h[0], h[1], h[2], h[3]);
            sh[sl][1][q] = make_float4(h[4], h[5], h[6], h[7]);
        }
    }
    __syncthreads();

    auto one_row = [&](int64_t row_in, uint4 (&v)[CPL], uint4 (&vn)[CPL]) {
        const int64_t row = uniform(row_in);
        load_part(row + LA * kNormRowWaves, vn, 0, kEarly);   // into the buffer the previous row freed
        __builtin_amdgcn_sched_barrier(0);
        const bool valid = row < row_end;
        const int64_t ti = table_row(row);
        const int slot = !valid || ti == t0 ? 0 : ti == t1 ? 1 : -1;   // wave-uniform
        float ssp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t w4[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                ssp[e] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w4[e]),
                                                         __builtin_bit_cast(bf16x2_t, w4[e]), ssp[e], false);
        }
        const float ss = wave_sum_f32((ssp[0] + ssp[1]) + (ssp[2] + ssp[3]));
        const float rstd = __builtin_amdgcn_rsqf(ss / (float)p.K + p.eps);   // v_rsq_f32 (1 ulp)
        float mf = 0.0f;                             // row maximum of |n| (binary32)
        auto norm_chunk = [&](int c, const float (&f)[8], const float (&h)[8]) {
            const uint32_t xw[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float a = bf16_lo(xw[e]) * rstd, b = bf16_hi(xw[e]) * rstd;
                if (AFFINE) {
                    a = __builtin_fmaf(a, f[2 * e], h[2 * e]);
                    b = __builtin_fmaf(b, f[2 * e + 1], h[2 * e + 1]);
                } else {
                    a *= f[2 * e];
                    b *= f[2 * e + 1];
                }
                o[e] = pack_bf16x2(a, b);
                mf = __builtin_elementwise_maximum(
                    mf, __builtin_elementwise_maximum(__builtin_fabsf(a), __builtin_fabsf(b)));
            }
            // chunks past K hold zeros (x = 0, f = 0, shift = 0): nothing to the maximum
            v[c] = make_uint4(o[0], o[1], o[2], o[3]);
        };
        if (slot >= 0) {
            // the factors from the slot, each chunk's read one chunk ahead of its use (the
            // scheduling barriers keep the compiler from hoisting every read, and the
            // registers they would hold, to the top)
            float f[2][8], h[2][8];
            auto read = [&](int c, float (&fo)[8], float (&ho)[8]) {
                const int q = lane + kLanes * c;
                const float4 f0 = sf[slot][0][q], f1 = sf[slot][1][q];
                fo[0] = f0.x; fo[1] = f0.y; fo[2] = f0.z; fo[3] = f0.w; fo[4] = f1.x; fo[5] = f1.y; fo[6] = f1.z; fo[7] = f1.w;
                if (AFFINE) {
                    const float4 h0 = sh[slot][0][q], h1 = sh[slot][1][q];
                    ho[0] = h0.x; ho[1] = h0.y; ho[2] = h0.z; ho[3] = h0.w; ho[4] = h1.x; ho[5] = h1.y; ho[6] = h1.z; ho[7] = h1.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) ho[e] = 0.0f;
                }
            };
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                read(c, f[0], h[0]);
                norm_chunk(c, f[0], h[0]);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            // a table row outside both slots: the factors from the tables, chunk by chunk
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                float f[8], h[8];
                norm_factors<AFFINE>(p, ti, lane + kLanes * c, rowbytes, f, h);
                norm_chunk(c, f, h);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (kLate) {
            __builtin_amdgcn_sched_barrier(0);
            load_part(row + LA * kNormRowWaves, vn, kEarly, CPL);  // once the row's factors no longer hold registers
            __builtin_amdgcn_sched_barrier(0);
        }
        const __amdgpu_buffer_rsrc_t nrs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)uniform((int64_t)(p.normed ? p.normed + (valid ? row : 0) * p.ldn : nullptr)), 0,
            (valid && p.normed) ? rowbytes : 0, 0x00020000);
        if (!QUANT) {
#pragma unroll
            for (int c = 0; c < CPL; ++c)
                store_b128_settled<NT ? kBufferLoadOnce : 0>(__builtin_bit_cast(i32x4_t, v[c]), nrs, lane16,
                                                             c * kLanes * 16);
            return;
        }
        const uint32_t mbits = wave_max_u32(pack_bf16x2(mf, 0.0f) & 0x7fffu);
        const float scale = row_scale(bf16_to_f32((uint16_t)mbits));
        if (valid && lane == 0) p.y_scale[row] = scale;
        const float r = 1.0f / scale;
        const bool finite = __builtin_isfinite(scale);
        const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)uniform((int64_t)(p.y + (valid ? row : 0) * p.ldy)), 0, valid ? nch * 8 : 0, 0x00020000);
        auto out_chunk = [&](int c, uint2 q) {
            if (p.normed)
                store_b128_settled<NT ? kBufferLoadOnce : 0>(__builtin_bit_cast(i32x4_t, v[c]), nrs, lane16,
                                                             c * kLanes * 16);
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2_t, q), yrs, lane16 / 2, c * kLanes * 8, 0);
            __builtin_amdgcn_sched_barrier(0);
        };
        if (finite) {                                // one uniform branch per row
#pragma unroll
            for (int c = 0; c < CPL; ++c) out_chunk(c, quantize_chunk<false, false>(v[c], scale, r));
        } else {                                     // a row holding inf or NaN: IEEE division
#pragma unroll
            for (int c = 0; c < CPL; ++c) out_chunk(c, quantize_chunk<false, true>(v[c], scale, r));
        }
    };
    // groups of LA + 1 rows, buffer j always holding the group's row j
    for (int64_t r = row0 + wave; r < row_end; r += (LA + 1) * kNormRowWaves) {
#pragma unroll
        for (int j = 0; j <= LA; ++j)
            if (j == 0 || r + j * kNormRowWaves < row_end)
                one_row(r + j * kNormRowWaves, vbuf[j], vbuf[(j + LA) % (LA + 1)]);
    }
}

// Wide rows (K > 8192 in the H3 FFN: 14336): WPR waves share a row, each holding
// every WPR-th 1 KiB slice of it, so the binary32 activations fit in registers at
// a useful occupancy; the row maximum is combined through LDS.
template <int CPL, int WPR, bool NT>
__global__ __launch_bounds__(kWavesPerBlock * kLanes) void k_swiglu_quant_split(
    const uint16_t* __restrict__ h, int64_t M, int64_t K, int64_t ldh,
    uint8_t* __restrict__ y, int64_t ldy, float* __restrict__ scale_out)
{
    static_assert(kWavesPerBlock % WPR == 0, "rows per workgroup");
    __shared__ uint32_t smax[kWavesPerBlock];
    const int lane = threadIdx.x & (kLanes - 1), wave = threadIdx.x / kLanes;
    const int part = wave % WPR;
    const int64_t row = (int64_t)blockIdx.x * (kWavesPerBlock / WPR) + wave / WPR;
    const bool valid = row < M;                      // no early return: the barrier below
    const int nch = (int)(K >> 3);
    const int64_t r0 = valid ? row : 0;
    const uint4* ar = reinterpret_cast<const uint4*>(h + r0 * ldh);
    const uint4* gr = reinterpret_cast<const uint4*>(h + r0 * ldh + K);

    float act[CPL][8];
    float amax = 0.0f;
    bool nan_seen = false;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int idx = part * kLanes + lane + kLanes * WPR * c;
        uint4 a = make_uint4(0u, 0u, 0u, 0u), g = a;
        if (valid && idx < nch) { a = load_once(ar + idx); g = load_once(gr + idx); }
        const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, gw[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            act[c][2 * j] = swiglu(bf16_lo(aw[j]), bf16_lo(gw[j]));
            act[c][2 * j + 1] = swiglu(bf16_hi(aw[j]), bf16_hi(gw[j]));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            nan_seen |= __builtin_isnan(act[c][j]);
            amax = fmaxf(amax, fabsf(act[c][j]));
        }
    }
    uint32_t mbits = wave_max_u32(nan_seen ? 0x7fc00000u : __float_as_uint(amax));
    if (lane == 0) smax[wave] = mbits;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < WPR; ++w) mbits = max(mbits, smax[(wave / WPR) * WPR + w]);
    if (!valid) return;
    const float scale = row_scale(__uint_as_float(mbits));
    if (part == 0 && lane == 0) scale_out[row] = scale;
    const float r = 1.0f / scale;
    const bool finite = __builtin_isfinite(scale);
    uint2* yr = reinterpret_cast<uint2*>(y + row * ldy);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int idx = part * kLanes + lane + kLanes * WPR * c;
        if (idx >= nch) continue;
        float q[8];
        if (finite) {
#pragma unroll
            for (int j = 0; j < 8; ++j) q[j] = quotient<false>(act[c][j], scale, r);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) q[j] = quotient<true>(act[c][j], scale, r);
        }
        store_codes<NT>(yr + idx, make_uint2(pack_e4m3x4(q[0], q[1], q[2], q[3]), pack_e4m3x4(q[4], q[5], q[6], q[7])));
    }
}

// Rows of 4096..16384 elements: four waves per row (chunks per lane rounded up to
// an instantiated CPL; [32760, 13824]: 0.224 ms against 0.229 ms with two; [32760,
// 5120] 76.3 against 77.3 us, the [15360, 5120] weight 39.4 against 39.9 us).
// Returns false for other widths.
template <bool kWeight, bool NT, bool GELU = false>
bool launch_rowquant_pair(hipStream_t st, const uint16_t* x, int64_t M, int64_t K, int64_t ldx,
                          uint8_t* y, int64_t ldy, float* s)
{
    const int64_t nch = K / 8;
    if (nch < 8 * kLanes || nch > 2 * 16 * kLanes) return false;
    const dim3 block(kWavesPerBlock * kLanes);
    const int64_t per = (nch + 4 * kLanes - 1) / (4 * kLanes);     // chunks per lane
    const dim3 grid((unsigned)M);
#define VDN_CASE(n)                                                                                    \
    if (per <= n) {                                                                                    \
        hipLaunchKernelGGL((k_rowquant<n, kWeight, 4, NT, GELU>), grid, block, 0, st, x, M, K, ldx, y, ldy, s); \
        return true;                                                                                   \
    }
    VDN_CASE(2) VDN_CASE(3) VDN_CASE(4) VDN_CASE(5) VDN_CASE(6) VDN_CASE(7) VDN_CASE(8)
#undef VDN_CASE
    return false;
}

template <bool kWeight, bool GELU = false>
void launch_rowquant(int cpl, dim3 grid, hipStream_t st, const uint16_t* x, int64_t M, int64_t K,
                     int64_t ldx, uint8_t* y, int64_t ldy, float* s)
{
    // non-temporal code stores for activation outputs beyond the last-level cache and for
    // every weight (its codes are read by later GEMMs, not by the next kernel: [15360,
    // 5120] 37.7 us against 38.3 us cached, weight read from HBM)
    const bool nt = kWeight || M * K >= kNtStoreBytes;
    if (nt ? launch_rowquant_pair<kWeight, true, GELU>(st, x, M, K, ldx, y, ldy, s)
           : launch_rowquant_pair<kWeight, false, GELU>(st, x, M, K, ldx, y, ldy, s))
        return;
    const dim3 block(kWavesPerBlock * kLanes);
#define VDN_CASE(n)                                                                           \
    case n:                                                                                   \
        if (nt) hipLaunchKernelGGL((k_rowquant<n, kWeight, 1, true, GELU>), grid, block, 0, st, x, M, K, ldx, y, ldy, s); \
        else hipLaunchKernelGGL((k_rowquant<n, kWeight, 1, false, GELU>), grid, block, 0, st, x, M, K, ldx, y, ldy, s); \
        return;
    switch (cpl) {
        VDN_CASE(1) VDN_CASE(2) VDN_CASE(3) VDN_CASE(4) VDN_CASE(6) VDN_CASE(8) VDN_CASE(10)
        VDN_CASE(12) VDN_CASE(16) VDN_CASE(20) VDN_CASE(24) VDN_CASE(28) VDN_CASE(32)
        default:   // (the GELU entry point takes rows of at most 16384 elements)
            if constexpr (!GELU) hipLaunchKernelGGL((k_rowquant_wide<kWeight>), grid, block, 0, st, x, M, K, ldx, y, ldy, s);
    }
#undef VDN_CASE
}

// Smallest instantiated chunks-per-lane that covers nch chunks, 0 for the wide kernel.

}  // namespace

}  // namespace vdn

using namespace vdn;

extern "C" int vdn_fp8_quantize_rows(const void* x, int64_t M, int64_t K, int64_t ldx, void* y,
                                     int64_t ldy, float* scale, hipStream_t stream)
{
    if (M < 0 || K < 0) return set_error(VDN_FP8_EINVAL, "quantize_rows: negative shape [%lld, %lld]", (long long)M, (long long)K);
    if (M == 0 || K == 0) {
        if (M > 0 && K == 0) return set_error(VDN_FP8_EINVAL, "quantize_rows: K must be positive");
        return VDN_FP8_OK;
    }
    if (!x || !y || !scale) return set_error(VDN_FP8_EINVAL, "quantize_rows: null pointer");
    if (K % 8 || ldx % 8 || ldy % 8 || ldx < K || ldy < K)
        return set_error(VDN_FP8_EINVAL, "quantize_rows: need K, ldx, ldy multiples of 8 and ldx, ldy >= K (K=%lld ldx=%lld ldy=%lld)",
                         (long long)K, (long long)ldx, (long long)ldy);
    if (!aligned(x, 16) || !aligned(y, 8) || !aligned(scale, 4))
        return set_error(VDN_FP8_EINVAL, "quantize_rows: x must be 16-byte and y 8-byte aligned");
    const dim3 grid((unsigned)((M + kWavesPerBlock - 1) / kWavesPerBlock));
    launch_rowquant<false>(pick_cpl(K / 8), grid, stream, (const uint16_t*)x, M, K, ldx, (uint8_t*)y, ldy, scale);
    return check_launch("quantize_rows");
}

extern "C" int vdn_fp8_gelu_quantize_rows(const void* h, int64_t M, int64_t K, int64_t ldh, void* y,
                                          int64_t ldy, float* scale, hipStream_t stream)
{
    if (M < 0 || K < 0) return set_error(VDN_FP8_EINVAL, "gelu_quantize_rows: negative shape [%lld, %lld]", (long long)M, (long long)K);
    if (M == 0 || K == 0) {
        if (M > 0 && K == 0) return set_error(VDN_FP8_EINVAL, "gelu_quantize_rows: K must be positive");
        return VDN_FP8_OK;
    }
    if (!h || !y || !scale) return set_error(VDN_FP8_EINVAL, "gelu_quantize_rows: null pointer");
    if (K % 8 || ldh % 8 || ldy % 8 || ldh < K || ldy < K)
        return set_error(VDN_FP8_EINVAL, "gelu_quantize_rows: need K, ldh, ldy multiples of 8 and ldh, ldy >= K (K=%lld ldh=%lld ldy=%lld)",
                         (long long)K, (long long)ldh, (long long)ldy);
    if (!aligned(h, 16) || !aligned(y, 8) || !aligned(scale, 4))
        return set_error(VDN_FP8_EINVAL, "gelu_quantize_rows: h must be 16-byte and y 8-byte aligned");
    if (K / 8 > 32 * kLanes) return set_error(VDN_FP8_EINVAL, "gelu_quantize_rows: K=%lld above the supported 16384", (long long)K);
    const dim3 grid((unsigned)((M + kWavesPerBlock - 1) / kWavesPerBlock));
    launch_rowquant<false, true>(pick_cpl(K / 8), grid, stream, (const uint16_t*)h, M, K, ldh, (uint8_t*)y, ldy, scale);
    return check_launch("gelu_quantize_rows");
}

extern "C" int vdn_fp8_swiglu_quantize_rows(const void* h, int64_t M, int64_t K, int64_t ldh, void* y,
                                            int64_t ldy, float* scale, hipStream_t stream)
{
    if (M < 0 || K < 0) return set_error(VDN_FP8_EINVAL, "swiglu_quantize_rows: negative shape");
    if (M == 0) return VDN_FP8_OK;
    if (K == 0) return set_error(VDN_FP8_EINVAL, "swiglu_quantize_rows: K must be positive");
    if (!h || !y || !scale) return set_error(VDN_FP8_EINVAL, "swiglu_quantize_rows: null pointer");
    if (K % 8 || ldh % 8 || ldy % 8 || ldh < 2 * K || ldy < K)
        return set_error(VDN_FP8_EINVAL, "swiglu_quantize_rows: need K, ldh, ldy multiples of 8, ldh >= 2K, ldy >= K");
    if (!aligned(h, 16) || !aligned(y, 8)) return set_error(VDN_FP8_EINVAL, "swiglu_quantize_rows: misaligned pointer");
    const int64_t nch = K / 8;
    if (nch > 32 * kLanes) return set_error(VDN_FP8_EINVAL, "swiglu_quantize_rows: K=%lld above the supported 16384", (long long)K);
    const dim3 grid((unsigned)((M + kWavesPerBlock - 1) / kWavesPerBlock)), block(kWavesPerBlock * kLanes);
    const uint16_t* hp = (const uint16_t*)h;
    uint8_t* yp = (uint8_t*)y;
    if (nch > 12 * kLanes) {            // K > 6144: four waves per row
        const dim3 g1((unsigned)M);
        const int cpl = pick_cpl((nch + 3) / 4);
        const bool nt = M * K >= kNtStoreBytes;
#define VDN_SPLIT(n)                                                                                                  \
        if (nt) hipLaunchKernelGGL((k_swiglu_quant_split<n, 4, true>), g1, block, 0, stream, hp, M, K, ldh, yp, ldy, scale); \
        else hipLaunchKernelGGL((k_swiglu_quant_split<n, 4, false>), g1, block, 0, stream, hp, M, K, ldh, yp, ldy, scale);
        if (cpl <= 4) { VDN_SPLIT(4) }
        else if (cpl <= 6) { VDN_SPLIT(6) }
        else { VDN_SPLIT(8) }
#undef VDN_SPLIT
        return check_launch("swiglu_quantize_rows");
    }
    switch (pick_cpl(nch)) {
#define VDN_CASE(n) case n: hipLaunchKernelGGL(k_swiglu_quant<n>, grid, block, 0, stream, hp, M, K, ldh, yp, ldy, scale); break;
        VDN_CASE(1) VDN_CASE(2) VDN_CASE(3) VDN_CASE(4) VDN_CASE(6) VDN_CASE(8) VDN_CASE(10)
        VDN_CASE(12) VDN_CASE(16) VDN_CASE(20) VDN_CASE(24) VDN_CASE(28) VDN_CASE(32)
#undef VDN_CASE
        default: return set_error(VDN_FP8_EINVAL, "swiglu_quantize_rows: unsupported K");
    }
    return check_launch("swiglu_quantize_rows");
}

namespace vdn {
namespace {
// k_norm_quant_blocks: WPR waves per row and workgroup, rows in blocks of rb per
// workgroup, kNormWavesPerCU waves per CU; false when no instantiated chunk count
// covers the row.
constexpr int kNormWavesPerCU = 12;
// k_norm_quant_rows: one workgroup per CU (fewer for short inputs), each walking a
// contiguous block of rows.
template <bool QUANT>
void launch_norm_rows(int64_t nch, int64_t M, const NormArgs& p, int cus, hipStream_t st)
{
    const bool nt = p.normed && M * nch * 16 >= kNtStoreBytes;   // the normed bf16 output
    const bool affine = p.mod_scale != nullptr;
    auto go = [&](auto cpl) {
        constexpr int n = decltype(cpl)::value;
        auto launch = [&](auto af) {
            constexpr bool AF = decltype(af)::value;
            constexpr int waves = norm_row_waves(n, AF);
            const int64_t wgs = min((int64_t)cus, (M + waves - 1) / waves);
            const int64_t rb = (M + wgs - 1) / wgs;
            const dim3 grid((unsigned)((M + rb - 1) / rb)), block(waves * kLanes);
            if (nt) hipLaunchKernelGGL((k_norm_quant_rows<n, true, AF, QUANT>), grid, block, 0, st, p, rb);
            else hipLaunchKernelGGL((k_norm_quant_rows<n, false, AF, QUANT>), grid, block, 0, st, p, rb);
        };
        if (affine) launch(std::true_type{});
        else launch(std::false_type{});
    };
    if (nch <= 6 * kLanes) go(std::integral_constant<int, 6>{});
    else if (nch <= 8 * kLanes) go(std::integral_constant<int, 8>{});
    else if (nch <= 10 * kLanes) go(std::integral_constant<int, 10>{});
    else if (nch <= 11 * kLanes) go(std::integral_constant<int, 11>{});   // H3's 5376
    else if (nch <= 12 * kLanes) go(std::integral_constant<int, 12>{});
    else go(std::integral_constant<int, 14>{});
}

template <int WPR, bool QUANT>
bool launch_norm_blocks(int64_t nch, int64_t M, const NormArgs& p, int cus, hipStream_t st)
{
    const bool nt = p.normed && M * nch * 16 >= kNtStoreBytes;   // the normed bf16 output
    const int64_t per = (nch + WPR * kLanes - 1) / (WPR * kLanes);
    const int64_t wgs = min((int64_t)cus * (kNormWavesPerCU / WPR), M);
    const int64_t rb = (M + wgs - 1) / wgs;
    const dim3 grid((unsigned)((M + rb - 1) / rb)), block(WPR * kLanes);
    const bool affine = p.mod_scale != nullptr;
#define VDN_LAUNCH(n, NT_, AF_) hipLaunchKernelGGL((k_norm_quant_blocks<n, WPR, NT_, AF_, QUANT>), grid, block, 0, st, p, rb)
#define VDN_CASE(n)                                                          \
    if (per <= n) {                                                          \
        if (affine) { if (nt) VDN_LAUNCH(n, true, true); else VDN_LAUNCH(n, false, true); }     \
        else { if (nt) VDN_LAUNCH(n, true, false); else VDN_LAUNCH(n, false, false); }          \
        return true;                                                         \
    }
    VDN_CASE(1) VDN_CASE(2) VDN_CASE(3) VDN_CASE(4) VDN_CASE(5) VDN_CASE(6) VDN_CASE(7) VDN_CASE(8)
#undef VDN_CASE
#undef VDN_LAUNCH
    return false;
}

}  // namespace
}  // namespace vdn

extern "C" int vdn_fp8_norm_quantize_rows(const void* x, int64_t M, int64_t K, int64_t ldx, const void* weight,
                                          float eps, const void* mod_scale, const void* mod_shift, int64_t ldmod,
                                          const int32_t* mod_index, int64_t mod_rows, void* y, int64_t ldy,
                                          float* y_scale, void* normed, int64_t ldn, hipStream_t stream)
{
    if (M < 0 || K < 0) return set_error(VDN_FP8_EINVAL, "norm_quantize_rows: negative shape");
    if (M == 0) return VDN_FP8_OK;
    if (K == 0) return set_error(VDN_FP8_EINVAL, "norm_quantize_rows: K must be positive");
    if (!x || (!y != !y_scale) || (!y && !normed))
        return set_error(VDN_FP8_EINVAL, "norm_quantize_rows: null pointer (y and y_scale may be NULL together "
                                         "only when normed is given)");
    if (!mod_scale != !mod_shift) return set_error(VDN_FP8_EINVAL, "norm_quantize_rows: scale and shift go together");
    if (K % 8 || ldx % 8 || ldx < K || (y && (ldy % 8 || ldy < K)) || (normed && (ldn % 8 || ldn < K)) ||
        (mod_scale && (ldmod % 8 || ldmod < K || mod_rows < 1)))
        return set_error(VDN_FP8_EINVAL, "norm_quantize_rows: need K and the row strides multiples of 8 and >= K, "
                                         "and a modulation table of >= 1 row");
    if (!(eps >= 0.0f)) return set_error(VDN_FP8_EINVAL, "norm_quantize_rows: eps must be >= 0");
    if (!aligned(x, 16) || (y && !aligned(y, 8)) || (weight && !aligned(weight, 16)) || (mod_scale && !aligned(mod_scale, 16)) ||
        (mod_shift && !aligned(mod_shift, 16)) || (normed && !aligned(normed, 16)) || (mod_index && !aligned(mod_index, 4)))
        return set_error(VDN_FP8_EINVAL, "norm_quantize_rows: misaligned pointer (x, weight, scale, shift, normed 16 B; y 8 B)");
    const int64_t nch = K / 8;
    if (nch > 32 * kLanes) return set_error(VDN_FP8_EINVAL, "norm_quantize_rows: K=%lld above the supported 16384", (long long)K);
    NormArgs p{(const uint16_t*)x, M, K, ldx, (const uint16_t*)weight, eps, (const uint16_t*)mod_scale,
               (const uint16_t*)mod_shift, ldmod, mod_index, mod_rows, (uint8_t*)y, ldy, y_scale, (uint16_t*)normed, ldn};
    // rows in blocks per wave group; one wave per row up to 2048 elements, two up to
    // 8192, four beyond
    const int cus = device_cus();
    if (cus <= 0) return set_error(VDN_FP8_ELAUNCH, "norm_quantize_rows: cannot query the device's compute units");
    // rows of 2049-7168 elements: one wave per row, the factors in LDS
    if (nch > 4 * kLanes && nch <= 14 * kLanes) {
        if (y) launch_norm_rows<true>(nch, M, p, cus, stream);
        else launch_norm_rows<false>(nch, M, p, cus, stream);
        return check_launch("norm_quantize_rows");
    }
    bool ok;
    if (y) ok = nch <= 4 * kLanes    ? launch_norm_blocks<1, true>(nch, M, p, cus, stream)
                : nch <= 16 * kLanes ? launch_norm_blocks<2, true>(nch, M, p, cus, stream)
                                     : launch_norm_blocks<4, true>(nch, M, p, cus, stream);
    else ok = nch <= 4 * kLanes    ? launch_norm_blocks<1, false>(nch, M, p, cus, stream)
              : nch <= 16 * kLanes ? launch_norm_blocks<2, false>(nch, M, p, cus, stream)
                                   : launch_norm_blocks<4, false>(nch, M, p, cus, stream);
    if (!ok) return set_error(VDN_FP8_EINVAL, "norm_quantize_rows: unsupported K");
    return check_launch("norm_quantize_rows");
}

namespace vdn {
int launch_lora_requant(const uint16_t* w, int64_t N, int64_t K, int64_t ldw, const uint16_t* a,
                        const uint16_t* b, int64_t rank, float lora_scale, uint8_t* wq, int64_t ldq,
                        float* w_scale, uint16_t* w_merged, hipStream_t stream);
}

extern "C" int vdn_fp8_requantize_weight(const void* w, int64_t N, int64_t K, int64_t ldw, const void* lora_a,
                                         const void* lora_b, int64_t rank, float lora_scale, void* wq,
                                         int64_t ldq, float* w_scale, void* w_merged, hipStream_t stream)
{
    if (N < 0 || K < 0) return set_error(VDN_FP8_EINVAL, "requantize_weight: negative shape");
    if (N == 0) return VDN_FP8_OK;
    if (K == 0) return set_error(VDN_FP8_EINVAL, "requantize_weight: K must be positive");
    const bool merge_only = !wq && !w_scale && w_merged && lora_a && lora_b;
    if (!w || (!merge_only && (!wq || !w_scale)))
        return set_error(VDN_FP8_EINVAL, "requantize_weight: null pointer (wq and w_scale may be NULL only "
                                         "for a LoRA merge into w_merged)");
    if (K % 8 || ldw % 8 || ldw < K || (!merge_only && (ldq % 8 || ldq < K)))
        return set_error(VDN_FP8_EINVAL, "requantize_weight: need K, ldw, ldq multiples of 8 and >= K");
    if (!aligned(w, 16) || (wq && !aligned(wq, 8))) return set_error(VDN_FP8_EINVAL, "requantize_weight: misaligned pointer");
    if (lora_a || lora_b) {
        if (!lora_a || !lora_b) return set_error(VDN_FP8_EINVAL, "requantize_weight: lora_a and lora_b go together");
        return launch_lora_requant((const uint16_t*)w, N, K, ldw, (const uint16_t*)lora_a, (const uint16_t*)lora_b,
                                   rank, lora_scale, (uint8_t*)wq, ldq, w_scale, (uint16_t*)w_merged, stream);
    }
    const dim3 grid((unsigned)((N + kWavesPerBlock - 1) / kWavesPerBlock));
    launch_rowquant<true>(pick_cpl(K / 8), grid, stream, (const uint16_t*)w, N, K, ldw, (uint8_t*)wq, ldq, w_scale);
    int st = check_launch("requantize_weight");
    if (st == VDN_FP8_OK && w_merged && w_merged != w) {
        // Without LoRA the "merged" weight is the weight itself.
        if (hipMemcpy2DAsync(w_merged, ldw * 2, w, ldw * 2, K * 2, N, hipMemcpyDeviceToDevice, stream) != hipSuccess)
            return set_error(VDN_FP8_ELAUNCH, "requantize_weight: copy of the merged weight failed");
    }
    return st;
}

// The typed entry points: binary16 and binary32 rows through the kernels above, bf16
// rows through the entry points they extend.
namespace {
// The shared contract of a typed row call: shapes, strides, alignment, the type.
int check_typed_rows(const char* what, const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, int64_t kx,
                     const void* y, int64_t ldy, const float* scale)
{
    if (dtype != VDN_FP8_DTYPE_F16 && dtype != VDN_FP8_DTYPE_F32)
        return set_error(VDN_FP8_EINVAL, "%s: unknown dtype %d", what, dtype);
    if (M < 0 || K < 0) return set_error(VDN_FP8_EINVAL, "%s: negative shape [%lld, %lld]", what, (long long)M, (long long)K);
    if (M > 0 && K == 0) return set_error(VDN_FP8_EINVAL, "%s: K must be positive", what);
    if (M == 0) return VDN_FP8_OK;
    if (!x || !y || !scale) return set_error(VDN_FP8_EINVAL, "%s: null pointer", what);
    if (K % 8 || ldx % 8 || ldy % 8 || ldx < kx || ldy < K)
        return set_error(VDN_FP8_EINVAL, "%s: need K, the row strides multiples of 8, ldx >= %lld and ldy >= K "
                         "(K=%lld ldx=%lld ldy=%lld)", what, (long long)kx, (long long)K, (long long)ldx, (long long)ldy);
    if (!aligned(x, 16) || !aligned(y, 8) || !aligned(scale, 4))
        return set_error(VDN_FP8_EINVAL, "%s: x must be 16-byte and y 8-byte aligned", what);
    return -1;   // go on
}
}  // namespace

extern "C" int vdn_fp8_quantize_rows_typed(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, void* y,
                                           int64_t ldy, float* scale, hipStream_t stream)
{
    if (dtype == VDN_FP8_DTYPE_BF16) return vdn_fp8_quantize_rows(x, M, K, ldx, y, ldy, scale, stream);
    const int st = check_typed_rows("quantize_rows", x, dtype, M, K, ldx, K, y, ldy, scale);
    if (st >= 0) return st;
    const dim3 grid((unsigned)((M + kWavesPerBlock - 1) / kWavesPerBlock)), block(kWavesPerBlock * kLanes);
    if (dtype == VDN_FP8_DTYPE_F32)
        hipLaunchKernelGGL((k_rowquant_float<float, false>), grid, block, 0, stream, (const float*)x, M, K, ldx,
                           (uint8_t*)y, ldy, scale);
    else
        hipLaunchKernelGGL((k_rowquant_float<_Float16, false>), grid, block, 0, stream, (const _Float16*)x, M, K,
                           ldx, (uint8_t*)y, ldy, scale);
    return check_launch("quantize_rows");
}

extern "C" int vdn_fp8_swiglu_quantize_rows_typed(const void* h, int dtype, int64_t M, int64_t K, int64_t ldh,
                                                  void* y, int64_t ldy, float* scale, hipStream_t stream)
{
    if (dtype == VDN_FP8_DTYPE_BF16) return vdn_fp8_swiglu_quantize_rows(h, M, K, ldh, y, ldy, scale, stream);
    const int st = check_typed_rows("swiglu_quantize_rows", h, dtype, M, K, ldh, 2 * K, y, ldy, scale);
    if (st >= 0) return st;
    const dim3 grid((unsigned)((M + kWavesPerBlock - 1) / kWavesPerBlock)), block(kWavesPerBlock * kLanes);
    if (dtype == VDN_FP8_DTYPE_F32)
        hipLaunchKernelGGL((k_swiglu_quant_float<float>), grid, block, 0, stream, (const float*)h, M, K, ldh,
                           (uint8_t*)y, ldy, scale);
    else
        hipLaunchKernelGGL((k_swiglu_quant_float<_Float16>), grid, block, 0, stream, (const _Float16*)h, M, K, ldh,
                           (uint8_t*)y, ldy, scale);
    return check_launch("swiglu_quantize_rows");
}

extern "C" int vdn_fp8_requantize_weight_typed(const void* w, int dtype, int64_t N, int64_t K, int64_t ldw, void* wq,
                                               int64_t ldq, float* w_scale, hipStream_t stream)
{
    if (dtype == VDN_FP8_DTYPE_BF16)
        return vdn_fp8_requantize_weight(w, N, K, ldw, nullptr, nullptr, 0, 0.0f, wq, ldq, w_scale, nullptr, stream);
    const int st = check_typed_rows("requantize_weight", w, dtype, N, K, ldw, K, wq, ldq, w_scale);
    if (st >= 0) return st;
    const dim3 grid((unsigned)((N + kWavesPerBlock - 1) / kWavesPerBlock)), block(kWavesPerBlock * kLanes);
    if (dtype == VDN_FP8_DTYPE_F32)
        hipLaunchKernelGGL((k_rowquant_float<float, true>), grid, block, 0, stream, (const float*)w, N, K, ldw,
                           (uint8_t*)wq, ldq, w_scale);
    else
        hipLaunchKernelGGL((k_rowquant_float<_Float16, true>), grid, block, 0, stream, (const _Float16*)w, N, K, ldw,
                           (uint8_t*)wq, ldq, w_scale);
    return check_launch("requantize_weight");
}
