// QK preparation: per-head RMSNorm followed by rotary embedding, one pass.
//
// For each token t and head h of q (or k) [T, H, d] (bf16):
//   rstd    = 1 / sqrt(sum_i x[i]^2 / d + eps)                        (binary32)
//   n[i]    = (x[i] * rstd) * w[i]                                    (w = 1 if absent)
//   c[i], s[i] = bf16(cos[t][i]), bf16(sin[t][i])                     (i < rotary_dim)
//   r[i]    = -n[i + R/2] if i < R/2, n[i - R/2] if R/2 <= i < R      (R = rotary_dim)
//   out[i]  = bf16(n[i] * c[i] + r[i] * s[i])   for i < R
//   out[i]  = bf16(n[i])                        for i >= R
// The chain stays in binary32 and rounds once at the store, as the compiled
// `_qk_prep` of the reference does (softmax_attention/kernels.py:8-45); the
// cos/sin tables are rounded to bf16 first, as its `cos.to(x.dtype)` does.
//
// Layout: one wave per token, 16-byte chunks (8 elements) with lane L taking
// chunks L, L + 64, ... A head of d elements is d / 8 consecutive chunks, so
// with d in {64, 128, 256} every head sits in one group of d / 8 lanes of one
// sweep: the sum of squares is a butterfly inside the group, and the rotary
// partner of a chunk (R/2 elements away) is R/16 lanes away in the same group.
// Each lane's position inside its head is fixed (64 is a multiple of d / 8),
// so its weight and cos/sin values are loaded once per token.
#include <stdint.h>

#include "vdn_common.h"

namespace vdn {
namespace {

constexpr int kLanes = 64;
constexpr int kWavesPerBlock = 4;   // tokens per workgroup
// Outputs of at least this many bytes are stored non-temporally: beyond what the
// 256 MB last-level cache holds, cached stores only evict each other
// ([32760, 40, 128]: 0.130 ms against 0.142 ms).
constexpr int64_t kNtStoreBytes = 256ll << 20;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct QkArgs {
    const uint16_t* x;
    int64_t T, H, d, ldx;
    const uint16_t* weight;   // [d] or NULL
    float eps;
    const void* cos;          // [T, R] (row stride ldcs), binary32 or bf16; NULL when R == 0
    const void* sin;
    int64_t R, ldcs;
    int cs_bf16;
    uint16_t* out;
    int64_t ldo;
};

// Eight table values for elements i0 .. i0 + 7 of one row, rounded to bf16 and
// returned as binary32, from the 32 bytes at the row's element i0 (binary32
// tables use both halves, bf16 tables the first).
__device__ __forceinline__ void decode_table8(uint4 lo, uint4 hi, bool bf16, float v[8])
{
    if (bf16) {
        const uint32_t w[4] = {lo.x, lo.y, lo.z, lo.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) { v[2 * e] = bf16_lo(w[e]); v[2 * e + 1] = bf16_hi(w[e]); }
    } else {
        const uint32_t raw[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const uint32_t r = pack_bf16x2(__uint_as_float(raw[e]), __uint_as_float(raw[e + 1]));
            v[e] = bf16_lo(r);
            v[e + 1] = bf16_hi(r);
        }
    }
}

// Lane exchanges inside a 16-lane DPP row (d = 128: one head per row), as
// register moves rather than LDS round trips.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xb1;         // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4e;         // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- 7 - i within each half row
constexpr int kDppMirror = 0x140;      // lane i <- 15 - i within each row
constexpr int kDppRor8 = 0x128;        // lane i <- lane (i + 8) mod 16 within each row

// Sum over the 16 lanes of a row, every lane receiving it.
__device__ __forceinline__ float row16_sum(float v)
{
    v += dpp_f32<kDppXor1>(v);
    v += dpp_f32<kDppXor2>(v);
    v += dpp_f32<kDppHalfMirror>(v);
    v += dpp_f32<kDppMirror>(v);
    return v;
}

// G = d / 8 lanes per head; CPL = chunks per lane; NT: non-temporal output stores.
template <int G, int CPL, bool NT, int WPR>
__global__ __launch_bounds__(kWavesPerBlock * kLanes) void k_qk_prep(QkArgs p)
{
    const int lane = threadIdx.x & (kLanes - 1);
    // the token as a uniform value: its row bases live in scalar registers. WPR
    // waves share a token, part w holding chunks [w * 64 CPL, (w + 1) * 64 CPL):
    // whole heads, since 64 is a multiple of G (heads are independent).
    const int64_t unit = (int64_t)blockIdx.x * kWavesPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x / kLanes);
    const int64_t t = unit / WPR;
    if (t >= p.T) return;
    const int base = (int)(unit - t * WPR) * kLanes * CPL;   // first chunk of this wave
    const int nch = (int)(p.H * G);                  // chunks per token
    const int j = lane % G;                           // chunk index inside the head
    const int i0 = 8 * j;                             // first element of this lane's chunks

    // The token's chunks (buffer loads: chunks past the token read zero, no branch).
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.x + t * p.ldx), 0, nch * 16, 0x00020000);
    uint4 v[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c)
        v[c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, (uint32_t)((base + lane + kLanes * c) * 16), 0,
                                                                              kBufferLoadOnce));

    // The weight and the token's cos/sin values, likewise by buffer loads issued
    // with the token's (an absent weight and the elements past the rotary
    // dimension fall outside their descriptors; no branch, so no load waits for
    // another before it is issued).
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.weight ? p.weight : p.x), 0, p.weight ? (int)(p.d * 2) : 0, 0x00020000);
    const uint4 wq = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, (uint32_t)(i0 * 2), 0, 0));
    const int esz = p.cs_bf16 ? 2 : 4;
    const int cbytes = p.R > 0 ? (int)(p.R * esz) : 0;
    const int64_t crow = t * p.ldcs * esz;
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.R > 0 ? static_cast<const uint8_t*>(p.cos) + crow : reinterpret_cast<const uint8_t*>(p.x)), 0, cbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.R > 0 ? static_cast<const uint8_t*>(p.sin) + crow : reinterpret_cast<const uint8_t*>(p.x)), 0, cbytes, 0x00020000);
    const uint32_t coff = (uint32_t)(i0 * esz);
    const uint4 c0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(cr, coff, 0, 0));
    const uint4 c1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(cr, coff + 16, 0, 0));
    const uint4 s0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(sr, coff, 0, 0));
    const uint4 s1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(sr, coff + 16, 0, 0));

    float w[8];
    {
        const uint32_t ww[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            w[2 * e] = p.weight ? bf16_lo(ww[e]) : 1.0f;
            w[2 * e + 1] = p.weight ? bf16_hi(ww[e]) : 1.0f;
        }
    }
    const int half = (int)(p.R / 2);
    const bool rot = i0 < p.R;                        // R % 16 == 0: whole chunks rotate or pass
    const bool first = i0 < half;                     // partner R/2 elements ahead (sign -1)
    const int partner = lane + (first ? half / 8 : -(half / 8));
    const bool full_rot = p.R == p.d;                 // uniform
    float cs[8], sn[8];
    decode_table8(c0, c1, p.cs_bf16, cs);
    decode_table8(s0, s1, p.cs_bf16, sn);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        cs[e] = rot ? cs[e] : 1.0f;
        sn[e] = rot ? sn[e] : 0.0f;
    }

    uint16_t* orow = p.out + t * p.ldo;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int q = base + lane + kLanes * c;
        const uint32_t xw[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
        float x[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) { x[2 * e] = bf16_lo(xw[e]); x[2 * e + 1] = bf16_hi(xw[e]); }
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
        if (G == 16) {
            ss = row16_sum(ss);
        } else {
#pragma unroll
            for (int off = 1; off < G; off <<= 1) ss += __shfl_xor(ss, off, kLanes);
        }
        const float rstd = 1.0f / __builtin_sqrtf(ss / (float)p.d + p.eps);
        float n[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) n[e] = (x[e] * rstd) * w[e];
        // every lane takes part in the exchange (the lanes of pass-through chunks
        // read a value they do not use)
        float o[8];
        if (G == 16 && full_rot) {
            // R = d = 128: the partner chunk is 8 lanes away inside the row
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float pe = dpp_f32<kDppRor8>(n[e]);
                o[e] = n[e] * cs[e] + (first ? -pe : pe) * sn[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float pe = __shfl(n[e], rot ? partner : lane, kLanes);
                const float r = first ? -pe : pe;
                o[e] = rot ? n[e] * cs[e] + r * sn[e] : n[e];
            }
        }
        if (q < nch) {
            const u32x4_t ov = {pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]), pack_bf16x2(o[4], o[5]),
                                pack_bf16x2(o[6], o[7])};
            if (NT) __builtin_nontemporal_store(ov, reinterpret_cast<u32x4_t*>(orow + 8 * q));
            else *reinterpret_cast<u32x4_t*>(orow + 8 * q) = ov;
        }
    }
}

template <int G>
int launch_g(const QkArgs& p, int cpl, hipStream_t stream)
{
    const bool nt = p.T * p.H * p.d * 2 >= kNtStoreBytes;
    const dim3 block(kWavesPerBlock * kLanes);
    if (cpl >= 4) {
        // tokens of at least 4 chunks per lane: two waves per token, whole heads each
        const int64_t nch = p.H * G, per = (nch + 2 * kLanes - 1) / (2 * kLanes);
        const dim3 g2((unsigned)((2 * p.T + kWavesPerBlock - 1) / kWavesPerBlock));
#define VDN_CASE2(n)                                                                        \
        if (per <= n) {                                                                     \
            if (nt) hipLaunchKernelGGL((k_qk_prep<G, n, true, 2>), g2, block, 0, stream, p);  \
            else hipLaunchKernelGGL((k_qk_prep<G, n, false, 2>), g2, block, 0, stream, p);    \
            return check_launch("qk_prep");                                                 \
        }
        VDN_CASE2(2) VDN_CASE2(3) VDN_CASE2(4) VDN_CASE2(5) VDN_CASE2(6) VDN_CASE2(8) VDN_CASE2(10)
        VDN_CASE2(12) VDN_CASE2(16)
#undef VDN_CASE2
    }
    const dim3 grid((unsigned)((p.T + kWavesPerBlock - 1) / kWavesPerBlock));
    switch (cpl) {
#define VDN_CASE(n)                                                                         \
    case n:                                                                                 \
        if (nt) hipLaunchKernelGGL((k_qk_prep<G, n, true, 1>), grid, block, 0, stream, p);  \
        else hipLaunchKernelGGL((k_qk_prep<G, n, false, 1>), grid, block, 0, stream, p);    \
        break;
        VDN_CASE(1) VDN_CASE(2) VDN_CASE(3) VDN_CASE(4) VDN_CASE(6) VDN_CASE(8) VDN_CASE(10)
        VDN_CASE(12) VDN_CASE(16) VDN_CASE(20) VDN_CASE(24) VDN_CASE(28) VDN_CASE(32)
#undef VDN_CASE
        default: return set_error(VDN_FP8_EINVAL, "qk_prep: unsupported H * d");
    }
    return check_launch("qk_prep");
}

}  // namespace
}  // namespace vdn

using namespace vdn;

extern "C" int vdn_fp8_qk_prep(const void* x, int64_t T, int64_t H, int64_t d, int64_t ldx, const void* weight,
                               float eps, const void* cos, const void* sin, int64_t rotary_dim, int64_t ldcs,
                               int cs_bf16, void* out, int64_t ldo, hipStream_t stream)
{
    if (T < 0 || H < 0 || d < 0) return set_error(VDN_FP8_EINVAL, "qk_prep: negative shape");
    if (T == 0 || H == 0) return VDN_FP8_OK;
    if (!x || !out) return set_error(VDN_FP8_EINVAL, "qk_prep: null pointer");
    if (d != 64 && d != 128 && d != 256) return set_error(VDN_FP8_EINVAL, "qk_prep: head dim %lld not in {64, 128, 256}", (long long)d);
    if (rotary_dim < 0 || rotary_dim > d || rotary_dim % 16)
        return set_error(VDN_FP8_EINVAL, "qk_prep: rotary_dim %lld must be a multiple of 16 in [0, d]", (long long)rotary_dim);
    if (rotary_dim > 0 && (!cos || !sin || ldcs < rotary_dim))
        return set_error(VDN_FP8_EINVAL, "qk_prep: rotary tables missing or row stride below rotary_dim");
    if (ldx % 8 || ldo % 8 || ldx < H * d || ldo < H * d)
        return set_error(VDN_FP8_EINVAL, "qk_prep: need ldx, ldo multiples of 8 and >= H * d");
    if (!(eps >= 0.0f)) return set_error(VDN_FP8_EINVAL, "qk_prep: eps must be >= 0");
    const int64_t csal = cs_bf16 ? 8 : 4;
    if (!aligned(x, 16) || !aligned(out, 16) || (weight && !aligned(weight, 16)) ||
        (rotary_dim > 0 && (!aligned(cos, 16) || !aligned(sin, 16) || ldcs % csal)))
        return set_error(VDN_FP8_EINVAL, "qk_prep: misaligned pointer (x, out, weight, cos, sin 16 B; table rows 16 B)");
    const int64_t nch = H * d / 8;
    const int cpl = pick_cpl(nch);
    if (cpl == 0) return set_error(VDN_FP8_EINVAL, "qk_prep: H * d = %lld above the supported 16384", (long long)(H * d));
    QkArgs p{(const uint16_t*)x, T, H, d, ldx, (const uint16_t*)weight, eps, cos, sin, rotary_dim, ldcs, cs_bf16,
             (uint16_t*)out, ldo};
    switch (d) {
        case 64: return launch_g<8>(p, cpl, stream);
        case 128: return launch_g<16>(p, cpl, stream);
        default: return launch_g<32>(p, cpl, stream);
    }
}
