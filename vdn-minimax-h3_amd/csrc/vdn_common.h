// Shared device helpers and host-side error plumbing for the fp8 linear path.
//
// Element formats:
//   bf16  -- stored as uint16_t bit patterns (the high half of a binary32);
//   e4m3  -- OCP float8 e4m3 "fn" (max 448, no infinities, 0x7f/0xff NaN),
//            the format of torch.float8_e4m3fn; stored as uint8_t codes.
// gfx950 converts to and from OCP e4m3 in hardware (v_cvt_pk_fp8_f32,
// round to nearest even).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vdn_fp8.h"

namespace vdn {

// ---------------------------------------------------------------------------
// host: error state (one message per host thread, read by vdn_fp8_last_error)
// ---------------------------------------------------------------------------
int set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* what);

// Compute units of the current device (cached per device); 0 if it cannot be queried.
int device_cus();

// Smallest 16-byte-chunks-per-lane template instance (1..32) that covers a row of
// nch chunks with one wave; 0 above 32 x 64 chunks.
int pick_cpl(int64_t nch);

inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

// ---------------------------------------------------------------------------
// device: bf16 / e4m3 conversions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// Two binary32 values -> two bf16 (round to nearest even), packed lo|hi<<16.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi)
{
    bf16x2_t p = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, p);
}

__device__ __forceinline__ float round_bf16(float v) { return bf16_lo(pack_bf16x2(v, 0.0f)); }

// The same rounding in one conversion: v into the high half, zero into the low half,
// so the word is bf16(v) as binary32 with no unpacking (written as assembly: the
// compiler turns the zero-low form back into a low-half conversion and a permute).
// Its operand must be a VALU result, never an MFMA accumulator read directly (inline
// assembly escapes the compiler's MFMA-to-VALU wait states).
__device__ __forceinline__ float round_bf16_hi(float v)
{
    uint32_t d;
    asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(d) : "v"(v));
    return __builtin_bit_cast(float, d);
}

// GELU(tanh), shared by the GEMM epilogue and the GELU quantizer so that both give the
// same bits: gelu_tanh(v) = 0.5 v (1 + tanh(u)) = v * sigmoid(2u), u = sqrt(2/pi) (v + 0.044715 v^3):
// exp(-2u) = 2^t with t = v (A + B v^2), A = -2 sqrt(2/pi) log2(e), B = 0.044715 A
// (the constants folded so that t costs three operations and exp one).
__device__ __forceinline__ float gelu_tanh(float v)
{
    constexpr float kA = -2.3022082f;            // -1.5957691216057308 * 1.4426950408889634
    constexpr float kB = -0.10294324f;           // kA * 0.044715
    const float t = v * __builtin_fmaf(kB, v * v, kA);
    return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

// 16-byte load of data read exactly once (activations streamed through a
// kernel): non-temporal, so the stream does not displace cached lines that are
// read again (the activation quantizer on [32760, 5120]: 0.080 ms against
// 0.083 ms with plain loads).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_once(const uint4* p)
{
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Cache-policy operand of the raw buffer intrinsics for a read-once load.
constexpr int kBufferLoadOnce = 2;   // nt

// Wait states after a 16-byte store (or a run of them with nothing between), before
// any later instruction can overwrite their data registers. The compiler allows two
// (an s_nop 1 before such a write); in one kernel here (the one-pass LoRA merge, with
// inline-assembly copies nearby) a VALU write of a 16-byte store's first data register
// two instructions after the store changed the stored value for the last four lanes
// of each 16-lane quarter, so every 16-byte store site is followed by eight.
__device__ __forceinline__ void settle_stores()
{
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7");
    __builtin_amdgcn_sched_barrier(0);
}

// One 16-byte buffer store, then settle_stores(). POL: the cache-policy operand.
template <int POL, typename V>
__device__ __forceinline__ void store_b128_settled(V v, __amdgpu_buffer_rsrc_t rs, uint32_t off, int soff)
{
    __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, soff, POL);
    settle_stores();
}

// Four binary32 values -> four e4m3 codes in one dword (byte i = value i).
__device__ __forceinline__ uint32_t pack_e4m3x4(float a, float b, float c, float d)
{
    uint32_t w = 0;
    w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, w, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return w;
}

// Four bf16 values (two packed words, lo|hi<<16 each) -> four e4m3 codes, with
// no unpacking: v_cvt_scalef32_pk_fp8_bf16 at scale 1.0 (round to nearest even).
// For finite inputs of magnitude <= 464 the codes equal pack_e4m3x4 of the same
// values (the conversions differ only beyond that, in overflow handling); the
// callers pass bf16 quotients of magnitude <= 450.
typedef short s16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_e4m3x4_bf16(uint32_t q01, uint32_t q23)
{
    s16x2_t w = {0, 0};
    w = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(w, __builtin_bit_cast(bf16x2_t, q01), 1.0f, false);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(w, __builtin_bit_cast(bf16x2_t, q23), 1.0f, true);
    return __builtin_bit_cast(uint32_t, w);
}

// Packed max of the magnitudes of two bf16 lanes: (bits & 0x7fff) orders the
// same way as |x| for every non-NaN pattern and puts NaN patterns above inf.
__device__ __forceinline__ uint32_t absmax_bf16x2(uint32_t acc, uint32_t w)
{
    u16x2_t a = __builtin_bit_cast(u16x2_t, acc);
    u16x2_t b = __builtin_bit_cast(u16x2_t, w & 0x7fff7fffu);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(a, b));
}

// Lane exchanges inside each row of 16 lanes (DPP, no LDS round trip): xor 1, xor 2,
// the mirror within 8 lanes and the mirror within 16. After the four steps of a
// reduction every lane of a row holds the row's result. The wavefront must be whole.
constexpr int kDppXor1 = 0xb1, kDppXor2 = 0x4e, kDppHalfMirror = 0x141, kDppMirror = 0x140;
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xf, 0xf, false);
}

// Maximum over the 64 lanes of a wavefront, wave-uniform: four DPP steps within the
// rows, then the four row maxima read into scalar registers.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    v = max(v, dpp_u32<kDppXor1>(v));
    v = max(v, dpp_u32<kDppXor2>(v));
    v = max(v, dpp_u32<kDppHalfMirror>(v));
    v = max(v, dpp_u32<kDppMirror>(v));
    const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16),
                   r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
    return max(max(r0, r1), max(r2, r3));
}

// The per-row scale of the reference: max(amax / 448, 1e-12) with IEEE
// binary32 division; NaN propagates (torch's clamp_min keeps NaN).
__device__ __forceinline__ float row_scale(float amax)
{
    float s = amax / 448.0f;
    return (s < 1e-12f) ? 1e-12f : s;
}

// x / s rounded to nearest binary32, from r = RN(1/s): one multiply and two
// fma -- Markstein's correction of a reciprocal-based quotient (P. Markstein,
// "Computation of elementary functions on the IBM RISC System/6000 processor",
// IBM J. Res. Dev. 34(1), 1990): q0 = x r, residual e = x - q0 s (exact by
// fma), q = q0 + e r. The remainder is written -fma(q0, s, -x) so that x = -0
// yields -0.
// Valid for finite, positive s; every (s, x) pair the quantizers can produce
// gives the same e4m3 code as the IEEE quotient (checked exhaustively).
__device__ __forceinline__ float div_by_scale(float x, float s, float r)
{
    float q0 = x * r;
    float e = -__builtin_fmaf(q0, s, -x);
    return __builtin_fmaf(e, r, q0);
}

}  // namespace vdn
