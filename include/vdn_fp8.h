/*
 * vdn_fp8.h -- C ABI of the MI355X (gfx950) fp8 quantized-linear library,
 * libvdnfp8.so.
 *
 * This is the drop-in boundary for the fp8 linear path of the VDN-H3 DiT
 * blocks. The reference reaches the same arithmetic from Python through
 * Triton kernels and torch._scaled_mm (src/models/ops/fp8_linear.py); each
 * entry point below names the reference interface it replaces. The Python
 * package vdn_fp8 binds these symbols with ctypes and keeps the reference's
 * module API on top of them.
 *
 * Conventions
 *   - Plain pointers to device memory (HBM) and sizes; no framework types.
 *   - bf16 tensors are uint16 bit patterns; e4m3 tensors are OCP float8
 *     e4m3 "fn" codes (torch.float8_e4m3fn: max 448, 0x7f/0xff NaN).
 *   - Matrices are row-major with an explicit leading dimension in ELEMENTS.
 *   - Every call is asynchronous on `stream` (NULL = the null stream) and
 *     neither allocates nor frees device memory; the caller owns all buffers.
 *   - Return 0 on success. A nonzero status leaves nothing launched, and
 *     vdn_fp8_last_error() returns the message (per host thread). Calls are
 *     re-entrant. The library's only mutable state is that message and a
 *     per-device cache of the compute-unit count (an atomic per device; only
 *     a successful query is kept, a failed one is retried by the next call).
 *   - Scales: x_scale / w_scale are binary32, one per row of X / W.
 *   - Table indices (gate_index, mod_index) outside the table are clamped into
 *     it; the reference's index_select raises on them instead (a deliberate
 *     difference: the kernels read the index with the row's data and never
 *     fault or report; check the range on the host if an error is wanted).
 */
#ifndef VDN_FP8_H
#define VDN_FP8_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VDN_FP8_ABI_VERSION 5

/* status codes */
#define VDN_FP8_OK 0
#define VDN_FP8_EINVAL 1   /* a contract violation: shape, alignment, null */
#define VDN_FP8_ELAUNCH 2  /* the HIP runtime refused the launch */

/* GEMM epilogues, applied to v = bf16(bf16(x_scale[m] * w_scale[n] * acc[m][n]) + bias[n]) */
#define VDN_FP8_EPI_NONE 0      /* out = v */
#define VDN_FP8_EPI_GELU_TANH 1 /* out = 0.5 v (1 + tanh(sqrt(2/pi)(v + 0.044715 v^3))) */
#define VDN_FP8_EPI_GATE 2      /* out = gate[gate_index[m]][n] * v (+ residual[m][n]) */
#define VDN_FP8_EPI_F32 3       /* out = x_scale[m] * w_scale[n] * acc, binary32 (no bias): the
                                   scaled GEMM of a model that does not run in bf16 */

/* Element types of the typed entry points (..._typed). */
#define VDN_FP8_DTYPE_BF16 0
#define VDN_FP8_DTYPE_F16 1
#define VDN_FP8_DTYPE_F32 2

/*
 * Per-token activation quantization: for each row m of x (bf16 [M, K]),
 *   scale[m] = max(max_k |x[m][k]| / 448, 1e-12)        (binary32)
 *   y[m][k]  = e4m3(x[m][k] / scale[m])                  (round to nearest even)
 * bit-exact with the reference's eager spelling.
 * Replaces: quantize_rows / _quantize_rows_kernel, src/models/ops/fp8_linear.py:110-117
 *           and :66-80 (contract: quantize_rows_reference, :132-135).
 * Requires: K % 8 == 0, ldx % 8 == 0, ldy % 8 == 0, x 16-byte and y 8-byte aligned.
 */
int vdn_fp8_quantize_rows(const void *x, int64_t M, int64_t K, int64_t ldx,
                          void *y, int64_t ldy, float *scale, hipStream_t stream);

/*
 * Fused GELU(tanh) + per-token quantization of h (bf16 [M, K], the FFN-up
 * projection's bf16 output before its activation): each element replaced by
 * bf16(gelu_tanh(h)) -- the same function, on the same bf16 value, as the GEMM's
 * VDN_FP8_EPI_GELU_TANH epilogue, so the codes are bit for bit those of that
 * epilogue's output passed to vdn_fp8_quantize_rows -- then the quantize_rows
 * arithmetic on those values (y e4m3 [M, K], scale [M]).
 * Replaces: quantize_rows (src/models/ops/fp8_linear.py:110-117) of a GELU(tanh) FFN's
 *           down-projection input, with the activation folded in (the reference's FFN is
 *           SwiGLU; a GELU FFN is the benchmark DiT block's).
 * Requires: K % 8 == 0, K <= 16384, ldh % 8 == 0, ldy % 8 == 0, h 16-byte and y 8-byte
 *           aligned.
 */
int vdn_fp8_gelu_quantize_rows(const void *h, int64_t M, int64_t K, int64_t ldh,
                               void *y, int64_t ldy, float *scale, hipStream_t stream);

/*
 * Fused SwiGLU + per-token quantization of h (bf16 [M, 2K], value half first,
 * gate half second): act = a * g * sigmoid(g) in binary32, never rounded to
 * bf16, then the quantize_rows arithmetic on act (y e4m3 [M, K], scale [M]).
 * Replaces: swiglu_quantize / _swiglu_quantize_kernel,
 *           src/models/ops/fp8_linear.py:120-129 and :83-99.
 * Requires: K % 8 == 0, ldh % 8 == 0, ldy % 8 == 0.
 */
int vdn_fp8_swiglu_quantize_rows(const void *h, int64_t M, int64_t K, int64_t ldh,
                                 void *y, int64_t ldy, float *scale, hipStream_t stream);

/*
 * Pre-norm of a DiT block fused with the per-token quantization of its output:
 *   rstd   = 1 / sqrt(sum_k x[m][k]^2 / K + eps)                     (binary32)
 *   n[m][k] = bf16(((x[m][k] * rstd) * weight[k]) * (1 + scale[i][k]) + shift[i][k])
 *   y, y_scale = the quantize_rows arithmetic on n               (codes exact given n)
 * with i = mod_index[m] clamped into [0, mod_rows) (row 0 when mod_index is
 * NULL). The chain runs in binary32 with one rounding at the end, as the
 * compiled `pre` of the reference does. weight may be NULL (no weight); the
 * modulation (mod_scale, mod_shift: bf16 [mod_rows, K], row stride ldmod) may
 * be NULL (plain RMSNorm). normed, if not NULL, receives n (bf16 [M, K], row
 * stride ldn). x bf16 [M, K] (row stride ldx); y e4m3 [M, K]; y_scale fp32 [M].
 * y and y_scale may both be NULL when normed is not: the call is then the
 * pre-norm alone (the compiled `pre`, for a consumer that is not an fp8 linear).
 * Replaces: _pre_ref / the compiled `pre` followed by quantize_rows,
 *           src/models/ops/fused_block.py:41-44,101-108 and
 *           src/models/ops/fp8_linear.py:110-117.
 * Requires: K % 8 == 0, K <= 16384, ldx, ldy, ldn, ldmod multiples of 8 and
 *           >= K; x, weight, mod_scale, mod_shift, normed 16-byte aligned; y 8-byte.
 */
int vdn_fp8_norm_quantize_rows(const void *x, int64_t M, int64_t K, int64_t ldx,
                               const void *weight, float eps, const void *mod_scale,
                               const void *mod_shift, int64_t ldmod, const int32_t *mod_index,
                               int64_t mod_rows, void *y, int64_t ldy, float *y_scale,
                               void *normed, int64_t ldn, hipStream_t stream);

/*
 * Rowwise weight quantization, optionally after a fused LoRA merge.
 *   W' = W                                        if lora_a == NULL
 *   W' = bf16(W + bf16(lora_scale * (B @ A)))     otherwise (fp32 accumulate)
 *   w_scale[n] = max(max_k |W'[n][k]| / 448, 1e-12)          (binary32, stored)
 *   wq[n][k]   = e4m3(bf16(W'[n][k] / bf16(w_scale[n])))     (two roundings)
 * w bf16 [N, K] (row stride ldw); lora_a bf16 [rank, K] and lora_b bf16
 * [N, rank], both contiguous; wq e4m3 [N, K] (row stride ldq). If w_merged is
 * not NULL, W' is also written there (bf16 [N, K], row stride ldw; it may
 * alias w -- the reference's in-place merge). With LoRA, wq and w_scale may
 * both be NULL: the call is then the merge alone (merge_lora_state).
 * Replaces: the rowwise branch of Fp8Linear.__init__,
 *           src/models/ops/fp8_linear.py:262-267, preceded by the update of
 *           merge_lora_state, src/inference/utils/lora.py:80-94.
 * Requires: K % 8 == 0, ldw % 8 == 0, ldq % 8 == 0; with LoRA: 1 <= rank <= 128,
 *           K % 16 == 0, lora_a 16-byte aligned, w_merged 8-byte aligned. With
 *           LoRA and codes, w_scale holds the row maxima between the kernels of
 *           the call (it is the only scratch the call needs).
 */
int vdn_fp8_requantize_weight(const void *w, int64_t N, int64_t K, int64_t ldw,
                              const void *lora_a, const void *lora_b, int64_t rank,
                              float lora_scale, void *wq, int64_t ldq, float *w_scale,
                              void *w_merged, hipStream_t stream);

/*
 * The quantizers for rows of another float type (dtype: VDN_FP8_DTYPE_F16 or
 * VDN_FP8_DTYPE_F32; VDN_FP8_DTYPE_BF16 forwards to the bf16 entry points above).
 * The reference's kernels load any float type and compute in binary32; its weight
 * branch divides in the weight's own type:
 *   quantize_rows_typed          as vdn_fp8_quantize_rows on the binary32 values of x
 *   swiglu_quantize_rows_typed   as vdn_fp8_swiglu_quantize_rows on those of h
 *   requantize_weight_typed      w_scale[n] = max(max_k |w[n][k]| / 448, 1e-12),
 *                                wq[n][k] = e4m3(T(w[n][k] / T(w_scale[n])))  (T: w's type)
 * Codes follow torch's non-saturating cast: a quotient above 464 in magnitude
 * (possible for binary16 weights, whose T(scale) can round far below the scale)
 * is NaN. No LoRA here: a merge into such a weight is the reference's own update
 * on the host side, followed by this call.
 * Replaces: quantize_rows / swiglu_quantize, src/models/ops/fp8_linear.py:66-129
 *           (binary16 / binary32 inputs), and the rowwise branch of
 *           Fp8Linear.__init__, :262-267, for binary16 / binary32 weights.
 * Requires: K % 8 == 0; row strides multiples of 8 (elements), ldx (ldh) >= K (2K),
 *           ldy >= K; x (h, w) 16-byte and y (wq) 8-byte aligned.
 */
int vdn_fp8_quantize_rows_typed(const void *x, int dtype, int64_t M, int64_t K, int64_t ldx,
                                void *y, int64_t ldy, float *scale, hipStream_t stream);
int vdn_fp8_swiglu_quantize_rows_typed(const void *h, int dtype, int64_t M, int64_t K,
                                       int64_t ldh, void *y, int64_t ldy, float *scale,
                                       hipStream_t stream);
int vdn_fp8_requantize_weight_typed(const void *w, int dtype, int64_t N, int64_t K, int64_t ldw,
                                    void *wq, int64_t ldq, float *w_scale, hipStream_t stream);

/*
 * fp8 x fp8 GEMM with per-token x per-output-channel dequantization and a
 * fused epilogue:
 *   acc[m][n] = sum_k xq[m][k] * wq[n][k]                 (fp32 accumulate)
 *   v         = bf16(x_scale[m] * w_scale[n] * acc[m][n])
 *   v         = bf16(v + bias[n])                          (bias optional)
 *   out[m][n] = bf16(epilogue(v))                          (fp32 inside)
 * The bf16 roundings sit where the reference's op sequence has them: the
 * scaled GEMM's bf16 output, the bf16 bias add, the epilogue on that tensor.
 * xq e4m3 [M, K] (row stride ldx), wq e4m3 [N, K] (row stride ldw) -- both
 * K-contiguous, the layout of torch._scaled_mm(x_fp8, weight_fp8.t()).
 * bias bf16 [N] or NULL. For VDN_FP8_EPI_GATE: gate bf16 [gate_rows, N] (row
 * stride ldgate), gate_index int32 [M] (NULL = row 0 for every m; an index
 * outside [0, gate_rows) is clamped into it), residual bf16 [M, N] (row stride
 * ldres) or NULL. out bf16 [M, N] (row stride ldo). A per-row gate or a
 * residual on 16-byte aligned rows applies in the GEMM's epilogue; on other
 * rows, or rows whose byte offsets within 256 rows exceed 31 bits, the call
 * runs two kernels on the stream (the GEMM writing v, then the gated residual
 * add in place on out). The result is the same.
 * Replaces: Fp8Linear.forward_quantized, src/models/ops/fp8_linear.py:270-277
 *           (torch._scaled_mm rowwise + bias add); the GELU epilogue has no
 *           reference function; the gate epilogue replaces _post_ref /
 *           the compiled `post`, src/models/ops/fused_block.py:47-49,101-110.
 * VDN_FP8_EPI_F32 writes the binary32 x_scale[m] * w_scale[n] * acc[m][n] to
 * out (float [M, N], row stride ldo in floats, 16-byte aligned) with bias, gate
 * and residual NULL: the reference's _scaled_mm with out_dtype binary32 (the
 * caller rounds to binary16 and adds the bias for the other types, as the
 * reference does).
 * Requires: K % 16 == 0; ldx, ldw % 16 == 0; ldo, ldres, ldgate % 4 == 0;
 *           xq, wq, x_scale, w_scale, bias, gate_index 16-byte aligned;
 *           out, residual, gate 8-byte aligned.
 */
int vdn_fp8_gemm(const void *xq, const float *x_scale, const void *wq, const float *w_scale,
                 int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                 const void *bias, int epilogue, const void *gate, const int32_t *gate_index,
                 int64_t gate_rows, int64_t ldgate, const void *residual, int64_t ldres,
                 void *out, int64_t ldo, hipStream_t stream);

/*
 * Bytes of workspace vdn_fp8_gemm_ws takes for an [M, N, K] GEMM on the current
 * device (0: the shape does not split). Only rows of K >= 8192 split: when the
 * 256 x 256 output tiles leave a last round of at most half the compute units,
 * those tiles run as several K slices whose binary32 partial sums go to the
 * workspace (256 KiB per slice), then a reduction kernel sums them, slice by
 * slice, and applies the epilogue.
 * Replaces: nothing in the reference (torch._scaled_mm sizes its own workspace,
 *           src/models/ops/fp8_linear.py:272); the query for the next call.
 */
int vdn_fp8_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int64_t *bytes);

/*
 * vdn_fp8_gemm with a caller-provided split-K workspace (device memory, 16-byte
 * aligned, at least vdn_fp8_gemm_workspace_size bytes; NULL: no split, the same
 * call as vdn_fp8_gemm). The summation order of an output depends only on K,
 * its tile's position and the split, so a shape gives the same bits call after
 * call; a split shape's last-round tiles sum their K slices in binary32 after
 * the matrix cores, so their bits can differ from vdn_fp8_gemm's by a rounding.
 * Replaces: Fp8Linear.forward_quantized, src/models/ops/fp8_linear.py:270-277,
 *           as vdn_fp8_gemm does.
 * Requires: as vdn_fp8_gemm; workspace_bytes >= the size query's answer.
 */
int vdn_fp8_gemm_ws(const void *xq, const float *x_scale, const void *wq, const float *w_scale,
                    int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                    const void *bias, int epilogue, const void *gate, const int32_t *gate_index,
                    int64_t gate_rows, int64_t ldgate, const void *residual, int64_t ldres,
                    void *out, int64_t ldo, void *workspace, int64_t workspace_bytes,
                    hipStream_t stream);

/*
 * vdn_fp8_gemm_ws without the workspace argument and without allocating: a split
 * shape uses a static 64 MiB device array of the library instead (one per GPU,
 * held until the process ends; its address is looked up on the first call on
 * each device). Same kernels, same bits as vdn_fp8_gemm_ws. Shapes whose split
 * workspace would exceed 64 MiB are refused (EINVAL); on a 256-CU part none
 * does. Every call on one GPU shares that array and nothing in it needs to start
 * at zero (each split fully writes its partial sums before they are read), but
 * two calls that overlap on one GPU (different streams) race on it.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.
 * Requires: as vdn_fp8_gemm.
 */
int vdn_fp8_gemm_noalloc(const void *xq, const float *x_scale, const void *wq, const float *w_scale,
                         int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                         const void *bias, int epilogue, const void *gate, const int32_t *gate_index,
                         int64_t gate_rows, int64_t ldgate, const void *residual, int64_t ldres,
                         void *out, int64_t ldo, hipStream_t stream);

/*
 * QK preparation between the q (or k) projection and attention: per-head
 * RMSNorm, then rotary embedding, in one pass.
 *   rstd   = 1 / sqrt(sum_i x[t][h][i]^2 / d + eps)                (binary32)
 *   n[i]   = (x[t][h][i] * rstd) * weight[i]            (weight NULL: no factor)
 *   c, s   = bf16(cos[t][i]), bf16(sin[t][i])           (i < rotary_dim = R)
 *   out[t][h][i] = bf16(n[i] c[i] - n[i + R/2] s[i])    for i < R/2
 *                = bf16(n[i] c[i] + n[i - R/2] s[i])    for R/2 <= i < R
 *                = bf16(n[i])                           for i >= R
 * binary32 throughout with one rounding at the store, as the compiled kernel
 * of the reference (not bitwise with its eager chain, which rounds per op).
 * x bf16 [T, H, d] (token row stride ldx, heads contiguous), out bf16 likewise
 * (row stride ldo); weight bf16 [d] or NULL; cos, sin [T, R] (row stride ldcs),
 * binary32 (cs_bf16 = 0) or bf16 (cs_bf16 = 1); R = 0 means no rotation (cos
 * and sin may then be NULL).
 * Replaces: _qk_prep / _qk_prep_body and _rope_body,
 *           src/models/softmax_attention/kernels.py:8-45, as called from
 *           HybridAttention._qkv, src/models/hybrid_attention.py:128-130.
 * Requires: d in {64, 128, 256}; H * d <= 16384; R % 16 == 0 and R <= d;
 *           ldx, ldo multiples of 8 and >= H * d; x, out, weight, cos, sin
 *           16-byte aligned and table rows 16-byte multiples.
 */
int vdn_fp8_qk_prep(const void *x, int64_t T, int64_t H, int64_t d, int64_t ldx,
                    const void *weight, float eps, const void *cos, const void *sin,
                    int64_t rotary_dim, int64_t ldcs, int cs_bf16, void *out, int64_t ldo,
                    hipStream_t stream);

/*
 * The block's gated residual add:
 *   out[m][n] = bf16(residual[m][n] + gate[i][n] * branch[m][n])    (binary32 inside)
 * with i = gate_index[m] clamped into [0, gate_rows) (row 0 when gate_index is
 * NULL). residual, branch, out bf16 [M, N] (row strides ldr, ldb, ldo; out may
 * alias residual or branch); residual may be NULL (out = bf16(gate[i][n] *
 * branch[m][n])); gate bf16 [gate_rows, N] (row stride ldgate). The same
 * arithmetic as the GEMM's gate epilogue, for a branch that does not end in
 * one of this library's GEMMs.
 * Replaces: _post_ref / the compiled `post`, src/models/ops/fused_block.py:47-49,
 *           as fast_block_forward applies it (fused_block.py:101-110).
 * Requires: N and the row strides multiples of 8; residual, gate, branch, out
 *           16-byte aligned; gate_index 4-byte aligned.
 */
int vdn_fp8_gated_residual(const void *residual, int64_t ldr, const void *gate, int64_t ldgate,
                           const int32_t *gate_index, int64_t gate_rows, const void *branch,
                           int64_t ldb, void *out, int64_t ldo, int64_t M, int64_t N,
                           hipStream_t stream);

/* The message of the last failed call on this host thread ("" if none). */
const char *vdn_fp8_last_error(void);

/* VDN_FP8_ABI_VERSION of the loaded library. */
int vdn_fp8_abi_version(void);

/*
 * The sources the library was built from, as a JSON object: {"sources": {file:
 * sha256}, "flags": sha256, "digest": sha256}. A loader compares it with the
 * sources it ships beside the library and refuses a stale build. No
 * counterpart in the reference (which compiles its Triton kernels at run time).
 */
const char *vdn_fp8_build_info(void);

#ifdef __cplusplus
}
#endif

#endif /* VDN_FP8_H */
