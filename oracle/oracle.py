"""CPU oracle for the fp8 quantized-linear path -- TEST INFRASTRUCTURE ONLY.

Only tests/, `__graft_entry__.smoke()` and the `cpu_baseline` leg of bench.py may
import this module, and only to compare the product's results with it. The product (the `vdn_fp8` package and
its HIP library) never imports it and has no CPU fallback.

Bit-level arithmetic (e4m3 / bf16 rounding, the row and weight quantizers, the LoRA
merge) lives in `fp8_oracle.c` and is reached through ctypes; the dequantized matmul
and the epilogues are numpy. bf16 tensors travel as numpy uint16 bit patterns, e4m3
codes as uint8.

Reference functions restated (paths relative to the reference checkout):
  quantize_rows         src/models/ops/fp8_linear.py:132-135 (quantize_rows_reference)
  swiglu_quantize_rows  src/models/ops/fp8_linear.py:83-99
  quantize_weight       src/models/ops/fp8_linear.py:262-267 (Fp8Linear.__init__, rowwise)
  quantize_rows_float, swiglu_quantize_rows_float, quantize_weight_float
                        the same three for float16 / float32 rows (numpy, binary32 IEEE
                        arithmetic; the e4m3 cast is the C encoder)
  dequant_linear_typed  forward_quantized with a float16 / float32 out_dtype
  lora_merge            src/inference/utils/lora.py:91-92 (merge_lora_state)
  dequant_linear        src/models/ops/fp8_linear.py:270-277 (forward_quantized: the
                        rowwise _scaled_mm then `out + bias`), dequantized in float64,
                        rounded to bf16 at the reference's op boundaries
  gelu_tanh             no reference function (the reference FFN is SwiGLU); the textbook
                        tanh approximation of GELU, pinned against torch's
                        F.gelu(approximate="tanh")
  gelu_quantize_rows    quantize_rows (fp8_linear.py:110-117) of bf16(gelu_tanh(h)): a GELU
                        FFN's down-projection input
  gated / gated_residual  src/models/ops/fused_block.py:47-49 (_post_ref, as the compiled
                        `post` evaluates it: one bf16 rounding)
  norm_quantize_rows    src/models/ops/fused_block.py:41-44 (_pre_ref, as the compiled
                        `pre` evaluates it: binary32-or-better chain, one bf16 rounding),
                        then quantize_rows on the bf16 result
  qk_prep               src/models/softmax_attention/kernels.py:8-45 (_qk_prep: per-head
                        RMSNorm, then the half-split rotary embedding of _rope_body, as
                        the compiled kernel evaluates it: cos/sin rounded to bf16, the
                        rest binary32-or-better, one bf16 rounding at the end)
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

FP8_MAX = 448.0
SCALE_FLOOR = np.float32(1e-12)


def _threads():
    return int(os.environ.get("ORACLE_THREADS", min(16, os.cpu_count() or 1)))


def build():
    """Compile fp8_oracle.c with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        p, i64, f32, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
        L.oracle_quantize_rows.argtypes = [p, i64, i64, i64, p, i64, p, i32]
        L.oracle_swiglu_quantize_rows.argtypes = [p, i64, i64, i64, p, i64, p, i32]
        L.oracle_quantize_weight.argtypes = [p, i64, i64, i64, p, i64, p, i32]
        L.oracle_lora_merge.argtypes = [p, i64, i64, i64, p, p, i64, f32, p, i64, i32]
        L.oracle_e4m3_encode.argtypes = [p, i64, p]
        L.oracle_e4m3_decode.argtypes = [p, i64, p]
        L.oracle_bf16_encode.argtypes = [p, i64, p]
        for name in ("oracle_quantize_rows", "oracle_swiglu_quantize_rows", "oracle_quantize_weight",
                     "oracle_lora_merge", "oracle_e4m3_encode", "oracle_e4m3_decode",
                     "oracle_bf16_encode"):
            getattr(L, name).restype = None
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _u16(a):
    a = np.ascontiguousarray(a)
    if a.dtype != np.uint16:
        raise TypeError(f"expected bf16 bit patterns as uint16, got {a.dtype}")
    return a


# ---------------------------------------------------------------------------------
# element-wise conversions
# ---------------------------------------------------------------------------------

def e4m3_encode(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint8)
    lib().oracle_e4m3_encode(_ptr(x), x.size, _ptr(y))
    return y


def e4m3_decode(c):
    c = np.ascontiguousarray(c, dtype=np.uint8)
    y = np.empty(c.shape, np.float32)
    lib().oracle_e4m3_decode(_ptr(c), c.size, _ptr(y))
    return y


def bf16_encode(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().oracle_bf16_encode(_ptr(x), x.size, _ptr(y))
    return y


def bf16_decode(h):
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------------
# the quantizers and the merge
# ---------------------------------------------------------------------------------

def quantize_rows(x):
    """bf16 bits [M, K] -> (e4m3 codes [M, K], fp32 scale [M])."""
    x = _u16(x)
    M, K = x.shape
    y = np.empty((M, K), np.uint8)
    s = np.empty(M, np.float32)
    lib().oracle_quantize_rows(_ptr(x), M, K, K, _ptr(y), K, _ptr(s), _threads())
    return y, s


def swiglu_quantize_rows(h):
    """bf16 bits [M, 2K] -> (e4m3 codes [M, K], fp32 scale [M])."""
    h = _u16(h)
    M, K2 = h.shape
    if K2 % 2:
        raise ValueError("swiglu input needs an even width")
    K = K2 // 2
    y = np.empty((M, K), np.uint8)
    s = np.empty(M, np.float32)
    lib().oracle_swiglu_quantize_rows(_ptr(h), M, K, K2, _ptr(y), K, _ptr(s), _threads())
    return y, s


def quantize_weight(w):
    """bf16 bits [N, K] -> (e4m3 codes [N, K], fp32 scale [N])."""
    w = _u16(w)
    N, K = w.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty(N, np.float32)
    lib().oracle_quantize_weight(_ptr(w), N, K, K, _ptr(q), K, _ptr(s), _threads())
    return q, s


def _row_scales(xf):
    """max(row absmax / 448, 1e-12) in binary32 with NaN propagating (torch's amax and
    clamp_min); xf binary32 [M, K]."""
    with np.errstate(invalid="ignore"):
        amax = np.abs(xf).max(axis=1)          # NaN anywhere in a row -> NaN
        s = (amax / np.float32(FP8_MAX)).astype(np.float32)
        return np.where(s < SCALE_FLOOR, SCALE_FLOOR, s).astype(np.float32)   # NaN < x is False: NaN stays


def quantize_rows_float(x):
    """float16 / float32 [M, K] -> (e4m3 codes [M, K], fp32 scale [M]): quantize_rows_reference
    (fp8_linear.py:132-135) on other float types -- x.float() / scale in binary32 (IEEE
    division), then the cast. numpy's float32 division is the IEEE one."""
    x = np.ascontiguousarray(x)
    if x.dtype not in (np.float16, np.float32):
        raise TypeError(f"expected float16 or float32 rows, got {x.dtype}")
    xf = x.astype(np.float32)
    s = _row_scales(xf)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        q = (xf / s[:, None]).astype(np.float32)
    return e4m3_encode(q), s


def swiglu_quantize_rows_float(h):
    """float16 / float32 [M, 2K] -> (e4m3 codes [M, K], fp32 scale [M]): the reference's
    SwiGLU quantizer (fp8_linear.py:83-99) on binary32 loads of h; sigmoid as 1 / (1 +
    exp(-g)) in binary32 (numpy's exp: a kernel with another exp is compared within one
    fp8 code, as for the bf16 oracle)."""
    h = np.ascontiguousarray(h)
    if h.dtype not in (np.float16, np.float32):
        raise TypeError(f"expected float16 or float32 rows, got {h.dtype}")
    hf = h.astype(np.float32)
    K = hf.shape[1] // 2
    a, g = hf[:, :K], hf[:, K:]
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        act = (a * g * (np.float32(1.0) / (np.float32(1.0) + np.exp(-g)))).astype(np.float32)
        s = _row_scales(act)
        q = (act / s[:, None]).astype(np.float32)
    return e4m3_encode(q), s


def quantize_weight_float(w):
    """float16 / float32 [N, K] -> (e4m3 codes [N, K], fp32 scale [N]): the rowwise branch
    of Fp8Linear.__init__ (fp8_linear.py:262-267) for those types -- the scale from the
    binary32 row maximum, then weight / scale.to(weight.dtype) in the weight's type (torch
    divides float16 tensors in binary32 and rounds the quotient to float16), then the cast."""
    w = np.ascontiguousarray(w)
    if w.dtype not in (np.float16, np.float32):
        raise TypeError(f"expected float16 or float32 rows, got {w.dtype}")
    wf = w.astype(np.float32)
    s = _row_scales(wf)
    st = s.astype(w.dtype).astype(np.float32)            # scale.to(weight.dtype)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        q = (wf / st[:, None]).astype(np.float32)
        q = q.astype(w.dtype).astype(np.float32)          # the quotient in the weight's type
    return e4m3_encode(q), s


def lora_merge(w, a, b, scale=1.0):
    """bf16 bits: w [N, K], a [r, K], b [N, r] -> merged w' [N, K] (bf16 bits)."""
    w, a, b = _u16(w), _u16(a), _u16(b)
    N, K = w.shape
    r = a.shape[0]
    if a.shape != (r, K) or b.shape != (N, r):
        raise ValueError(f"lora shapes do not match: w {w.shape}, a {a.shape}, b {b.shape}")
    out = np.empty((N, K), np.uint16)
    lib().oracle_lora_merge(_ptr(w), N, K, K, _ptr(a), _ptr(b), r, float(scale), _ptr(out), K,
                            _threads())
    return out


# ---------------------------------------------------------------------------------
# the dequantized matmul and the epilogues
# ---------------------------------------------------------------------------------

def gelu_tanh(v):
    """0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3)))."""
    c = np.sqrt(2.0 / np.pi)
    return 0.5 * v * (1.0 + np.tanh(c * (v + 0.044715 * v * v * v)))


def _bf16_round(v):
    """Round float64 values to bf16 (through binary32, as torch's .to(bfloat16) of a
    float32 tensor does) and return them as float64."""
    return bf16_decode(bf16_encode(np.asarray(v, np.float64).astype(np.float32))).astype(np.float64)


def gelu_quantize_rows(h):
    """bf16 bits [M, K] -> (e4m3 codes [M, K], fp32 scale [M]): each element replaced by
    bf16(gelu_tanh(h)) (the textbook formula in float64, rounded through binary32 as a
    bf16 cast of a float32 result rounds), then quantize_rows."""
    h = _u16(h)
    g = gelu_tanh(bf16_decode(h).astype(np.float64))
    return quantize_rows(bf16_encode(g.astype(np.float32)))


def dequant_linear_typed(qx, sx, qw, sw, bias=None, out_dtype=np.float32):
    """forward_quantized with a float16 / float32 out_dtype (fp8_linear.py:272-276): the
    dequantized matmul in float64, rounded to out_dtype (the scaled GEMM's output), then
    `out + bias` in that type (bias: an array of out_dtype, or None). Returns out_dtype."""
    x = e4m3_decode(qx).astype(np.float64) * np.asarray(sx, np.float32).reshape(-1, 1).astype(np.float64)
    w = e4m3_decode(qw).astype(np.float64) * np.asarray(sw, np.float32).reshape(-1, 1).astype(np.float64)
    out = (x @ w.T).astype(np.float32).astype(out_dtype)
    if bias is not None:
        # torch adds float16 tensors in binary32 and rounds once
        out = (out.astype(np.float32) + np.asarray(bias).astype(np.float32)[None, :]).astype(out_dtype)
    return out


def dequant_linear(qx, sx, qw, sw, bias=None, epilogue="none", gate=None, gate_index=None,
                   residual=None, rounding="reference"):
    """The reference's dequantized matmul, (qx * sx) @ (qw * sw)^T, then bias and the
    epilogue, in float64.

    rounding="reference" rounds to bf16 where the reference's dtype flow does:
      bf16(matmul)                        the rowwise _scaled_mm, out_dtype=bf16 (fp8_linear.py:272-274)
      bf16(out + bias)                    the separate bf16 bias add (fp8_linear.py:275-276)
      bf16(gelu_tanh(out))                F.gelu(approximate="tanh") on that bf16 tensor
      bf16(gate[idx] * out + residual)    the compiled gated residual add, fp32 inside,
                                          one rounding (fused_block.py:47-49,101-110)
    and returns the bf16 values as float64. rounding="none" returns the unrounded
    float64 result.

    qx uint8 [M, K], sx [M]; qw uint8 [N, K], sw [N]; bias bf16 bits [N] or None;
    epilogue "none" | "gelu_tanh" | "gate"; gate bf16 bits [T, N] (or [N]); gate_index
    int [M] rows of the gate table (None -> row 0); residual bf16 bits [M, N] or None."""
    if rounding not in ("reference", "none"):
        raise ValueError(f"unknown rounding {rounding!r}")
    rnd = _bf16_round if rounding == "reference" else (lambda v: v)
    x = e4m3_decode(qx).astype(np.float64) * np.asarray(sx, np.float32).reshape(-1, 1).astype(np.float64)
    w = e4m3_decode(qw).astype(np.float64) * np.asarray(sw, np.float32).reshape(-1, 1).astype(np.float64)
    out = rnd(x @ w.T)
    if bias is not None:
        out = rnd(out + bf16_decode(bias).astype(np.float64)[None, :])
    if epilogue == "gelu_tanh":
        out = rnd(gelu_tanh(out))
    elif epilogue == "gate":
        g = bf16_decode(gate).astype(np.float64)
        if g.ndim == 1:
            g = g[None, :]
        idx = np.zeros(out.shape[0], np.int64) if gate_index is None else np.asarray(gate_index)
        out = out * g[idx]
        if residual is not None:
            out = out + bf16_decode(residual).astype(np.float64)
        out = rnd(out)
    elif epilogue != "none":
        raise ValueError(f"unknown epilogue {epilogue!r}")
    return out


def norm_rows(x, weight=None, eps=1e-6, scale=None, shift=None, indices=None, return_terms=False):
    """RMSNorm + AdaLN affine in float64, rounded once to bf16 (through binary32):
    n = bf16(x * rsqrt(mean(x^2) + eps) * w * (1 + scale[i]) + shift[i]).
    x bf16 bits [M, K]; weight bf16 bits [K] or None; scale/shift bf16 bits [T, K] or
    None; indices [M] (clamped into the table) or None (row 0). Returns bf16 bits, and
    with return_terms also the magnitude of the affine's two terms, |n - shift| + |shift|
    (float64), the scale at which a binary32 evaluation of the chain errs."""
    xv = bf16_decode(_u16(x)).astype(np.float64)
    M, K = xv.shape
    rstd = 1.0 / np.sqrt(np.mean(xv * xv, axis=1, keepdims=True) + float(np.float32(eps)))
    v = xv * rstd
    if weight is not None:
        v = v * bf16_decode(_u16(weight)).astype(np.float64).reshape(1, K)
    if scale is not None:
        sc = bf16_decode(_u16(scale)).astype(np.float64).reshape(-1, K)
        sh = bf16_decode(_u16(shift)).astype(np.float64).reshape(-1, K)
        idx = np.zeros(M, np.int64) if indices is None else np.clip(np.asarray(indices, np.int64), 0, sc.shape[0] - 1)
        v = v * (1.0 + sc[idx])
        terms = np.abs(v) + np.abs(sh[idx])
        v = v + sh[idx]
    else:
        terms = np.abs(v)
    out = bf16_encode(v.astype(np.float32))
    return (out, terms) if return_terms else out


def gated_residual(residual, gate, indices, branch):
    """residual + gate[i] * branch in float64, rounded once to bf16 (through binary32):
    the compiled `post` (fused_block.py:47-49). residual, branch bf16 bits [M, N]; gate
    bf16 bits [T, N] (or [N]); indices [M] (clamped into the table) or None (row 0)."""
    r = bf16_decode(_u16(residual)).astype(np.float64)
    b = bf16_decode(_u16(branch)).astype(np.float64)
    g = bf16_decode(_u16(gate)).astype(np.float64).reshape(-1, r.shape[1])
    idx = np.zeros(r.shape[0], np.int64) if indices is None else np.clip(np.asarray(indices, np.int64), 0, g.shape[0] - 1)
    return bf16_encode((r + g[idx] * b).astype(np.float32))


def norm_quantize_rows(x, weight=None, eps=1e-6, scale=None, shift=None, indices=None):
    """(codes, scales, normed bf16 bits) of the fused pre-norm + quantize_rows."""
    n = norm_rows(x, weight, eps, scale, shift, indices)
    q, s = quantize_rows(n)
    return q, s, n


def qk_prep(x, weight=None, eps=1e-6, cos=None, sin=None, return_terms=False):
    """QK-norm + rope of one projection in float64, rounded once to bf16 (through
    binary32). x bf16 bits [T, H, d]; weight bf16 bits [d] or None; cos/sin [T, R]
    float32 values (rounded to bf16 here, as `cos.to(x.dtype)`) or bf16 bits (uint16),
    or None. Returns bf16 bits [T, H, d], and with return_terms the magnitude of the
    rotation's two products |n c| + |r s| (float64), the scale at which a binary32
    evaluation errs."""
    xv = bf16_decode(_u16(x)).astype(np.float64)
    T, H, d = xv.shape
    rstd = 1.0 / np.sqrt(np.mean(xv * xv, axis=2, keepdims=True) + float(np.float32(eps)))
    n = xv * rstd
    if weight is not None:
        n = n * bf16_decode(_u16(weight)).astype(np.float64).reshape(1, 1, d)
    terms = np.abs(n)
    out = n.copy()
    if cos is not None:
        def table(t):
            t = np.asarray(t)
            bits = t if t.dtype == np.uint16 else bf16_encode(t.astype(np.float32))
            return bf16_decode(bits).astype(np.float64)[:, None, :]
        c, s = table(cos), table(sin)
        R = c.shape[-1]
        h = R // 2
        rot = np.concatenate([-n[..., h:R], n[..., :h]], axis=-1)
        out[..., :R] = n[..., :R] * c + rot * s
        terms[..., :R] = np.abs(n[..., :R] * c) + np.abs(rot * s)
    out = bf16_encode(out.astype(np.float32))
    return (out, terms) if return_terms else out


def rel_l2(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def max_abs(got, want):
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))))
