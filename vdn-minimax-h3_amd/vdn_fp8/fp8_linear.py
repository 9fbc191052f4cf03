"""fp8 e4m3 Linears for the DiT blocks, on MI355X (gfx950) -- a drop-in for the
reference module `src.models.ops.fp8_linear` (src/models/ops/fp8_linear.py).

Same names, signatures, buffers and error behaviour as the reference; every kernel is
hand-written HIP in libvdnfp8.so (include/vdn_fp8.h), reached through ctypes on torch's
current HIP stream. There is no CPU path: like the reference's Triton quantizer, the
operators refuse CPU tensors with ValueError.

What runs where (reference -> here):
  _quantize_rows_kernel (Triton)        -> vdn_fp8_quantize_rows (one HBM read per row)
  _swiglu_quantize_kernel (Triton)      -> vdn_fp8_swiglu_quantize_rows
  Fp8Linear.__init__ eager weight quant -> vdn_fp8_requantize_weight (+ fused LoRA merge)
  torch._scaled_mm + `out + bias`       -> vdn_fp8_gemm (MFMA fp8, scales/bias/epilogue fused)

Scale granularity. The reference picks per-tensor scales on sm100 and rowwise
(per-token x per-channel) elsewhere (fp8_linear.py:141-147). gfx950 reports compute
capability 9.5, so `per_tensor_gemm()` is False here and the rowwise path is the one
implemented; the per-tensor family (quantize_tensor & co.) is not part of this module.

Float types: as the reference, the quantizers take bf16, float16 or float32 rows (computed
in binary32), Fp8Linear takes a Linear of any of the three (the weight's quotient in its own
type), and `forward` returns the rows' type (vdn_fp8_*_typed and the GEMM's binary32
output; the float16 cast and the bias add then follow as the reference's own ops).

Extensions (keyword-only, additive): `Fp8Linear.forward_quantized` and `forward` take an
`epilogue` ("gelu_tanh" or "gate") with `gate`, `gate_index` and `residual`, fused into
the GEMM; `Fp8Linear(linear, lora=(A, B, scale))` quantizes W + scale * B @ A in one
kernel without writing the merged bf16 weight.
"""
import ctypes
import os

import torch
import torch.nn as nn

from . import _lib

FP8_DTYPE = torch.float8_e4m3fn
_FP8_MAX = torch.finfo(FP8_DTYPE).max
MIN_WIDTH = 4096
SKIP_END_BLOCKS = 4

_EPILOGUES = {None: _lib.EPI_NONE, "none": _lib.EPI_NONE, "gelu_tanh": _lib.EPI_GELU_TANH,
              "gate": _lib.EPI_GATE}


def _stream(t):
    return ctypes_stream(t.device)


def ctypes_stream(device):
    """torch's current HIP stream on `device`, as the raw handle the C ABI takes."""
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _aligned16(t):
    """t itself when its data starts on a 16-byte boundary (the GEMM reads its
    vectors 16 bytes at a time), else a fresh copy, which the allocator aligns."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


# Element types the quantizers and the GEMM's output take, with their C ABI codes. The
# reference's Triton kernels load any float type and compute in binary32 (fp8_linear.py:72);
# float64 is refused here (its rows would be rounded to binary32 first).
_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16, torch.float32: _lib.DTYPE_F32}


def _rows(x, dtypes=(torch.bfloat16,)):
    """The reference's input check (fp8_linear.py:102-107): GPU, 2-D, then contiguous;
    and an element type among `dtypes`."""
    if not x.is_cuda:
        raise ValueError("the fp8 quantiser is a HIP kernel; the input must be on the GPU")
    if x.dim() != 2:
        raise ValueError(f"expected [M, K], got {tuple(x.shape)}")
    if x.dtype not in dtypes:
        names = ", ".join(str(d).replace("torch.", "") for d in dtypes)
        raise ValueError(f"the fp8 quantiser takes {names} input, got {x.dtype}")
    return x.contiguous()


_WS_BYTES = {}


def gemm_workspace_bytes(M, N, K, device):
    """Bytes of split-K workspace the GEMM of [M, N, K] takes on `device` (0 for most
    shapes: only long rows, K >= 8192, whose tiles leave a last round of at most half the
    compute units split it). The C side allocates nothing: torch provides the buffer."""
    key = (device.index, M, N, K)
    if key not in _WS_BYTES:
        out = ctypes.c_int64(0)
        _lib.check(_lib.load().vdn_fp8_gemm_workspace_size(M, N, K, ctypes.byref(out)), "gemm_workspace_size")
        _WS_BYTES[key] = out.value
    return _WS_BYTES[key]


_CHECK_INDICES = os.environ.get("VDN_FP8_CHECK_INDICES", "") not in ("", "0")


def set_index_checks(enabled):
    """Table indices outside [0, rows) (the gate table of the GEMM's gate epilogue and of
    `post`, the modulation tables of the pre-norm) are clamped into the table by the
    kernels, where the reference's index_select raises. With checks enabled (or
    VDN_FP8_CHECK_INDICES=1 in the environment) every such call first checks the range on
    the device -- a reduction and a host synchronization per call -- and raises IndexError
    as index_select does. Returns the previous setting."""
    global _CHECK_INDICES
    prev, _CHECK_INDICES = _CHECK_INDICES, bool(enabled)
    return prev


def check_index_range(indices, rows, what):
    """Raises IndexError if `indices` (a tensor) holds a value outside [0, rows) and index
    checks are enabled (set_index_checks); a no-op otherwise."""
    if not _CHECK_INDICES or indices is None or indices.numel() == 0:
        return
    lo, hi = int(indices.min()), int(indices.max())
    if lo < 0 or hi >= rows:
        raise IndexError(f"{what}: index out of range in self (indices span [{lo}, {hi}], the table has "
                         f"{rows} rows)")


def quantize_rows(x):
    """Per-token quantization: each row of the [M, K] input (bf16, float16 or float32) is
    divided by its own scale max(row absmax / 448, 1e-12), in binary32, and cast to e4m3.
    Returns the codes [M, K] and the binary32 scales [M, 1].

    Codes and scales are bit-identical to `quantize_rows_reference` (the reference's
    eager spelling, fp8_linear.py:132-135). Replaces fp8_linear.py:110-117."""
    x = _rows(x, tuple(_DTYPES))
    M, K = x.shape
    y = torch.empty_like(x, dtype=FP8_DTYPE)
    scale = torch.empty(M, 1, device=x.device, dtype=torch.float32)
    lib = _lib.load()
    if x.dtype == torch.bfloat16:
        st = lib.vdn_fp8_quantize_rows(_ptr(x), M, K, K, _ptr(y), K, _ptr(scale), _stream(x))
    else:
        st = lib.vdn_fp8_quantize_rows_typed(_ptr(x), _DTYPES[x.dtype], M, K, K, _ptr(y), K, _ptr(scale), _stream(x))
    _lib.check(st, "quantize_rows")
    return y, scale


def swiglu_quantize(h):
    """SwiGLU and per-token quantization in one kernel. h is the FFN projection's bf16
    output [M, 2K]: its first K columns are the value a, its last K the gate g. The
    activation a * g * sigmoid(g) stays binary32 (it is never stored as bf16) and is
    quantized row by row as in `quantize_rows`; returns e4m3 [M, K] and scales [M, 1].
    h may also be float16 or float32 (computed in binary32, as the reference's kernel
    loads it). Replaces fp8_linear.py:120-129."""
    h = _rows(h, tuple(_DTYPES))
    M, K2 = h.shape
    if K2 % 2:
        raise ValueError(f"swiglu_quantize needs an even width, got {K2}")
    K = K2 // 2
    y = torch.empty(M, K, device=h.device, dtype=FP8_DTYPE)
    scale = torch.empty(M, 1, device=h.device, dtype=torch.float32)
    lib = _lib.load()
    if h.dtype == torch.bfloat16:
        st = lib.vdn_fp8_swiglu_quantize_rows(_ptr(h), M, K, K2, _ptr(y), K, _ptr(scale), _stream(h))
    else:
        st = lib.vdn_fp8_swiglu_quantize_rows_typed(_ptr(h), _DTYPES[h.dtype], M, K, K2, _ptr(y), K, _ptr(scale),
                                                   _stream(h))
    _lib.check(st, "swiglu_quantize")
    return y, scale


def gelu_quantize(h):
    """GELU(tanh) and per-token quantization in one kernel. h is a GELU FFN's up-projection
    output before its activation, bf16 [M, K] (K <= 16384): each element becomes
    bf16(gelu_tanh(h)) -- the GEMM's "gelu_tanh" epilogue on the same bf16 value, so the
    codes are bit for bit quantize_rows(forward_quantized(..., epilogue="gelu_tanh")) --
    and the rows are quantized as in `quantize_rows`; returns e4m3 [M, K] and scales
    [M, 1]. The activation costs less here, where the row quantizer is bound by HBM, than
    in the GEMM's epilogue, where the matrix cores wait for it. The reference's FFN is
    SwiGLU (see `swiglu_quantize`); this serves a GELU FFN's down projection, whose
    quantize_rows it replaces (fp8_linear.py:110-117)."""
    h = _rows(h)
    M, K = h.shape
    y = torch.empty(M, K, device=h.device, dtype=FP8_DTYPE)
    scale = torch.empty(M, 1, device=h.device, dtype=torch.float32)
    _lib.check(_lib.load().vdn_fp8_gelu_quantize_rows(_ptr(h), M, K, h.stride(0), _ptr(y), K, _ptr(scale), _stream(h)),
               "gelu_quantize")
    return y, scale


def quantize_rows_reference(x):
    """The eager spelling of `quantize_rows` (fp8_linear.py:132-135), kept for API
    compatibility: plain torch ops, the contract the HIP kernel is bit-exact with.
    Never called by the fp8 path itself."""
    scale = (x.float().abs().amax(dim=1, keepdim=True) / _FP8_MAX).clamp_min(1e-12)
    return (x.float() / scale).to(FP8_DTYPE), scale


_PER_TENSOR = None


def per_tensor_gemm():
    """True only on compute capability >= 10 (sm100), as in the reference
    (fp8_linear.py:141-147). gfx950 reports 9.5: rowwise scales."""
    global _PER_TENSOR
    if _PER_TENSOR is None:
        _PER_TENSOR = (torch.cuda.is_available()
                       and torch.cuda.get_device_capability(0)[0] >= 10)
    return _PER_TENSOR


def _rowwise_only():
    if per_tensor_gemm():
        raise NotImplementedError("per-tensor fp8 scales (the sm100 branch) are not part of the "
                                  "gfx950 build; this device should report capability 9.x")


def quantize_activation(x):
    """What the GEMM callers use (fp8_linear.py:233-236): rowwise on gfx950."""
    _rowwise_only()
    return quantize_rows(x)


def swiglu_quantize_activation(h):
    """fp8_linear.py:239-240: rowwise on gfx950."""
    _rowwise_only()
    return swiglu_quantize(h)


def requantize_weight(weight, lora=None, merged_out=None):
    """weight [N, K] -> (fp8 codes [N, K], fp32 scale [N]) with the rowwise arithmetic of
    Fp8Linear.__init__ (fp8_linear.py:262-267): the quotient in the weight's own type
    (bf16, float16 or float32), then the cast.

    lora = (A [r, K], B [N, r], scale) folds W + bf16(scale * B @ A) in first, as
    merge_lora_state does (lora.py:91-92): with bf16 factors of rank <= 128 inside the same
    kernel; other adapters (fp16 / fp32 factors, larger ranks) take the reference's own
    fp32 product on the GPU (a plain library GEMM), rounded to bf16 and added, and the
    kernel requantizes the merged weight. merged_out, if given (bf16 [N, K], may be
    `weight` itself), receives the merged weight."""
    if not weight.is_cuda:
        raise ValueError("the fp8 requantizer is a HIP kernel; the weight must be on the GPU")
    if weight.dim() != 2 or weight.dtype not in _DTYPES:
        raise ValueError(f"expected a bfloat16, float16 or float32 [N, K] weight, got {weight.dtype} "
                         f"{tuple(weight.shape)}")
    w = weight.contiguous()
    N, K = w.shape
    q = torch.empty(N, K, device=w.device, dtype=FP8_DTYPE)
    s = torch.empty(N, device=w.device, dtype=torch.float32)
    if w.dtype != torch.bfloat16:
        # float16 / float32 weights: a LoRA is merged by the reference's own update
        # (lora.py:91-92, in the weight's type), then the typed requantization
        if merged_out is not None and (merged_out.shape != (N, K) or merged_out.dtype != w.dtype
                                       or not merged_out.is_contiguous() or merged_out.device != w.device):
            raise ValueError("merged_out must be a contiguous [N, K] tensor of the weight's type and device")
        if lora is not None:
            a, b, lscale = lora
            a, b = _lora_factor(a, w, "A"), _lora_factor(b, w, "B")
            rank = a.shape[0]
            if a.shape != (rank, K) or b.shape != (N, rank):
                raise ValueError(f"LoRA shapes {tuple(a.shape)} / {tuple(b.shape)} do not fit a [{N}, {K}] weight")
            w = w + lora_delta(a, b, lscale, dtype=w.dtype)
        if merged_out is not None:
            merged_out.copy_(w)
        lib = _lib.load()
        _lib.check(lib.vdn_fp8_requantize_weight_typed(_ptr(w), _DTYPES[w.dtype], N, K, K, _ptr(q), K, _ptr(s),
                                                       _stream(w)), "requantize_weight")
        return q, s
    a = b = None
    rank, lscale = 0, 1.0
    if merged_out is not None:
        if merged_out.shape != (N, K) or merged_out.dtype != torch.bfloat16 or not merged_out.is_contiguous() \
                or merged_out.device != w.device:
            raise ValueError("merged_out must be a contiguous bf16 [N, K] tensor on the weight's device")
    if lora is not None:
        a, b, lscale = lora
        a, b = _lora_factor(a, w, "A"), _lora_factor(b, w, "B")
        rank = a.shape[0]
        if a.shape != (rank, K) or b.shape != (N, rank):
            raise ValueError(f"LoRA shapes {tuple(a.shape)} / {tuple(b.shape)} do not fit a [{N}, {K}] weight")
        if not lora_in_kernel(a, b):
            merged = w + lora_delta(a, b, lscale)
            if merged_out is not None:
                merged_out.copy_(merged)
            return requantize_weight(merged)
        a = _aligned16(a)
    lib = _lib.load()
    _lib.check(lib.vdn_fp8_requantize_weight(_ptr(w), N, K, K, _ptr(a), _ptr(b), rank, float(lscale),
                                             _ptr(q), K, _ptr(s), _ptr(merged_out), _stream(w)),
               "requantize_weight")
    return q, s


def _lora_factor(t, w, name):
    if t.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"LoRA factor {name} must be bfloat16, float16 or float32 (got {t.dtype})")
    return t.to(w.device).contiguous()


# Largest LoRA rank the fused merge kernel takes (its A^T slice is staged in LDS).
LORA_KERNEL_MAX_RANK = 128


def lora_in_kernel(a, b):
    """True when the fused merge + requantize kernel takes these factors: bf16 A [r, K]
    and B [N, r] with 1 <= r <= 128 and K % 16 == 0. Other adapters (fp16 / fp32
    factors, larger ranks) take `lora_delta`, the reference's own update."""
    r, K = a.shape
    return (a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16 and 1 <= r <= LORA_KERNEL_MAX_RANK
            and K % 16 == 0)


def lora_delta(a, b, scale, dtype=torch.bfloat16):
    """(scale * (B.float() @ A.float())).to(dtype): the reference's update (lora.py:91-92),
    as an fp32 GEMM on the factors' device (a plain library GEMM), for the adapters the
    fused kernel does not take (`lora_in_kernel`) and for targets that are not contiguous
    bf16 GPU weights."""
    return ((b.to(torch.float32) @ a.to(torch.float32)) * scale).to(dtype)


class Fp8Linear(nn.Module):
    """nn.Linear replacement with e4m3 operands and an fp32-accumulating MFMA GEMM
    (the reference's class: fp8_linear.py:243-283).

    Construction turns the Linear's bf16 weight into codes with one scale per output
    channel (the only time the weight is read); the module keeps those codes and the
    scales, plus the Linear's own bias Parameter, and holds no reference to the bf16
    weight. Each `forward` quantizes its input per token first; a caller that feeds one
    activation to several projections quantizes it once and calls `forward_quantized`.

    Buffers: weight_fp8 e4m3 [N, K], weight_scale fp32 [1, N]; `bias` is the source
    Linear's Parameter object itself.
    """

    def __init__(self, linear: nn.Linear, *, lora=None):
        super().__init__()
        _rowwise_only()
        w = linear.weight.detach()
        home = w.device
        if not w.is_cuda:
            # The reference's rowwise branch is eager torch on any device
            # (fp8_linear.py:262-267); here the requantization is a HIP kernel, so a
            # host-resident Linear is requantized on the current GPU and its buffers are
            # returned to the Linear's device, as the reference's would live there.
            if not torch.cuda.is_available():
                raise ValueError("Fp8Linear needs a GPU: the fp8 requantizer is a HIP kernel "
                                 f"(the Linear's weight is on {home})")
            w = w.to(torch.device("cuda", torch.cuda.current_device()))
        q, s = requantize_weight(w, lora=lora)
        self.register_buffer("weight_fp8", q.to(home))
        self.register_buffer("weight_scale", s.reshape(1, -1).contiguous().to(home))
        self.register_parameter("bias", linear.bias)

    @property
    def in_features(self):
        return self.weight_fp8.shape[1]

    @property
    def out_features(self):
        return self.weight_fp8.shape[0]

    def forward_quantized(self, x_fp8, x_scale, out_dtype=torch.bfloat16, *, epilogue=None,
                          gate=None, gate_index=None, residual=None):
        """[M, K] fp8 rows and their [M, 1] scales -> [M, N] (fp8_linear.py:270-277).

        Computes bf16(epi(x_scale * w_scale * (x_fp8 @ weight_fp8.T) + bias)) in one
        kernel; with out_dtype float32 or float16 (a model that does not run in bf16: what
        `forward` passes for such rows, as the reference does) the GEMM writes the binary32
        product, then the cast and `+ bias` follow as in the reference. epilogue: None, "gelu_tanh", or "gate" -- gate [T, N] (or [N]) table,
        gate_index [M] rows of it (None = row 0; out-of-range indices are clamped),
        residual [M, N] (optional): gate[gate_index] * out + residual, the gated residual
        add of the block (fused_block.py:47-49)."""
        if out_dtype not in _DTYPES:
            raise ValueError(f"the fp8 GEMM writes bfloat16, float16 or float32 (out_dtype={out_dtype})")
        if out_dtype != torch.bfloat16 and (epilogue is not None or gate is not None or residual is not None):
            raise ValueError(f"the fused epilogues write bfloat16 (out_dtype={out_dtype})")
        if not x_fp8.is_cuda or x_fp8.dtype != FP8_DTYPE or x_fp8.dim() != 2:
            raise ValueError("x_fp8 must be a float8_e4m3fn [M, K] tensor on the GPU")
        M, K = x_fp8.shape
        N = self.weight_fp8.shape[0]
        if K != self.weight_fp8.shape[1]:
            raise ValueError(f"x has K={K}, the weight has K={self.weight_fp8.shape[1]}")
        if x_scale.numel() != M or x_scale.dtype != torch.float32:
            raise ValueError("x_scale must be the fp32 [M, 1] rowwise scale (per-tensor scales are "
                             "the sm100 branch, not built for gfx950)")
        dev = x_fp8.device
        if x_scale.device != dev or self.weight_fp8.device != dev:
            raise ValueError(f"x_fp8 ({dev}), x_scale ({x_scale.device}) and the fp8 weight "
                             f"({self.weight_fp8.device}) must be on one device")
        if x_fp8.stride(1) != 1:
            x_fp8 = x_fp8.contiguous()
        x_fp8 = _aligned16(x_fp8)
        x_scale = _aligned16(x_scale.contiguous())
        lib = _lib.load()
        ws_bytes = gemm_workspace_bytes(M, N, K, dev)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if ws_bytes else None
        if out_dtype != torch.bfloat16:
            # the reference's _scaled_mm with a float16 / float32 out_dtype, then `out + bias`
            # (fp8_linear.py:272-276): the GEMM writes the binary32 product, and the
            # rounding to float16 and the bias add are the reference's own two ops
            out = torch.empty(M, N, device=dev, dtype=torch.float32)
            _lib.check(lib.vdn_fp8_gemm_ws(_ptr(x_fp8), _ptr(x_scale), _ptr(self.weight_fp8),
                                           _ptr(self.weight_scale), M, N, K, x_fp8.stride(0), K,
                                           None, _lib.EPI_F32, None, None, 0, 0, None, 0,
                                           _ptr(out), N, _ptr(ws), ws_bytes, _stream(x_fp8)),
                       "fp8 gemm")
            if out_dtype != torch.float32:
                out = out.to(out_dtype)
            if self.bias is not None:
                out = out + self.bias
            return out
        out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
        epi = _EPILOGUES.get(epilogue)
        if epi is None:
            raise ValueError(f"unknown epilogue {epilogue!r}")
        bias = self.bias
        late_bias = None
        if bias is not None:
            if bias.numel() != N:
                raise ValueError("the bias must hold one value per output channel")
            if bias.dtype != torch.bfloat16:
                # a bias of another type (a float32 / float16 Linear fed bf16 rows): the
                # reference's `out + bias` promotes to that type, so it is added after the
                # GEMM as the reference's own op (no fused epilogue then)
                if epi != _lib.EPI_NONE:
                    raise ValueError(f"the fused epilogues take a bfloat16 bias (got {bias.dtype})")
                late_bias, bias = bias, None
            else:
                bias = _aligned16(bias.detach().to(dev).contiguous())
        g = gi = res = None
        ldgate = ldres = grows = 0
        if epi == _lib.EPI_GATE:
            if gate is None:
                raise ValueError('epilogue="gate" needs a gate table')
            g = gate.detach().to(dev).reshape(-1, N)
            if g.dtype != torch.bfloat16 or g.stride(1) != 1:
                g = g.to(torch.bfloat16).contiguous()
            ldgate, grows = g.stride(0), g.shape[0]
            if gate_index is not None:
                gi = _aligned16(gate_index.to(device=dev, dtype=torch.int32).contiguous())
                if gi.numel() != M:
                    raise ValueError("gate_index must hold one table row per token")
                check_index_range(gi, grows, "gate_index")
            if residual is not None:
                res = residual.detach()
                if res.device != dev:
                    raise ValueError(f"residual is on {res.device}, the activation on {dev}")
                if res.shape != (M, N) or res.dtype != torch.bfloat16 or res.stride(1) != 1:
                    raise ValueError("residual must be a bfloat16 [M, N] tensor with unit column stride")
                ldres = res.stride(0)
        elif gate is not None or residual is not None or gate_index is not None:
            raise ValueError('gate / gate_index / residual need epilogue="gate"')
        _lib.check(lib.vdn_fp8_gemm_ws(_ptr(x_fp8), _ptr(x_scale), _ptr(self.weight_fp8),
                                       _ptr(self.weight_scale), M, N, K, x_fp8.stride(0), K,
                                       _ptr(bias), epi, _ptr(g), _ptr(gi), grows, ldgate, _ptr(res), ldres,
                                       _ptr(out), N, _ptr(ws), ws_bytes, _stream(x_fp8)),
                   "fp8 gemm")
        return out if late_bias is None else out + late_bias

    def forward(self, x, **epilogue):
        shape = x.shape
        rows = x.reshape(-1, shape[-1])
        if "residual" in epilogue and epilogue["residual"] is not None:
            epilogue["residual"] = epilogue["residual"].reshape(rows.shape[0], -1)
        out = self.forward_quantized(*quantize_activation(rows), out_dtype=rows.dtype, **epilogue)
        return out.reshape(*shape[:-1], -1)


def _blocks_to_skip(model, skip_end_blocks):
    """The set of id()s of all modules that belong to the leading or trailing
    `skip_end_blocks` entries of model.transformer_blocks (empty when the model has no
    such list): those stay bf16 (fp8_linear.py:286-295)."""
    blocks = getattr(model, "transformer_blocks", None)
    if not blocks or skip_end_blocks <= 0:
        return set()
    keep = set()
    for index, block in enumerate(blocks):
        if index < skip_end_blocks or index >= len(blocks) - skip_end_blocks:
            keep.update(id(m) for m in block.modules())
    return keep


def convert_linear_to_fp8(model, min_width=MIN_WIDTH, skip_end_blocks=SKIP_END_BLOCKS):
    """Replace, inside `model`, every nn.Linear whose input and output widths are both at
    least `min_width` (outside the end blocks `_blocks_to_skip` names) by an Fp8Linear.
    Works in place and returns the number replaced (fp8_linear.py:298-323).

    The weights are read here, so LoRA has to be merged before this runs
    (`vdn_fp8.lora.merge_lora_and_convert` does both per weight). The list of work holds
    (parent module, attribute name) pairs rather than the Linears: once a parent points
    at its Fp8Linear nothing keeps the bf16 Linear alive, so at most one bf16 weight and
    its fp8 copy coexist beyond the model itself."""
    skip = _blocks_to_skip(model, skip_end_blocks)
    targets = [(parent, name) for parent in model.modules()
               for name, child in parent.named_children()
               if isinstance(child, nn.Linear) and child.in_features >= min_width
               and child.out_features >= min_width and id(child) not in skip]
    for parent, name in targets:
        child = getattr(parent, name)
        setattr(parent, name, Fp8Linear(child).to(child.weight.device))
        del child
    return len(targets)
