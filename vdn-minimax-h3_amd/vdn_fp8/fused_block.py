"""The DiT block's pre-norm fused with the fp8 quantization of its output.

Mirrors the part of `src.models.ops.fused_block` that feeds an fp8 linear: in the
reference, `fast_block_forward` runs the compiled `pre` (`_pre_ref`: RMSNorm, then the
AdaLN affine, fused_block.py:41-44,101-108) and the projection that consumes its output
then quantizes it per token (`Fp8Linear.forward` -> `quantize_rows`, fp8_linear.py:110-117,
279-283). Here one kernel does both, so the bf16 normed activation never has to be
written (`return_normed=True` writes it as well, for a consumer that needs it).

The gated residual add (`_post_ref`, fused_block.py:47-49) is the GEMM's gate epilogue:
`Fp8Linear.forward_quantized(..., epilogue="gate", gate=..., gate_index=..., residual=...)`.
"""
import torch

from . import _lib
from .fp8_linear import FP8_DTYPE, _aligned16, _ptr, _rows, _stream


def pre_quantize(hidden, weight, eps, scale=None, shift=None, indices=None, return_normed=False):
    """RMSNorm(hidden; weight, eps) * (1 + scale[indices]) + shift[indices], rounded to
    bf16 once, then quantized per token -> (fp8 [M, K], fp32 scale [M, 1][, bf16 normed]).

    hidden bf16 [M, K] (or [..., K]); weight bf16 [K] or None; scale/shift bf16 [T, K]
    (or [K]) or None; indices int [M] or None (row 0 of the table). The codes and scales
    equal quantize_rows(normed) bit for bit."""
    shape = hidden.shape
    x = _rows(hidden.reshape(-1, shape[-1]))
    M, K = x.shape
    dev = x.device
    w = None
    if weight is not None:
        if weight.numel() != K or weight.dtype != torch.bfloat16:
            raise ValueError("weight must be a bfloat16 [K] tensor")
        w = _aligned16(weight.detach().to(dev).contiguous())
    sc = sh = idx = None
    rows = ld = 0
    if (scale is None) != (shift is None):
        raise ValueError("scale and shift go together")
    if scale is not None:
        sc = scale.detach().to(dev).reshape(-1, K)
        sh = shift.detach().to(dev).reshape(-1, K)
        if sc.dtype != torch.bfloat16 or sh.dtype != torch.bfloat16 or sc.shape != sh.shape:
            raise ValueError("scale and shift must be bfloat16 tables of the same shape [T, K]")
        sc, sh = _aligned16(sc.contiguous()), _aligned16(sh.contiguous())
        rows, ld = sc.shape[0], K
        if indices is not None:
            idx = indices.to(device=dev, dtype=torch.int32).contiguous()
            if idx.numel() != M:
                raise ValueError("indices must hold one table row per token")
    elif indices is not None:
        raise ValueError("indices need a scale/shift table")
    y = torch.empty(M, K, device=dev, dtype=FP8_DTYPE)
    s = torch.empty(M, 1, device=dev, dtype=torch.float32)
    normed = torch.empty(M, K, device=dev, dtype=torch.bfloat16) if return_normed else None
    lib = _lib.load()
    _lib.check(lib.vdn_fp8_norm_quantize_rows(_ptr(x), M, K, x.stride(0), _ptr(w), float(eps), _ptr(sc), _ptr(sh),
                                              ld, _ptr(idx), rows, _ptr(y), K, _ptr(s), _ptr(normed), K, _stream(x)),
               "norm_quantize_rows")
    if return_normed:
        return y, s, normed.reshape(shape)
    return y, s
