"""QK preparation for the softmax attention branch, MI355X-native.

Mirrors `_qk_prep` of the reference's `src.models.softmax_attention.kernels`
(kernels.py:8-45): everything between the q (or k) projection and the attention
call -- the per-head RMSNorm (`norm_q` / `norm_k`) and the rotary embedding -- in one
pass over [T, H, d], as `HybridAttention._qkv` uses it at inference
(hybrid_attention.py:128-130). The reference compiles the pair with inductor; here
it is a hand-written HIP kernel (`vdn_fp8_qk_prep`). Numerics follow the compiled
kernel: binary32 throughout, the cos/sin tables rounded to bf16 first
(`cos.to(x.dtype)`), one rounding at the store -- not bitwise with the eager chain,
which rounds after every op, exactly as the reference notes for its own kernel.
"""
import torch

from . import _lib
from .fp8_linear import _aligned16, _ptr, _stream


def qk_prep(t, weight, eps, cos=None, sin=None):
    """RMSNorm over the last dim (weight, eps), then rotary embedding with
    (cos, sin) of shape [T, R] (R <= d; the first R channels rotate as two halves,
    the rest pass through). t bf16 [T, H, d] (heads contiguous; any token stride)
    -> a new contiguous bf16 [T, H, d]."""
    if not t.is_cuda:
        raise ValueError("qk_prep runs on the GPU (a HIP kernel); got a CPU tensor")
    if t.dim() != 3 or t.dtype != torch.bfloat16:
        raise ValueError(f"qk_prep wants a bfloat16 [T, H, d] tensor (got {t.dtype} {tuple(t.shape)})")
    T, H, d = t.shape
    if t.stride(2) != 1 or t.stride(1) != d:
        t = t.contiguous()
    if t.data_ptr() % 16 or t.stride(0) % 8:
        t = t.contiguous()
    dev = t.device
    w = None
    if weight is not None:
        if weight.numel() != d or weight.dtype != torch.bfloat16:
            raise ValueError("weight must be a bfloat16 [d] tensor")
        w = _aligned16(weight.detach().to(dev).reshape(d).contiguous())
    R, ldcs, cs_bf16 = 0, 0, 0
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin go together")
    if cos is not None:
        cos = cos.detach().to(dev).reshape(-1, cos.shape[-1])
        sin = sin.detach().to(dev).reshape(-1, sin.shape[-1])
        if cos.shape != sin.shape or cos.shape[0] != T or cos.dtype != sin.dtype:
            raise ValueError(f"cos/sin must both be [T={T}, R] of one dtype (got {tuple(cos.shape)}, "
                             f"{tuple(sin.shape)})")
        if cos.dtype not in (torch.float32, torch.bfloat16):
            cos, sin = cos.float(), sin.float()
        cos, sin = _aligned16(cos.contiguous()), _aligned16(sin.contiguous())
        R, ldcs, cs_bf16 = cos.shape[1], cos.shape[1], int(cos.dtype == torch.bfloat16)
    out = torch.empty(T, H, d, device=dev, dtype=torch.bfloat16)
    lib = _lib.load()
    _lib.check(lib.vdn_fp8_qk_prep(_ptr(t), T, H, d, t.stride(0), _ptr(w), float(eps), _ptr(cos), _ptr(sin),
                                   R, ldcs, cs_bf16, _ptr(out), H * d, _stream(t)), "qk_prep")
    return out


# The reference's name (softmax_attention/kernels.py:33).
_qk_prep = qk_prep


def qkv(x, to_q, to_k, to_v, heads, norm_q, norm_k, rotary_emb=None):
    """The inference body of `HybridAttention._qkv` (hybrid_attention.py:108-137) on this
    library: with fp8 projections x is quantized ONCE and shared by the three GEMMs
    (hybrid_attention.py:118-124), then QK-norm + rope run as one pass each (`_qk_prep`,
    :128-130). x [T, hidden] bf16; to_q/k/v the projection modules (Fp8Linear or any
    callable); norm_q/norm_k modules with `.weight` and `.eps` (RMSNorm); rotary_emb
    (cos, sin) [T, R] or None. Returns (query, key, value, (query_raw, key_raw, value)),
    everything [T, heads, d] -- the raw q/k are the ones the linear branch consumes.
    Without rotary_emb the norms alone run (the same kernel with no rotation), as the
    reference's eager branch would apply them."""
    from .fp8_linear import Fp8Linear, quantize_activation

    projections = (to_q, to_k, to_v)
    if all(isinstance(p, Fp8Linear) for p in projections):
        x_fp8, x_scale = quantize_activation(x)
        out = [p.forward_quantized(x_fp8, x_scale, out_dtype=x.dtype) for p in projections]
    else:
        out = [p(x) for p in projections]
    query_raw, key_raw, value = (t.unflatten(-1, (heads, -1)) for t in out)
    cos, sin = (None, None) if rotary_emb is None else rotary_emb
    query = qk_prep(query_raw, norm_q.weight, norm_q.eps, cos, sin)
    key = qk_prep(key_raw, norm_k.weight, norm_k.eps, cos, sin)
    return query, key, value, (query_raw, key_raw, value)
