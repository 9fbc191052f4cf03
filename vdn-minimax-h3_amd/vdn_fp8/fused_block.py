"""The pointwise stretches of a DiT block, and the block's feed-forward, on MI355X.

A drop-in for `src.models.ops.fused_block` (src/models/ops/fused_block.py). The reference
hands each pointwise stretch to inductor: `pre` (RMSNorm, then the AdaLN affine,
`_pre_ref`, fused_block.py:41-44), `post` (the gated residual add, `_post_ref`, :47-49) and
the SwiGLU activation (`_swiglu_ref`, :67-70); `fast_ff_forward` (:73-90) and
`fast_block_forward` (:93-111) are the FeedForward and block forwards built on them. Here
each stretch is a HIP kernel of libvdnfp8.so, and where an fp8 linear consumes or
produces it the stretch is fused into that linear's kernels:

  pre + the next projection's quantization     vdn_fp8_norm_quantize_rows (`pre_quantize`)
  SwiGLU + the down projection's quantization  vdn_fp8_swiglu_quantize_rows
  down projection + post                       the GEMM's gate epilogue (with residual)

so with fp8 projections the whole feed-forward sub-layer of `fast_block_forward` is four
kernels and neither the bf16 normed input nor the bf16 SwiGLU activation nor the bf16 FF
output is ever written. Numerics follow the compiled reference: binary32 inside each
stretch, one rounding at its store (the reference's own caveat: not bitwise with the eager
bodies, which round after every op).

The eager bodies `_pre_ref`, `_post_ref`, `_swiglu_ref` are kept with the reference's names
and meaning for callers that import them; nothing on the fast path uses them (a bf16
feed-forward uses `_swiglu_one_rounding`, the compiled body's arithmetic).
"""
import torch
import torch.nn.functional as F

from . import _lib
from .fp8_linear import (FP8_DTYPE, Fp8Linear, _aligned16, _ptr, _rows, _stream, check_index_range,
                         swiglu_quantize_activation)


# --------------------------------------------------------------------------------------
# The eager bodies (the reference's, fused_block.py:41-49,67-70).
# --------------------------------------------------------------------------------------

def _pre_ref(hidden, weight, eps, scale, shift, indices):
    """RMSNorm, then the AdaLN affine: x_hat * (1 + scale[i]) + shift[i] (eager)."""
    normed = F.rms_norm(hidden, (hidden.shape[-1],), weight, eps)
    return normed * (1.0 + scale.index_select(0, indices)) + shift.index_select(0, indices)


def _post_ref(residual, gate, indices, branch_out):
    """The gated residual add: residual + gate[i] * branch_out (eager)."""
    return residual + gate.index_select(0, indices) * branch_out


def _swiglu_ref(h):
    """SwiGLU after its projection: a * silu(gate), (a, gate) = h.chunk(2) (eager)."""
    a, gate = h.chunk(2, dim=-1)
    return a * F.silu(gate)


def _swiglu_one_rounding(h):
    """The SwiGLU body as the reference's compiled region computes it
    (`_compiled("swiglu", _swiglu_ref)`, fused_block.py:88): a * silu(gate) in binary32,
    rounded once to h's dtype (eager rounds silu first, then the product)."""
    a, gate = h.chunk(2, dim=-1)
    return (a.float() * F.silu(gate.float())).to(h.dtype)


# --------------------------------------------------------------------------------------
# The kernels.
# --------------------------------------------------------------------------------------

def _pre_args(x, weight, scale, shift, indices):
    """Device copies / views of the pre-norm's operands, checked."""
    M, K = x.shape
    dev = x.device
    w = None
    if weight is not None:
        if weight.numel() != K or weight.dtype != torch.bfloat16:
            raise ValueError("weight must be a bfloat16 [K] tensor")
        w = _aligned16(weight.detach().to(dev).reshape(K).contiguous())
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
            idx = indices.to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
            if idx.numel() != M:
                raise ValueError("indices must hold one table row per token")
            check_index_range(idx, rows, "pre: indices")
    elif indices is not None:
        raise ValueError("indices need a scale/shift table")
    return w, sc, sh, ld, idx, rows


def pre_quantize(hidden, weight, eps, scale=None, shift=None, indices=None, return_normed=False):
    """RMSNorm(hidden; weight, eps) * (1 + scale[indices]) + shift[indices], rounded to
    bf16 once, then quantized per token -> (fp8 [M, K], fp32 scale [M, 1][, bf16 normed]).

    hidden bf16 [M, K] (or [..., K]); weight bf16 [K] or None; scale/shift bf16 [T, K]
    (or [K]) or None; indices int [M] or None (row 0 of the table). The codes and scales
    equal quantize_rows(normed) bit for bit."""
    shape = hidden.shape
    x = _aligned16(_rows(hidden.reshape(-1, shape[-1])))
    M, K = x.shape
    dev = x.device
    w, sc, sh, ld, idx, rows = _pre_args(x, weight, scale, shift, indices)
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


def pre(hidden, weight, eps, scale, shift, indices):
    """The compiled `pre` (fused_block.py:41-44,101-102): RMSNorm then the AdaLN affine
    with the table rows chosen per token, one bf16 rounding. Same arguments as `_pre_ref`
    (scale/shift bf16 [T, K], indices [M]); returns bf16 of hidden's shape."""
    shape = hidden.shape
    x = _aligned16(_rows(hidden.reshape(-1, shape[-1])))
    M, K = x.shape
    w, sc, sh, ld, idx, rows = _pre_args(x, weight, scale, shift, indices)
    normed = torch.empty(M, K, device=x.device, dtype=torch.bfloat16)
    lib = _lib.load()
    _lib.check(lib.vdn_fp8_norm_quantize_rows(_ptr(x), M, K, x.stride(0), _ptr(w), float(eps), _ptr(sc), _ptr(sh),
                                              ld, _ptr(idx), rows, None, 0, None, _ptr(normed), K, _stream(x)),
               "pre")
    return normed.reshape(shape)


def post(residual, gate, indices, branch_out):
    """The compiled `post` (fused_block.py:47-49,103-104): residual + gate[i] * branch_out,
    binary32 inside, one bf16 rounding. Same arguments as `_post_ref`; returns bf16 of
    residual's shape."""
    shape = residual.shape
    r = _aligned16(_rows(residual.reshape(-1, shape[-1])))
    M, N = r.shape
    dev = r.device
    b = branch_out.reshape(-1, branch_out.shape[-1])
    if b.shape != (M, N) or b.dtype != torch.bfloat16:
        raise ValueError(f"branch_out must be bfloat16 of the residual's shape (got {b.dtype} {tuple(b.shape)})")
    b = _aligned16(_rows(b))
    g = gate.detach().to(dev).reshape(-1, N)
    if g.dtype != torch.bfloat16:
        raise ValueError("gate must be a bfloat16 [T, N] table")
    g = _aligned16(g.contiguous())
    idx = None
    if indices is not None:
        idx = indices.to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
        if idx.numel() != M:
            raise ValueError("indices must hold one table row per token")
        check_index_range(idx, g.shape[0], "post: indices")
    out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    lib = _lib.load()
    _lib.check(lib.vdn_fp8_gated_residual(_ptr(r), r.stride(0), _ptr(g), N, _ptr(idx), g.shape[0], _ptr(b),
                                          b.stride(0), _ptr(out), N, M, N, _stream(r)), "post")
    return out.reshape(shape)


# --------------------------------------------------------------------------------------
# The forwards.
# --------------------------------------------------------------------------------------

def fast_ff_forward(self, hidden_states):
    """Drop-in for FeedForward.forward ([SwiGLU, Dropout, Linear]) at inference
    (fused_block.py:73-90): the projection GEMM, then -- with an fp8 down projection --
    SwiGLU fused with the down projection's quantization (the bf16 activation is never
    written) and the down GEMM; otherwise the activation with one rounding, as the
    reference's compiled body, and the down layer."""
    swiglu, _, down = self.net
    shape = hidden_states.shape
    h = swiglu.proj(hidden_states.reshape(-1, shape[-1]))
    if isinstance(down, Fp8Linear):
        out = down.forward_quantized(*swiglu_quantize_activation(h), out_dtype=h.dtype)
    else:
        out = down(_swiglu_one_rounding(h))
    return out.reshape(*shape[:-1], -1)


def _ff_fp8(ff):
    """(proj, down) when the feed-forward's two linears are both fp8, else None."""
    net = getattr(ff, "net", None)
    if net is None or len(net) != 3:
        return None
    proj, down = getattr(net[0], "proj", None), net[2]
    if isinstance(proj, Fp8Linear) and isinstance(down, Fp8Linear):
        return proj, down
    return None


def fast_block_forward(self, hidden_states, temb, adaln_indices, rotary_emb, attention_mask=None):
    """Drop-in for MiniMaxH3TransformerBlock.forward at inference (fused_block.py:93-111).

    The attention sub-layer: `pre` and `post` as one kernel each around `self.attn`. The
    feed-forward sub-layer, when both of its linears are fp8: the pre-norm fused with the
    projection's quantization, the projection GEMM, SwiGLU fused with the down
    projection's quantization, and the down GEMM with the gated residual add in its
    epilogue -- four kernels; otherwise `pre`, `self.ff`, `post`."""
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = self.adaln_proj(temb)
    normed = pre(hidden_states, self.norm1.weight, self.norm1.eps, scale_msa, shift_msa, adaln_indices)
    hidden_states = post(hidden_states, gate_msa, adaln_indices, self.attn(normed, rotary_emb, attention_mask))

    fp8 = _ff_fp8(self.ff)
    if fp8 is None:
        normed = pre(hidden_states, self.norm2.weight, self.norm2.eps, scale_mlp, shift_mlp, adaln_indices)
        return post(hidden_states, gate_mlp, adaln_indices, self.ff(normed))
    proj, down = fp8
    shape = hidden_states.shape
    resid = _rows(hidden_states.reshape(-1, shape[-1]))
    xq, xs = pre_quantize(resid, self.norm2.weight, self.norm2.eps, scale_mlp, shift_mlp, adaln_indices)
    h = proj.forward_quantized(xq, xs, out_dtype=resid.dtype)
    yq, ys = swiglu_quantize_activation(h)
    gi = None if adaln_indices is None else adaln_indices.to(device=resid.device, dtype=torch.int32).reshape(-1)
    out = down.forward_quantized(yq, ys, out_dtype=resid.dtype, epilogue="gate",
                                 gate=gate_mlp.reshape(-1, shape[-1]), gate_index=gi, residual=resid)
    return out.reshape(shape)
