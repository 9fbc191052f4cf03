"""LoRA merging at inference on MI355X -- a drop-in for the reference's
`src.inference.utils.lora` (src/inference/utils/lora.py).

    W += scale * (B @ A)     delta in fp32, added in the weight's dtype (bf16)

`merge_lora_state` keeps the reference's in-place semantics and return value; for
contiguous bf16 GPU weights and bf16 adapters of rank <= 128 the update runs in the HIP
kernel behind vdn_fp8_requantize_weight (merge-only mode), for any other target or
adapter it is the reference's own torch update (`merge_into`).
`merge_lora_and_convert` fuses the merge into the fp8 conversion: for every Linear
that `convert_linear_to_fp8` would swap, W + scale * B @ A is quantized directly
(the merged bf16 weight is never written), and the remaining pairs are merged in
place -- the reference's "merge LoRA, then convert" order (assemble.py:116-175) in
one pass over each weight.

Adapter files: `load_external_lora` and `_translate_original_layout` read peft-named
safetensors and the original (non-diffusers) key layout, as lora.py:25-117 does.
"""
import re

import torch
import torch.nn as nn

from . import _lib
from .fp8_linear import (MIN_WIDTH, SKIP_END_BLOCKS, Fp8Linear, _aligned16, _blocks_to_skip, _ptr,
                         _stream, lora_delta, lora_in_kernel)

# Original-layout module names -> diffusers names (lora.py:22-30).
_ORIGINAL_RENAMES = (
    (".mlp.fc1.", ".ff.net.0.proj."),
    (".mlp.fc2.", ".ff.net.2."),
    (".attn.out_proj.", ".attn.to_out.0."),
)


def _translate_original_layout(state):
    """Rewrite original-layout adapter keys onto diffusers names (lora.py:32-66).

    - `diffusion_model.` prefixes are dropped; `blocks.N` becomes `transformer_blocks.N`;
      the refiner and final-layer modules are renamed;
    - a fused `qkv_proj` pair becomes three pairs: lora_A shared, lora_B split in
      (q, k, v) row order;
    - the SwiGLU halves of `mlp.fc1`'s lora_B are swapped: the original packs
      [gate; value], diffusers' ff.net.0.proj packs [value; gate].
    Diffusers-named adapters (no `.qkv_proj.` key) pass through unchanged."""
    if not any(".qkv_proj." in key for key in state):
        return state
    out = {}
    for key, tensor in state.items():
        name = key[len("diffusion_model."):] if key.startswith("diffusion_model.") else key
        name = re.sub(r"^blocks\.", "transformer_blocks.", name)
        name = name.replace("token_refiner.blocks.", "token_refiner.refiner_blocks.")
        name = name.replace("final_layer.adaln_proj.linear.", "norm_out.linear.")
        if ".mlp.fc1." in name and ".lora_B." in name:
            gate_half, value_half = tensor.chunk(2, dim=0)
            tensor = torch.cat([value_half, gate_half], dim=0)
        for old, new in _ORIGINAL_RENAMES:
            name = name.replace(old, new)
        if ".attn.qkv_proj." in name:
            parts = (tensor,) * 3 if ".lora_A." in name else tensor.chunk(3, dim=0)
            for proj, part in zip(("to_q", "to_k", "to_v"), parts):
                out[name.replace(".attn.qkv_proj.", f".attn.{proj}.")] = part
            continue
        out[name] = tensor
    return out


def _resolve(params, target):
    """The parameter a LoRA target names; tries the `.attn.orig.` re-rooting of a
    hybrid model second (lora.py:69-77)."""
    if target in params:
        return params[target]
    if ".attn." in target:
        rerooted = target.replace(".attn.", ".attn.orig.", 1)
        if rerooted in params:
            return params[rerooted]
    raise KeyError(f"LoRA target {target!r} has no parameter in the model "
                   "(also tried the .attn.orig. rerooting)")


def _pairs(state):
    """(target weight name, A, B) for every lora_A key, in state order."""
    for name, a in state.items():
        if ".lora_A." not in name:
            continue
        b = state[name.replace(".lora_A.", ".lora_B.")]
        yield name.split(".lora_A.")[0] + ".weight", a, b


def merge_into(weight, a, b, scale=1.0):
    """weight (W [N, K]) += (scale * (B @ A)).to(W.dtype), in place (lora.py:91-92).

    A contiguous bf16 weight on the GPU with bf16 factors of rank <= 128 is merged by the
    HIP kernel (merge-only mode of vdn_fp8_requantize_weight). Every other target -- an
    fp32 or fp16 weight (the hybrid attention's parameters before their bf16 cast,
    assemble.py:124 vs :148-151), a non-contiguous view, a weight still in host memory --
    and every other adapter (fp16 / fp32 factors, larger ranks) takes the reference's own
    arithmetic where the weight lives: the fp32 product of the factors, scaled, cast to
    the weight's dtype, then added."""
    for t, nm in ((a, "A"), (b, "B")):
        if t.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise ValueError(f"LoRA factor {nm} must be bfloat16, float16 or float32 (got {t.dtype})")
    if weight.dim() != 2:
        raise ValueError(f"a LoRA target must be a 2-D weight, got {tuple(weight.shape)}")
    N, K = weight.shape
    r = a.shape[0]
    if a.dim() != 2 or b.dim() != 2 or a.shape != (r, K) or b.shape != (N, r):
        raise ValueError(f"LoRA shapes {tuple(a.shape)} / {tuple(b.shape)} do not fit a [{N}, {K}] weight")
    a = a.to(weight.device).contiguous()
    b = b.to(weight.device).contiguous()
    if not (weight.is_cuda and weight.dtype == torch.bfloat16 and weight.is_contiguous()
            and lora_in_kernel(a, b)):
        weight.add_(lora_delta(a, b, scale, dtype=weight.dtype))
        return weight
    lib = _lib.load()
    a = _aligned16(a)
    _lib.check(lib.vdn_fp8_requantize_weight(_ptr(weight), N, K, K, _ptr(a), _ptr(b), r, float(scale),
                                             None, 0, None, _ptr(weight), _stream(weight)),
               "merge_lora_state")
    return weight


def merge_lora_state(model, state, scale=1.0):
    """Fold peft-named `.lora_A. / .lora_B.` pairs into the model, in place.
    Returns the number of pairs merged (lora.py:80-94)."""
    params = dict(model.named_parameters())
    merged = 0
    for target, a, b in _pairs(state):
        w = _resolve(params, target)
        merge_into(w.data, a, b, scale)
        merged += 1
    return merged


def merge_lora_and_convert(model, state, scale=1.0, min_width=MIN_WIDTH,
                           skip_end_blocks=SKIP_END_BLOCKS):
    """merge_lora_state followed by convert_linear_to_fp8, fused per weight.

    Returns (pairs merged, Linears converted). Every Linear the conversion selects gets
    its LoRA (if any) folded inside the requantize kernel; pairs whose target stays bf16
    are merged in place."""
    params = dict(model.named_parameters())
    by_param = {}
    for target, a, b in _pairs(state):
        by_param[id(_resolve(params, target))] = (a, b)
    skip = _blocks_to_skip(model, skip_end_blocks)
    targets = [(parent, name) for parent in model.modules()
               for name, child in parent.named_children()
               if isinstance(child, nn.Linear) and child.in_features >= min_width
               and child.out_features >= min_width and id(child) not in skip]
    merged = 0
    for parent, name in targets:
        child = getattr(parent, name)
        pair = by_param.pop(id(child.weight), None)
        lora = None if pair is None else (pair[0], pair[1], scale)
        setattr(parent, name, Fp8Linear(child, lora=lora).to(child.weight.device))
        merged += pair is not None
        del child
    for pid, (a, b) in by_param.items():
        w = next(p for p in params.values() if id(p) == pid)
        merge_into(w.data, a, b, scale)
        merged += 1
    return merged, len(targets)


def load_external_lora(path, alpha=None):
    """Read a community LoRA safetensors -> (state, scale, ranks) (lora.py:97-117).

    The peft `.default.` infix is stripped; original-layout keys are translated;
    `alpha` (argument, else the file's metadata) scales the merge by alpha / rank, and a
    missing alpha means alpha == rank (scale 1.0)."""
    from safetensors import safe_open

    state = {}
    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
        for key in f.keys():
            state[key.replace(".default.", ".")] = f.get_tensor(key)
    state = _translate_original_layout(state)
    ranks = sorted({state[k].shape[0] for k in state if ".lora_A." in k})
    if alpha is None and "alpha" not in meta:
        scale = 1.0
    else:
        if len(ranks) != 1:
            raise ValueError(f"{path}: one alpha ({alpha or meta['alpha']}) cannot scale "
                             f"mixed ranks {ranks}")
        alpha = float(meta["alpha"]) if alpha is None else float(alpha)
        scale = alpha / ranks[0]
    return state, scale, ranks
