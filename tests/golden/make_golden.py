"""Writes the committed golden fixtures under tests/golden/ (run in the build container,
where the reference checkout is mounted read-only):

    python tests/golden/make_golden.py

Expected outputs come from torch's CPU eager ops spelled exactly as the reference's
own eager functions (quantize_rows_reference, fp8_linear.py:132-135; the rowwise
branch of Fp8Linear.__init__, fp8_linear.py:262-267; merge_lora_state's update,
lora.py:91-92) -- library routines independent of the C oracle, which the CPU tests
then check against these files. No reference module is imported or run.

Fixtures:
  prompt_rows.npz  32 rows of the reference's encoded prompt cache (prompts/example_0.pt,
                   loaded with weights_only=True): the rows holding the largest and
                   smallest maxima plus a seeded sample, with their codes and scales.
  single.json      sha256 of the 1024^3 single-linear workload's inputs (seed 0) and of
                   the expected activation/weight codes and scales, plus the output
                   checksum of the fp64 dequantized matmul.
  lora_small.npz   a small LoRA merge (w [48, 320], A [16, 320], B [48, 16], scale 0.5)
                   with torch's fp32-matmul merge and the requantized codes.
"""
import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "vdn-minimax-h3_amd"))
REFERENCE = "/root/reference"

FP8 = torch.float8_e4m3fn
FP8_MAX = torch.finfo(FP8).max


def rows_reference(x):
    """quantize_rows_reference, in torch CPU ops."""
    scale = (x.float().abs().amax(dim=1, keepdim=True) / FP8_MAX).clamp_min(1e-12)
    return (x.float() / scale).to(FP8), scale


def weight_reference(w):
    """Rowwise branch of Fp8Linear.__init__, in torch CPU ops."""
    scale = (w.abs().amax(dim=1, keepdim=True).float() / FP8_MAX).clamp_min(1e-12)
    return (w / scale.to(w.dtype)).to(FP8), scale.reshape(1, -1)


def u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def u8(t):
    return t.contiguous().view(torch.uint8).numpy()


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def prompt_rows():
    d = torch.load(os.path.join(REFERENCE, "prompts", "example_0.pt"), weights_only=True)
    x = d["prompt_embeds"]
    amax = x.float().abs().amax(dim=1)
    order = torch.argsort(amax)
    g = torch.Generator().manual_seed(0)
    pick = torch.cat([order[-8:], order[:8], torch.randperm(x.shape[0], generator=g)[:16]])
    pick = torch.unique(pick)
    rows = x[pick].contiguous()
    q, s = rows_reference(rows)
    np.savez_compressed(os.path.join(HERE, "prompt_rows.npz"), x=u16(rows), codes=u8(q),
                        scale=s.reshape(-1).numpy(), rows=pick.numpy())
    return len(pick)


def single():
    from vdn_fp8 import workloads
    x, w, b = workloads.dit_single()
    qx, sx = rows_reference(x)
    qw, sw = weight_reference(w)
    out = (qx.double() * sx.double()) @ (qw.double() * sw.double().reshape(-1, 1)).T + b.double()
    info = {
        "workload": "single linear 1024x1024x1024, seed 0",
        "x": sha(u16(x)), "w": sha(u16(w)), "bias": sha(u16(b)),
        "x_codes": sha(u8(qx)), "x_scale": sha(sx.reshape(-1).numpy()),
        "w_codes": sha(u8(qw)), "w_scale": sha(sw.reshape(-1).numpy()),
        "out_sum": float(out.sum()), "out_sumsq": float((out * out).sum()),
        "out_first_row_head": [float(v) for v in out[0, :8]],
    }
    with open(os.path.join(HERE, "single.json"), "w") as f:
        json.dump(info, f, indent=1)


def lora_small():
    g = torch.Generator().manual_seed(1)
    w = (torch.randn(48, 320, generator=g) * 0.02).to(torch.bfloat16)
    a = (torch.randn(16, 320, generator=g) * 0.05).to(torch.bfloat16)
    b = (torch.randn(48, 16, generator=g) * 0.05).to(torch.bfloat16)
    scale = 0.5
    merged = w.clone()
    delta = (b.to(torch.float32) @ a.to(torch.float32)) * scale
    merged.add_(delta.to(merged.dtype))
    q, s = weight_reference(merged)
    np.savez_compressed(os.path.join(HERE, "lora_small.npz"), w=u16(w), a=u16(a), b=u16(b),
                        scale=np.float32(scale), merged=u16(merged), codes=u8(q),
                        w_scale=s.reshape(-1).numpy())


if __name__ == "__main__":
    print("prompt rows:", prompt_rows())
    single()
    lora_small()
    print("written to", HERE)
