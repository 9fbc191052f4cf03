"""GPU tests of the model-level entry points: `convert_linear_to_fp8` (fp8_linear.py:298-323)
on a small model, and `merge_lora_and_convert` against the reference's order -- merge every
LoRA pair in place (`merge_lora_state`, lora.py:80-94), then convert -- which it fuses per
weight. The fused path must give the same fp8 weights bit for bit: the merged weight
W' = bf16(W + bf16(scale B A)) is formed by the same arithmetic in both, and its codes and
scales are the rowwise quantization of W'."""
import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle as O
import vdn_fp8
from conftest import bits, codes
from vdn_fp8 import lora as LR

pytestmark = pytest.mark.gpu


class _Attn(nn.Module):
    def __init__(self, w):
        super().__init__()
        self.to_q = nn.Linear(w, w, dtype=torch.bfloat16)
        self.to_k = nn.Linear(w, w, bias=False, dtype=torch.bfloat16)


class _Blk(nn.Module):
    def __init__(self, w):
        super().__init__()
        self.attn = _Attn(w)
        self.ff = nn.Linear(w, 2 * w, dtype=torch.bfloat16)
        self.small = nn.Linear(w, w // 4, dtype=torch.bfloat16)


class _Model(nn.Module):
    def __init__(self, n, w, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.transformer_blocks = nn.ModuleList(_Blk(w) for _ in range(n))
        self.proj_out = nn.Linear(w, w, dtype=torch.bfloat16)
        with torch.no_grad():
            for p in self.parameters():
                p.copy_((0.02 * torch.randn(p.shape, generator=g)).to(torch.bfloat16))


def _lora_state(model, rank, seed):
    g = torch.Generator().manual_seed(seed)
    state = {}
    for name, mod in model.named_modules():
        if isinstance(mod, nn.Linear) and name.endswith(("to_q", "ff", "small")):
            state[f"{name}.lora_A.weight"] = (0.02 * torch.randn(rank, mod.in_features, generator=g)).to(torch.bfloat16)
            state[f"{name}.lora_B.weight"] = (0.02 * torch.randn(mod.out_features, rank, generator=g)).to(torch.bfloat16)
    return state


def test_convert_linear_to_fp8_forward(device):
    m = _Model(5, 512, seed=1).to(device)
    ref_q = m.transformer_blocks[2].attn.to_q.weight.detach().clone()
    n = vdn_fp8.convert_linear_to_fp8(m, min_width=256, skip_end_blocks=1)
    assert n == 3 * 3 + 1                     # blocks 1..3: to_q, to_k, ff; proj_out
    lin = m.transformer_blocks[2].attn.to_q
    assert isinstance(lin, vdn_fp8.Fp8Linear) and isinstance(m.transformer_blocks[0].attn.to_q, nn.Linear)
    assert isinstance(m.transformer_blocks[2].small, nn.Linear)
    wq, ws = O.quantize_weight(bits(ref_q))
    assert np.array_equal(codes(lin.weight_fp8), wq)
    assert np.array_equal(lin.weight_scale.cpu().numpy().ravel().view(np.uint32), ws.view(np.uint32))
    x = torch.randn(3, 70, 512, device=device).to(torch.bfloat16)
    y = lin(x)
    torch.cuda.synchronize()
    assert y.shape == (3, 70, 512) and y.dtype == torch.bfloat16
    qx, sx = O.quantize_rows(bits(x.reshape(-1, 512)))
    want = O.dequant_linear(qx, sx, wq, ws, bias=bits(lin.bias))
    got = O.bf16_decode(bits(y.reshape(-1, 512)))
    assert O.rel_l2(got, want) <= 1e-3


@pytest.mark.parametrize("rank,scale", [(16, 1.0), (7, 0.5)])
def test_merge_lora_and_convert_equals_merge_then_convert(device, rank, scale):
    a = _Model(4, 512, seed=2).to(device)
    b = _Model(4, 512, seed=2).to(device)
    state = _lora_state(a, rank, seed=3)
    merged_a, converted_a = LR.merge_lora_and_convert(a, state, scale, min_width=256, skip_end_blocks=1)
    merged_b = LR.merge_lora_state(b, state, scale)
    converted_b = vdn_fp8.convert_linear_to_fp8(b, min_width=256, skip_end_blocks=1)
    torch.cuda.synchronize()
    assert merged_a == merged_b == len(state) // 2 and converted_a == converted_b
    for (na, ma), (nb, mb) in zip(a.named_modules(), b.named_modules()):
        assert na == nb and type(ma) is type(mb)
        if isinstance(ma, vdn_fp8.Fp8Linear):
            assert torch.equal(ma.weight_fp8.view(torch.uint8), mb.weight_fp8.view(torch.uint8)), na
            assert torch.equal(ma.weight_scale, mb.weight_scale), na
        elif isinstance(ma, nn.Linear):
            assert torch.equal(ma.weight, mb.weight), na      # pairs on kept-bf16 Linears merged in place
