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


def test_host_resident_linear(device):
    """A Linear still in host memory: requantized on the GPU, buffers returned to the
    host (where the reference's eager branch would leave them), identical to the GPU-built
    module's; moved to the GPU, it runs as usual."""
    torch.manual_seed(3)
    lin = torch.nn.Linear(512, 256, dtype=torch.bfloat16)
    f_host = vdn_fp8.Fp8Linear(lin)
    assert f_host.weight_fp8.device.type == "cpu" and f_host.weight_scale.device.type == "cpu"
    f_dev = vdn_fp8.Fp8Linear(_copy_to(lin, device))
    assert torch.equal(f_host.weight_fp8.view(torch.uint8), f_dev.weight_fp8.view(torch.uint8).cpu())
    assert torch.equal(f_host.weight_scale, f_dev.weight_scale.cpu())
    f_host = f_host.to(device)
    x = torch.randn(64, 512, dtype=torch.bfloat16, device=device)
    assert torch.equal(f_host(x).view(torch.int16), f_dev(x).view(torch.int16))


def _copy_to(lin, device):
    out = torch.nn.Linear(lin.in_features, lin.out_features, dtype=torch.bfloat16, device=device)
    with torch.no_grad():
        out.weight.copy_(lin.weight)
        out.bias.copy_(lin.bias)
    return out


def test_index_checks_raise_before_launch(device):
    """With index checks on, an out-of-range gate or modulation index raises IndexError (as
    index_select does) before anything runs; off, the kernels clamp it."""
    from vdn_fp8 import fused_block as FB
    torch.manual_seed(4)
    lin = vdn_fp8.Fp8Linear(_copy_to(torch.nn.Linear(256, 256, dtype=torch.bfloat16), device))
    qx, sx = vdn_fp8.quantize_rows(torch.randn(32, 256, dtype=torch.bfloat16, device=device))
    gate = torch.rand(3, 256, device=device).to(torch.bfloat16)
    bad = torch.tensor([0, 1, 2, 3] * 8, dtype=torch.int32, device=device)
    x = torch.randn(32, 256, dtype=torch.bfloat16, device=device)
    prev = vdn_fp8.set_index_checks(True)
    try:
        with pytest.raises(IndexError):
            lin.forward_quantized(qx, sx, epilogue="gate", gate=gate, gate_index=bad)
        with pytest.raises(IndexError):
            FB.post(x, gate, bad, x)
        with pytest.raises(IndexError):
            FB.pre(x, None, 1e-6, gate, gate, bad)
        ok = bad.clamp(0, 2)
        lin.forward_quantized(qx, sx, epilogue="gate", gate=gate, gate_index=ok)
    finally:
        vdn_fp8.set_index_checks(prev)
    clamped = lin.forward_quantized(qx, sx, epilogue="gate", gate=gate, gate_index=bad)
    want = lin.forward_quantized(qx, sx, epilogue="gate", gate=gate, gate_index=bad.clamp(0, 2))
    torch.cuda.synchronize()
    assert torch.equal(clamped.view(torch.int16), want.view(torch.int16))
