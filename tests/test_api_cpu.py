"""Host-side behaviour of the vdn_fp8 module API without a GPU: the reference's
names and constants, its error types for CPU / malformed input, the dispatch on
capability, and the conversion pass's target selection (fp8_linear.py:60-63,
102-107, 141-147, 286-323)."""
import pytest
import torch
import torch.nn as nn

import vdn_fp8
from vdn_fp8 import fp8_linear as F


def test_reference_constants():
    assert vdn_fp8.FP8_DTYPE is torch.float8_e4m3fn
    assert vdn_fp8._FP8_MAX == 448.0
    assert vdn_fp8.MIN_WIDTH == 4096 and vdn_fp8.SKIP_END_BLOCKS == 4


def test_quantizers_refuse_cpu_and_bad_rank():
    x = torch.zeros(4, 8, dtype=torch.bfloat16)
    for fn in (vdn_fp8.quantize_rows, vdn_fp8.swiglu_quantize, vdn_fp8.quantize_activation):
        with pytest.raises(ValueError, match="GPU"):
            fn(x)
    with pytest.raises(ValueError):
        F._rows(torch.zeros(2, 3, 4, dtype=torch.bfloat16).cuda() if torch.cuda.is_available() else
                _FakeCuda(torch.zeros(2, 3, 4)))


class _FakeCuda:
    """Stands in for a GPU tensor only as far as the shape check reads it."""
    def __init__(self, t):
        self._t = t
        self.is_cuda = True

    def dim(self):
        return self._t.dim()

    @property
    def shape(self):
        return self._t.shape


def test_requantize_refuses_cpu_weight():
    with pytest.raises(ValueError, match="GPU"):
        vdn_fp8.requantize_weight(torch.zeros(8, 8, dtype=torch.bfloat16))


def test_fp8_linear_refuses_cpu_linear():
    with pytest.raises(ValueError):
        vdn_fp8.Fp8Linear(nn.Linear(64, 64, dtype=torch.bfloat16))


def test_per_tensor_gemm_is_false_without_sm100():
    F._PER_TENSOR = None
    assert vdn_fp8.per_tensor_gemm() is False


def test_quantize_rows_reference_is_the_eager_spelling():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8, 64, generator=g).to(torch.bfloat16)
    q, s = vdn_fp8.quantize_rows_reference(x)
    want_s = (x.float().abs().amax(dim=1, keepdim=True) / 448.0).clamp_min(1e-12)
    assert torch.equal(s, want_s)
    assert torch.equal(q.view(torch.uint8), (x.float() / want_s).to(torch.float8_e4m3fn).view(torch.uint8))


class Block(nn.Module):
    def __init__(self, width):
        super().__init__()
        self.attn = nn.Module()
        self.attn.to_q = nn.Linear(width, width)
        self.ff = nn.Linear(width, 2 * width)
        self.small = nn.Linear(width, width // 2)


class Model(nn.Module):
    def __init__(self, n, width):
        super().__init__()
        self.transformer_blocks = nn.ModuleList(Block(width) for _ in range(n))
        self.proj_out = nn.Linear(width, width)


def test_blocks_to_skip_selects_first_and_last():
    m = Model(6, 16)
    keep = F._blocks_to_skip(m, 2)
    for i, blk in enumerate(m.transformer_blocks):
        inside = id(blk.attn.to_q) in keep
        assert inside == (i < 2 or i >= 4)
    assert F._blocks_to_skip(m, 0) == set()


def test_convert_selects_wide_linears(monkeypatch):
    """The conversion pass swaps exactly the Linears >= min_width on both sides outside
    the skipped blocks, one at a time, and returns the count (fp8_linear.py:298-323)."""
    made = []

    class Stub(nn.Module):
        def __init__(self, linear):
            super().__init__()
            made.append(linear)

    monkeypatch.setattr(F, "Fp8Linear", Stub)
    m = Model(6, 32)
    n = F.convert_linear_to_fp8(m, min_width=32, skip_end_blocks=1)
    # blocks 1..4: to_q (32x32) and ff (32->64) each; proj_out; small (16 out) never
    assert n == 4 * 2 + 1 == len(made)
    assert isinstance(m.transformer_blocks[0].attn.to_q, nn.Linear)
    assert isinstance(m.transformer_blocks[2].ff, Stub)
    assert isinstance(m.transformer_blocks[2].small, nn.Linear)


def test_translate_original_layout():
    from vdn_fp8.lora import _translate_original_layout
    a = torch.randn(4, 10)
    b = torch.randn(30, 4)
    fc1_b = torch.cat([torch.full((6, 4), 1.0), torch.full((6, 4), 2.0)])   # [gate; value]
    state = {
        "diffusion_model.blocks.3.attn.qkv_proj.lora_A.weight": a,
        "diffusion_model.blocks.3.attn.qkv_proj.lora_B.weight": b,
        "blocks.3.mlp.fc1.lora_B.weight": fc1_b,
        "blocks.3.attn.out_proj.lora_A.weight": a,
    }
    out = _translate_original_layout(state)
    for i, p in enumerate(("to_q", "to_k", "to_v")):
        assert torch.equal(out[f"transformer_blocks.3.attn.{p}.lora_A.weight"], a)
        assert torch.equal(out[f"transformer_blocks.3.attn.{p}.lora_B.weight"], b[10 * i:10 * (i + 1)])
    swapped = out["transformer_blocks.3.ff.net.0.proj.lora_B.weight"]
    assert torch.all(swapped[:6] == 2.0) and torch.all(swapped[6:] == 1.0)     # [value; gate]
    assert "transformer_blocks.3.attn.to_out.0.lora_A.weight" in out
    plain = {"transformer_blocks.0.attn.to_q.lora_A.weight": a}
    assert _translate_original_layout(plain) is plain


def test_resolve_reroots_through_attn_orig():
    from vdn_fp8.lora import _resolve
    params = {"transformer_blocks.0.attn.orig.to_q.weight": 1}
    assert _resolve(params, "transformer_blocks.0.attn.to_q.weight") == 1
    with pytest.raises(KeyError):
        _resolve(params, "transformer_blocks.0.attn.to_k.weight")


def test_load_external_lora_alpha(tmp_path):
    from safetensors.torch import save_file
    from vdn_fp8.lora import load_external_lora
    t = {"transformer_blocks.0.attn.to_q.lora_A.default.weight": torch.zeros(8, 16),
         "transformer_blocks.0.attn.to_q.lora_B.default.weight": torch.zeros(16, 8)}
    p = tmp_path / "a.safetensors"
    save_file(t, str(p), metadata={"alpha": "4"})
    state, scale, ranks = load_external_lora(str(p))
    assert scale == 0.5 and ranks == [8]
    assert "transformer_blocks.0.attn.to_q.lora_A.weight" in state
    save_file(t, str(p))
    assert load_external_lora(str(p))[1] == 1.0
    assert load_external_lora(str(p), alpha=16)[1] == 2.0


def test_swiglu_one_rounding_against_float64():
    """The bf16 feed-forward's SwiGLU rounds a * silu(gate) once, as the reference's
    compiled body (fused_block.py:88); the eager body rounds silu first. Against
    a * g / (1 + exp(-g)) in float64 rounded once: within one bf16 step everywhere and
    identical almost everywhere, while the eager body differs far more often."""
    import numpy as np
    from vdn_fp8 import fused_block as FB
    g = torch.Generator().manual_seed(11)
    h = (torch.randn(256, 2 * 512, generator=g) * torch.logspace(-2, 1, 2 * 512)).to(torch.bfloat16)
    got = FB._swiglu_one_rounding(h).float().numpy().astype(np.float64)
    eager = FB._swiglu_ref(h).float().numpy().astype(np.float64)
    a, gate = (t.float().numpy().astype(np.float64) for t in h.chunk(2, dim=-1))
    exact = a * gate / (1.0 + np.exp(-gate))
    want = torch.from_numpy(exact).to(torch.bfloat16).float().numpy().astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
    assert np.all(np.abs(got - want) <= ulp)
    same, same_eager = np.mean(got == want), np.mean(eager == want)
    assert same >= 0.995, same
    assert same_eager < same, (same_eager, same)


def test_host_linear_needs_a_gpu_here():
    """Fp8Linear of a host-resident Linear is requantized on the GPU and its buffers return
    to the Linear's device; without a GPU it raises (no CPU fallback)."""
    import torch
    import vdn_fp8
    if torch.cuda.is_available():
        pytest.skip("this container's check: no GPU")
    lin = torch.nn.Linear(64, 32, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="needs a GPU"):
        vdn_fp8.Fp8Linear(lin)


def test_index_checks_opt_in():
    """Out-of-range table indices are clamped by the kernels; with checks enabled the host
    raises IndexError first, as the reference's index_select does."""
    import torch
    import vdn_fp8
    from vdn_fp8.fp8_linear import check_index_range
    idx = torch.tensor([0, 3, 5])
    prev = vdn_fp8.set_index_checks(False)
    try:
        check_index_range(idx, 5, "gate_index")            # off: no check
        vdn_fp8.set_index_checks(True)
        check_index_range(torch.tensor([0, 4]), 5, "gate_index")
        with pytest.raises(IndexError, match="out of range"):
            check_index_range(idx, 5, "gate_index")
        with pytest.raises(IndexError):
            check_index_range(torch.tensor([-1]), 5, "indices")
    finally:
        vdn_fp8.set_index_checks(prev)
