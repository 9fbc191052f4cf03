"""Adapter files end to end on the GPU, and LoRA targets outside the kernel's domain.

An original-layout adapter (fused `qkv_proj`, `mlp.fc1` with its SwiGLU halves packed
[gate; value], `mlp.fc2`, `attn.out_proj`, peft `.default.` infixes, alpha in the file
metadata) is written to a safetensors file, read by `load_external_lora`
(lora.py:97-117), and folded into a small DiT-named model by `merge_lora_and_convert`.
The fp8 codes and scales of every converted projection must equal the oracle's
`quantize_weight(lora_merge(W, A, B, alpha / rank))` on factors that the test translates
itself from the file's tensors (qkv B rows split in thirds, fc1 B halves swapped,
lora.py:32-66).

The factors are small multiples of powers of two, so B @ A is exact in binary32 under any
summation order: the merged weight -- and therefore every code -- has one right answer,
and the comparison is bit-exact. Random-valued factors are covered by test_gpu_requant.py
(merged weight within one bf16 ulp, codes exact given it).

Targets and adapters the fused kernel does not take -- rank > 128, fp32 / fp16 target
weights (the hybrid attention's parameters before their bf16 cast, assemble.py:124 vs
:148-151), non-contiguous views and weights in host memory -- are merged with the
reference's own update (lora.py:91-92) and checked against the float64 restatement."""
import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle as O
import vdn_fp8
from conftest import bits, codes, from_bits
from vdn_fp8 import lora as LR

pytestmark = pytest.mark.gpu

H = 256          # hidden width of the toy model (K of every projection)


def _exact_factor(rng, shape, denom):
    """Integers in [-8, 8] / denom: any sum of up to 2^10 products of two such factors is
    exact in binary32."""
    return (rng.integers(-8, 9, size=shape).astype(np.float32) / denom)


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.to_q = nn.Linear(H, H, dtype=torch.bfloat16)
        self.to_k = nn.Linear(H, H, dtype=torch.bfloat16)
        self.to_v = nn.Linear(H, H, dtype=torch.bfloat16)
        self.to_out = nn.ModuleList([nn.Linear(H, H, dtype=torch.bfloat16)])


class _Hybrid(nn.Module):
    """A hybrid-attention wrapper: the dense attention one level down (`attn.orig.*`)."""
    def __init__(self):
        super().__init__()
        self.orig = _Attn()


class _FF(nn.Module):
    def __init__(self):
        super().__init__()
        self.net = nn.ModuleList([nn.Module(), nn.Identity(), nn.Linear(H, H, dtype=torch.bfloat16)])
        self.net[0].proj = nn.Linear(H, 2 * H, dtype=torch.bfloat16)


class _Block(nn.Module):
    def __init__(self, hybrid):
        super().__init__()
        self.attn = _Hybrid() if hybrid else _Attn()
        self.ff = _FF()


class _DiT(nn.Module):
    def __init__(self, seed, blocks=3):
        super().__init__()
        self.transformer_blocks = nn.ModuleList(_Block(hybrid=(i == 1)) for i in range(blocks))
        g = torch.Generator().manual_seed(seed)
        with torch.no_grad():
            for p in self.parameters():
                p.copy_((0.02 * torch.randn(p.shape, generator=g)).to(p.dtype))


def _original_layout_file(path, rank, alpha, dtype, seed, blocks=3):
    """Writes an adapter in the original checkpoint layout; returns the numpy factors per
    original module name (A [r, K], B as stored)."""
    from safetensors.torch import save_file
    rng = np.random.default_rng(seed)
    tensors, raw = {}, {}
    for i in range(blocks):
        for mod, rows in (("attn.qkv_proj", 3 * H), ("mlp.fc1", 2 * H), ("mlp.fc2", H), ("attn.out_proj", H)):
            a = _exact_factor(rng, (rank, H), 32.0)
            b = _exact_factor(rng, (rows, rank), 64.0)
            stem = f"diffusion_model.blocks.{i}.{mod}"
            infix = ".default" if i % 2 == 0 else ""          # peft's adapter infix on some keys
            tensors[f"{stem}.lora_A{infix}.weight"] = torch.from_numpy(a).to(dtype)
            tensors[f"{stem}.lora_B{infix}.weight"] = torch.from_numpy(b).to(dtype)
            raw[(i, mod)] = (a, b)
    save_file(tensors, str(path), metadata={"alpha": str(alpha)})
    return raw


def _expected_pairs(raw, blocks=3):
    """The file's pairs on diffusers module names, translated here independently of
    vdn_fp8.lora: qkv B split into (q, k, v) thirds sharing A; fc1 B [gate; value] ->
    [value; gate]."""
    out = {}
    for i in range(blocks):
        a, b = raw[(i, "attn.qkv_proj")]
        for j, proj in enumerate(("to_q", "to_k", "to_v")):
            out[(i, proj)] = (a, b[j * H:(j + 1) * H])
        a, b = raw[(i, "mlp.fc1")]
        out[(i, "ff.net.0.proj")] = (a, np.concatenate([b[H:], b[:H]], axis=0))
        out[(i, "ff.net.2")] = raw[(i, "mlp.fc2")]
        out[(i, "to_out.0")] = raw[(i, "attn.out_proj")]
    return out


def _module(model, i, name):
    blk = model.transformer_blocks[i]
    attn = blk.attn.orig if hasattr(blk.attn, "orig") else blk.attn
    return {"to_q": lambda: attn.to_q, "to_k": lambda: attn.to_k, "to_v": lambda: attn.to_v,
            "to_out.0": lambda: attn.to_out[0], "ff.net.0.proj": lambda: blk.ff.net[0].proj,
            "ff.net.2": lambda: blk.ff.net[2]}[name]()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_original_layout_adapter_end_to_end(device, tmp_path, dtype):
    rank, alpha = 16, 32.0                       # scale 2.0: exact
    path = tmp_path / "adapter.safetensors"
    raw = _original_layout_file(path, rank, alpha, dtype, seed=11)
    state, scale, ranks = LR.load_external_lora(str(path))
    assert ranks == [rank] and scale == alpha / rank
    assert not any(".default." in k for k in state)

    model = _DiT(seed=5)
    base = {(i, n): bits(_module(model, i, n).weight) for i in range(3)
            for n in ("to_q", "to_k", "to_v", "to_out.0", "ff.net.0.proj", "ff.net.2")}
    model = model.to(device)
    merged, converted = LR.merge_lora_and_convert(model, state, scale, min_width=H, skip_end_blocks=0)
    torch.cuda.synchronize()
    assert merged == len(state) // 2 == 3 * 6
    assert converted == 3 * 6
    for (i, name), (a, b) in _expected_pairs(raw).items():
        lin = _module(model, i, name)
        assert isinstance(lin, vdn_fp8.Fp8Linear), (i, name)
        # the oracle's merge of the file's factors (as stored: bf16 or binary32, both exact)
        want_w = O.lora_merge(base[(i, name)], O.bf16_encode(a), O.bf16_encode(b), scale)
        wq, ws = O.quantize_weight(want_w)
        got_q, got_s = codes(lin.weight_fp8), lin.weight_scale.cpu().numpy().ravel()
        assert np.array_equal(got_s.view(np.uint32), ws.view(np.uint32)), (i, name)
        assert np.array_equal(got_q, wq), (i, name, int((got_q != wq).sum()))


def test_diffusers_named_adapter_with_rerooting(device, tmp_path):
    """peft names against the dense model; block 1 is hybrid, so its targets resolve
    through `.attn.orig.` (lora.py:69-77); no alpha in the metadata -> scale 1.0."""
    from safetensors.torch import save_file
    rng = np.random.default_rng(3)
    tensors, pairs = {}, {}
    for i in range(3):
        for proj in ("to_q", "to_v"):
            a, b = _exact_factor(rng, (8, H), 16.0), _exact_factor(rng, (H, 8), 32.0)
            tensors[f"transformer_blocks.{i}.attn.{proj}.lora_A.default.weight"] = torch.from_numpy(a).to(torch.bfloat16)
            tensors[f"transformer_blocks.{i}.attn.{proj}.lora_B.default.weight"] = torch.from_numpy(b).to(torch.bfloat16)
            pairs[(i, proj)] = (a, b)
    save_file(tensors, str(tmp_path / "peft.safetensors"))
    state, scale, ranks = LR.load_external_lora(str(tmp_path / "peft.safetensors"))
    assert scale == 1.0 and ranks == [8]
    model = _DiT(seed=6)
    base = {k: bits(_module(model, *k).weight) for k in pairs}
    model = model.to(device)
    assert LR.merge_lora_state(model, state, scale) == 6
    torch.cuda.synchronize()
    for k, (a, b) in pairs.items():
        want = O.lora_merge(base[k], O.bf16_encode(a), O.bf16_encode(b), 1.0)
        assert np.array_equal(bits(_module(model, *k).weight), want), k


def _exact_case(rng, N, K, r):
    w = O.bf16_encode(rng.standard_normal((N, K), dtype=np.float32) * 0.02)
    return w, _exact_factor(rng, (r, K), 32.0), _exact_factor(rng, (N, r), 64.0)


@pytest.mark.parametrize("rank", [129, 256])
def test_bf16_adapter_above_the_kernel_rank(device, rank):
    """bf16 factors of rank > 128 take the reference's update (fp32 product, bf16 add)
    and then the requantize kernel: codes and scales equal the oracle's."""
    rng = np.random.default_rng(rank)
    w, a, b = _exact_case(rng, 96, 512, rank)
    aw, bw = from_bits(O.bf16_encode(a), device), from_bits(O.bf16_encode(b), device)
    q, s = vdn_fp8.requantize_weight(from_bits(w, device), lora=(aw, bw, 0.5))
    want_w = O.lora_merge(w, O.bf16_encode(a), O.bf16_encode(b), 0.5)
    wq, ws = O.quantize_weight(want_w)
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy().view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(codes(q), wq)
    # the in-place merge of the same adapter
    t = from_bits(w, device)
    LR.merge_into(t, aw, bw, 0.5)
    assert np.array_equal(bits(t), want_w)


def _f64_merge(w, a, b, scale, dtype):
    """float64 restatement of the reference update for a target of `dtype`: the product is
    exact here, so fp32(delta) is that value rounded once; then cast and add in dtype."""
    delta = (b.astype(np.float64) @ a.astype(np.float64)) * scale
    d = torch.from_numpy(delta.astype(np.float32)).to(dtype)
    return (torch.from_numpy(w).to(dtype) + d)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("where", ["gpu", "gpu_strided", "host"])
def test_merge_into_any_target(device, dtype, where):
    rng = np.random.default_rng(hash((str(dtype), where)) % 1000)
    N, K, r = 80, 384, 24
    w64 = rng.standard_normal((N, K)).astype(np.float32) * 0.02
    a, b = _exact_factor(rng, (r, K), 32.0), _exact_factor(rng, (N, r), 64.0)
    want = _f64_merge(w64, a, b, 1.5, dtype)
    wt = torch.from_numpy(w64).to(dtype)
    if where == "gpu":
        target = wt.to(device)
    elif where == "gpu_strided":
        big = torch.zeros(N, 2 * K, dtype=dtype, device=device)
        big[:, ::2] = wt.to(device)
        target = big[:, ::2]                      # a non-contiguous [N, K] view
    else:
        target = wt.clone()
    fa, fb = torch.from_numpy(a).to(torch.bfloat16), torch.from_numpy(b).to(torch.bfloat16)
    if where != "host":
        fa, fb = fa.to(device), fb.to(device)
    out = LR.merge_into(target, fa, fb, 1.5)
    assert out is target
    if where == "gpu_strided":
        assert torch.all(big[:, 1::2] == 0)       # the view's neighbours untouched
    got = target.cpu()
    assert got.dtype == dtype
    assert torch.equal(got, want), (dtype, where, (got != want).sum().item())
