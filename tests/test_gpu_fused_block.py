"""GPU tests of the block-level pieces (vdn_fp8.fused_block): `post` (the gated residual
add, vdn_fp8_gated_residual) bit-exact against the oracle's restatement of the compiled
`post` (fused_block.py:47-49); `pre` (the pre-norm alone) within one bf16 ulp of the
oracle's float64 RMSNorm + AdaLN affine; and the forwards -- `fast_ff_forward`
(fused_block.py:73-90) and `fast_block_forward` (:93-111) on a small block of fp8 linears --
against the unfused composition of the same kernels (bitwise: the fusions move roundings
nowhere) and, for the feed-forward, against the oracle's chain."""
import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle as O
import vdn_fp8
from conftest import bits, from_bits
from vdn_fp8 import fused_block as FB

pytestmark = pytest.mark.gpu


def _ulp(v):
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


@pytest.mark.parametrize("M,N,T", [(1, 8, 1), (37, 5120, 6), (300, 2056, 2), (4, 16392, 3)])
def test_post_bit_exact(device, M, N, T):
    print(f"post M={M} N={N} T={T}", flush=True)
    rng = np.random.default_rng(M + N + T)
    r = O.bf16_encode(rng.standard_normal((M, N), dtype=np.float32))
    b = O.bf16_encode(rng.standard_normal((M, N), dtype=np.float32) * 3)
    g = O.bf16_encode(rng.uniform(0, 2, (T, N)).astype(np.float32))
    idx = rng.integers(-1, T + 1, M)                 # out-of-range rows are clamped
    out = FB.post(from_bits(r, device), from_bits(g, device), torch.from_numpy(idx).to(device), from_bits(b, device))
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), O.gated_residual(r, g, idx, b))


def test_post_broadcast_gate_and_3d(device):
    rng = np.random.default_rng(5)
    r = O.bf16_encode(rng.standard_normal((1, 40, 256), dtype=np.float32))
    b = O.bf16_encode(rng.standard_normal((1, 40, 256), dtype=np.float32))
    g = O.bf16_encode(rng.uniform(0, 2, 256).astype(np.float32))
    out = FB.post(from_bits(r, device), from_bits(g, device), None, from_bits(b, device))
    torch.cuda.synchronize()
    assert out.shape == (1, 40, 256)
    assert np.array_equal(bits(out).reshape(40, 256), O.gated_residual(r.reshape(40, 256), g, None, b.reshape(40, 256)))


def test_pre_within_one_ulp(device):
    rng = np.random.default_rng(6)
    M, K, T = 70, 5120, 4
    x = O.bf16_encode(rng.standard_normal((M, K), dtype=np.float32))
    w = O.bf16_encode(1 + 0.1 * rng.standard_normal(K, dtype=np.float32))
    sc = O.bf16_encode(0.2 * rng.standard_normal((T, K), dtype=np.float32))
    sh = O.bf16_encode(0.2 * rng.standard_normal((T, K), dtype=np.float32))
    idx = rng.integers(0, T, M)
    out = FB.pre(from_bits(x, device), from_bits(w, device), 1e-6, from_bits(sc, device), from_bits(sh, device),
                 torch.from_numpy(idx).to(device))
    torch.cuda.synchronize()
    want, terms = O.norm_rows(x, w, 1e-6, sc, sh, idx, return_terms=True)
    gv, wv = O.bf16_decode(bits(out)).astype(np.float64), O.bf16_decode(want).astype(np.float64)
    assert np.all(np.abs(gv - wv) <= _ulp(np.maximum(np.abs(wv), terms)))
    assert np.mean(bits(out) == want) >= 0.995
    # pre then quantize_rows == the fused pre_quantize, bit for bit
    q1, s1 = vdn_fp8.quantize_rows(out)
    q2, s2 = FB.pre_quantize(from_bits(x, device), from_bits(w, device), 1e-6, from_bits(sc, device),
                             from_bits(sh, device), torch.from_numpy(idx).to(device))
    torch.cuda.synchronize()
    assert torch.equal(q1.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s1, s2)


@pytest.mark.parametrize("M,K", [(4000, 8192), (3200, 13824), (3200, 16384)])
def test_pre_wide_rows_many_per_block(device, M, K):
    """The norm-only pre-norm on rows that two or four waves share, with several rows per
    workgroup (M above the resident wave groups): each row's partial sums of squares must
    meet only its own row's, with one barrier per row in this form."""
    print(f"pre wide M={M} K={K}", flush=True)
    rng = np.random.default_rng(M + K)
    T = 3
    # rows of very different magnitude, so a sum of squares taken from a neighbouring
    # row would change the normed values by far more than a rounding
    x = O.bf16_encode(rng.standard_normal((M, K), dtype=np.float32) *
                      np.exp2(rng.integers(-6, 7, (M, 1))).astype(np.float32))
    w = O.bf16_encode(1 + 0.1 * rng.standard_normal(K, dtype=np.float32))
    sc = O.bf16_encode(0.2 * rng.standard_normal((T, K), dtype=np.float32))
    sh = O.bf16_encode(0.2 * rng.standard_normal((T, K), dtype=np.float32))
    idx = np.arange(M) * T // M
    out = FB.pre(from_bits(x, device), from_bits(w, device), 1e-6, from_bits(sc, device), from_bits(sh, device),
                 torch.from_numpy(idx).to(device))
    torch.cuda.synchronize()
    want, terms = O.norm_rows(x, w, 1e-6, sc, sh, idx, return_terms=True)
    gv, wv = O.bf16_decode(bits(out)).astype(np.float64), O.bf16_decode(want).astype(np.float64)
    assert np.all(np.abs(gv - wv) <= _ulp(np.maximum(np.abs(wv), terms)))
    assert np.mean(bits(out) == want) >= 0.995
    # the fused form (two barriers per row) gives the same normed bits
    _, _, n2 = FB.pre_quantize(from_bits(x, device), from_bits(w, device), 1e-6, from_bits(sc, device),
                               from_bits(sh, device), torch.from_numpy(idx).to(device), return_normed=True)
    torch.cuda.synchronize()
    assert np.array_equal(bits(n2), bits(out))


# --------------------------------------------------------------------------------------
# A small block with the reference block's structure (diffusers' MiniMaxH3 block as the
# reference's fast_block_forward uses it): adaln_proj -> 6 chunks, norm1/norm2 RMSNorm,
# attn(normed, rotary_emb, mask), ff.net = [SwiGLU(proj), Dropout, down].
# --------------------------------------------------------------------------------------

class _SwiGLU(nn.Module):
    def __init__(self, proj):
        super().__init__()
        self.proj = proj


class _FF(nn.Module):
    def __init__(self, proj, down):
        super().__init__()
        self.net = nn.ModuleList([_SwiGLU(proj), nn.Dropout(0.0), down])

    def forward(self, x):                       # diffusers' FeedForward: the net in order
        swiglu, drop, down = self.net
        return down(drop(FB._swiglu_ref(swiglu.proj(x))))


class _AdaLN(nn.Module):
    def __init__(self, table):
        super().__init__()
        self.table = table            # [6, T, C]

    def forward(self, temb):
        return tuple(self.table[i] for i in range(6))


class _Attn(nn.Module):
    def __init__(self, lin):
        super().__init__()
        self.lin = lin

    def forward(self, x, rotary_emb=None, attention_mask=None):
        return self.lin(x)


class _Block(nn.Module):
    def __init__(self, C, I, T, device, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        def lin(o, i, bias):
            l = nn.Linear(i, o, bias=bias, dtype=torch.bfloat16)
            with torch.no_grad():
                l.weight.copy_((0.02 * torch.randn(o, i, generator=g)).to(torch.bfloat16))
                if bias:
                    l.bias.copy_((0.01 * torch.randn(o, generator=g)).to(torch.bfloat16))
            return l
        tab = torch.empty(6, T, C)
        tab[[0, 3]] = 0.1 * torch.randn(2, T, C, generator=g)          # shifts
        tab[[1, 4]] = 0.2 * torch.randn(2, T, C, generator=g)          # scales
        tab[[2, 5]] = 2 * torch.rand(2, T, C, generator=g)             # gates
        self.adaln_proj = _AdaLN(tab.to(torch.bfloat16).to(device))
        self.norm1 = nn.RMSNorm(C, eps=1e-6, dtype=torch.bfloat16)
        self.norm2 = nn.RMSNorm(C, eps=1e-6, dtype=torch.bfloat16)
        with torch.no_grad():
            self.norm1.weight.copy_((1 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16))
            self.norm2.weight.copy_((1 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16))
        self.attn = _Attn(vdn_fp8.Fp8Linear(lin(C, C, False).to(device)))
        self.ff = _FF(vdn_fp8.Fp8Linear(lin(2 * I, C, True).to(device)),
                      vdn_fp8.Fp8Linear(lin(C, I, True).to(device)))
        self.to(device)


def _unfused_block(blk, hidden, temb, idx):
    """The reference's fast_block_forward order with every stretch a separate kernel."""
    s1, c1, g1, s2, c2, g2 = blk.adaln_proj(temb)
    normed = FB.pre(hidden, blk.norm1.weight, blk.norm1.eps, c1, s1, idx)
    hidden = FB.post(hidden, g1, idx, blk.attn(normed, None, None))
    normed = FB.pre(hidden, blk.norm2.weight, blk.norm2.eps, c2, s2, idx)
    return FB.post(hidden, g2, idx, FB.fast_ff_forward(blk.ff, normed))


@pytest.mark.parametrize("M,C,I,T", [(64, 4096, 2048, 3), (300, 5120, 4096, 2)])
def test_fast_block_forward_equals_unfused(device, M, C, I, T):
    print(f"fast_block_forward M={M} C={C} I={I}", flush=True)
    blk = _Block(C, I, T, device, seed=M + C)
    g = torch.Generator().manual_seed(7)
    hidden = torch.randn(1, M, C, generator=g).to(torch.bfloat16).to(device)
    idx = torch.randint(0, T, (M,), generator=g).to(device)
    with torch.no_grad():
        fused = FB.fast_block_forward(blk, hidden, None, idx, None)
        ref = _unfused_block(blk, hidden, None, idx)
    torch.cuda.synchronize()
    assert fused.shape == hidden.shape
    assert torch.equal(fused, ref)


def test_fast_ff_forward_matches_oracle_chain(device):
    """fast_ff_forward is exactly quantize -> projection GEMM (+bias) -> SwiGLU + quantize
    -> down GEMM (+bias) through the public entry points, and that chain stays close to
    the oracle's own chain (each stage's oracle fed the previous stage's oracle output).
    Not identical: ~1% of the projection's bf16 outputs sit one rounding step away from
    the oracle's (the fp8 MFMA accumulates below binary32 precision), a few SwiGLU codes
    then flip by one e4m3 step, and a down-projection output summing over such an input
    rounds differently -- so the bound is on rel-L2 and on most values being identical."""
    M, C, I = 96, 4096, 2048
    blk = _Block(C, I, 2, device, seed=11)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(M, C, generator=g).to(torch.bfloat16).to(device)
    proj, down = blk.ff.net[0].proj, blk.ff.net[2]
    with torch.no_grad():
        out = FB.fast_ff_forward(blk.ff, x)
        manual = down.forward_quantized(*vdn_fp8.swiglu_quantize(proj.forward_quantized(*vdn_fp8.quantize_rows(x))))
    torch.cuda.synchronize()
    assert torch.equal(out, manual)
    qx, sx = O.quantize_rows(bits(x))
    h = O.dequant_linear(qx, sx, proj.weight_fp8.view(torch.uint8).cpu().numpy(),
                         proj.weight_scale.cpu().numpy().ravel(), bias=bits(proj.bias))
    qy, sy = O.swiglu_quantize_rows(O.bf16_encode(h.astype(np.float32)))
    want = O.dequant_linear(qy, sy, down.weight_fp8.view(torch.uint8).cpu().numpy(),
                            down.weight_scale.cpu().numpy().ravel(), bias=bits(down.bias))
    got = O.bf16_decode(bits(out)).astype(np.float64)
    err = O.rel_l2(got, want)
    print(f"fast_ff_forward vs oracle chain: rel_l2 {err:.2e}, identical {np.mean(got == want):.3f}", flush=True)
    assert err <= 1e-2
    assert np.mean(got == want) >= 0.75


def test_fast_ff_forward_bf16_rounds_once(device):
    """A feed-forward whose linears stay bf16: the projection, the SwiGLU rounded once
    (the reference's compiled body, fused_block.py:88; its numerics are pinned against
    float64 in the CPU tests), then the down projection."""
    C, I = 256, 128
    g = torch.Generator().manual_seed(4)
    proj = nn.Linear(C, 2 * I, dtype=torch.bfloat16).to(device)
    down = nn.Linear(I, C, dtype=torch.bfloat16).to(device)
    ff = _FF(proj, down)
    x = torch.randn(2, 20, C, generator=g).to(torch.bfloat16).to(device)
    with torch.no_grad():
        got = FB.fast_ff_forward(ff, x)
        want = down(FB._swiglu_one_rounding(proj(x.reshape(-1, C)))).reshape(2, 20, C)
        eager = down(FB._swiglu_ref(proj(x.reshape(-1, C)))).reshape(2, 20, C)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    print(f"bf16 feed-forward: {torch.mean((got != eager).float()).item():.3f} of outputs differ from the "
          f"eager SwiGLU's", flush=True)


def test_fast_block_forward_bf16_ff(device):
    """A block whose feed-forward stays bf16 (no Fp8Linear): pre, the module, post."""
    M, C, I, T = 48, 512, 256, 2
    blk = _Block(C, I, T, device, seed=3)
    g = torch.Generator().manual_seed(9)
    proj = nn.Linear(C, 2 * I, dtype=torch.bfloat16).to(device)
    down = nn.Linear(I, C, dtype=torch.bfloat16).to(device)
    blk.ff = _FF(proj, down)
    hidden = torch.randn(M, C, generator=g).to(torch.bfloat16).to(device)
    idx = torch.randint(0, T, (M,), generator=g).to(device)
    with torch.no_grad():
        got = FB.fast_block_forward(blk, hidden, None, idx, None)
        s1, c1, g1, s2, c2, g2 = blk.adaln_proj(None)
        h = FB.post(hidden, g1, idx, blk.attn(FB.pre(hidden, blk.norm1.weight, blk.norm1.eps, c1, s1, idx)))
        n2 = FB.pre(h, blk.norm2.weight, blk.norm2.eps, c2, s2, idx)
        want = FB.post(h, g2, idx, down(FB._swiglu_ref(proj(n2))))
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_post_large_output(device):
    """An output beyond the last-level cache (>= 256 MiB: non-temporal stores) equals the
    same rows done in small batches (cached stores), and sampled rows match the oracle."""
    M, N, T = 32760, 5120, 3
    print(f"post large M={M} N={N}", flush=True)
    g = torch.Generator(device=device).manual_seed(8)
    r = torch.randn(M, N, device=device, generator=g).to(torch.bfloat16)
    b = (3 * torch.randn(M, N, device=device, generator=g)).to(torch.bfloat16)
    gt = (2 * torch.rand(T, N, device=device, generator=g)).to(torch.bfloat16)
    idx = torch.randint(0, T, (M,), device=device, generator=g)
    out = FB.post(r, gt, idx, b)
    for r0 in range(0, M, 8192):
        ob = FB.post(r[r0:r0 + 8192], gt, idx[r0:r0 + 8192], b[r0:r0 + 8192])
        assert torch.equal(out[r0:r0 + 8192].view(torch.int16), ob.view(torch.int16)), f"rows {r0}.. differ"
    rows = torch.arange(7, M, 2731, device=device)
    want = O.gated_residual(bits(r[rows]), bits(gt), idx[rows].cpu().numpy(), bits(b[rows]))
    assert np.array_equal(bits(out[rows]), want)


def test_pre_large_output(device):
    """The pre-norm alone on [32760, 5120] (a normed output beyond the last-level cache:
    non-temporal stores) equals the same rows done in small batches (cached stores)."""
    M, K, T = 32760, 5120, 4
    print(f"pre large M={M} K={K}", flush=True)
    g = torch.Generator(device=device).manual_seed(10)
    x = torch.randn(M, K, device=device, generator=g).to(torch.bfloat16)
    w = (1 + 0.05 * torch.randn(K, device=device, generator=g)).to(torch.bfloat16)
    sc = (0.2 * torch.randn(T, K, device=device, generator=g)).to(torch.bfloat16)
    sh = (0.2 * torch.randn(T, K, device=device, generator=g)).to(torch.bfloat16)
    idx = torch.randint(0, T, (M,), device=device, generator=g).to(torch.int32)
    out = FB.pre(x, w, 1e-6, sc, sh, idx)
    for r0 in range(0, M, 8192):
        ob = FB.pre(x[r0:r0 + 8192], w, 1e-6, sc, sh, idx[r0:r0 + 8192])
        assert torch.equal(out[r0:r0 + 8192].view(torch.int16), ob.view(torch.int16)), f"rows {r0}.. differ"
