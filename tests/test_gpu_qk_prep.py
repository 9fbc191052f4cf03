"""GPU parity of the QK-norm + rope pass (vdn_fp8_qk_prep) against the oracle.

The reference's `_qk_prep` (softmax_attention/kernels.py:8-45) is a compiled kernel
whose binary32 operation order is not specified and which its own docstring calls
not bitwise with the eager ops; parity is therefore tolerance-only: every output
within one bf16 ulp of the oracle's float64 evaluation, measured at the magnitude of
the rotation's two products (n c and r s can cancel), and identical almost
everywhere."""
import numpy as np
import pytest
import torch

import oracle as O
import vdn_fp8
from conftest import bits, from_bits

pytestmark = pytest.mark.gpu


def _ulp(v):
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def _tables(rng, T, R, kind):
    theta = rng.uniform(-np.pi, np.pi, (T, R // 2)) * np.linspace(1.0, 1e-3, R // 2)
    cos = np.concatenate([np.cos(theta), np.cos(theta)], 1).astype(np.float32)
    sin = np.concatenate([np.sin(theta), np.sin(theta)], 1).astype(np.float32)
    if kind == "bf16":
        return O.bf16_encode(cos), O.bf16_encode(sin)
    return cos, sin


def _check(x, device, w=None, eps=1e-6, cos=None, sin=None, x_view=None, min_same=0.99):
    xt = from_bits(x, device) if x_view is None else x_view
    def tab(t):
        if t is None:
            return None
        return from_bits(t, device) if t.dtype == np.uint16 else torch.from_numpy(t).to(device)
    out = vdn_fp8.qk_prep(xt, None if w is None else from_bits(w, device), eps, tab(cos), tab(sin))
    torch.cuda.synchronize()
    assert out.shape == tuple(x.shape) and out.is_contiguous()
    got = bits(out)
    want, terms = O.qk_prep(x, w, eps, cos, sin, return_terms=True)
    gv, wv = O.bf16_decode(got).astype(np.float64), O.bf16_decode(want).astype(np.float64)
    tol = _ulp(np.maximum(np.abs(wv), terms))
    assert np.all(np.abs(gv - wv) <= tol), f"off by {np.max(np.abs(gv - wv) / tol):.2f} ulp"
    same = float(np.mean(got == want))
    assert same >= min_same, same


@pytest.mark.parametrize("T,H,d,R,kind", [
    (1, 1, 64, 64, "f32"), (37, 40, 128, 128, "f32"), (5, 42, 128, 64, "f32"),
    (9, 8, 256, 256, "bf16"), (300, 40, 128, 128, "bf16"), (3, 128, 128, 128, "f32"),
    (11, 24, 64, 32, "bf16"), (4, 64, 256, 0, None)])
def test_qk_prep_shapes(device, T, H, d, R, kind):
    print(f"qk_prep T={T} H={H} d={d} R={R} {kind}", flush=True)
    rng = np.random.default_rng(T * 7 + H + d + R)
    x = O.bf16_encode(rng.standard_normal((T, H, d), dtype=np.float32) * 2)
    w = O.bf16_encode(1 + 0.1 * rng.standard_normal(d, dtype=np.float32))
    cos = sin = None
    if R:
        cos, sin = _tables(rng, T, R, kind)
    _check(x, device, w, 1e-6, cos, sin)


def test_qk_prep_no_weight_and_eps(device):
    rng = np.random.default_rng(41)
    x = O.bf16_encode(rng.standard_normal((20, 16, 128), dtype=np.float32) * 1e-3)
    cos, sin = _tables(rng, 20, 128, "f32")
    _check(x, device, None, 1e-2, cos, sin)          # eps comparable to mean(x^2)
    z = np.zeros((3, 4, 128), np.uint16)             # zero rows: eps keeps them finite
    _check(z, device, None, 1e-6, *_tables(rng, 3, 128, "f32"))


def test_qk_prep_strided_q_slice(device):
    """q as the first third of a fused QKV projection output [T, 3 * H * d] -- a view
    with token stride 3 H d, as `unflatten` of a column slice gives."""
    rng = np.random.default_rng(42)
    T, H, d = 33, 40, 128
    full = O.bf16_encode(rng.standard_normal((T, 3 * H * d), dtype=np.float32))
    ft = from_bits(full, device)
    q = ft[:, : H * d].unflatten(-1, (H, d))
    k = ft[:, H * d: 2 * H * d].unflatten(-1, (H, d))
    w = O.bf16_encode(1 + 0.1 * rng.standard_normal(d, dtype=np.float32))
    cos, sin = _tables(rng, T, d, "f32")
    _check(np.ascontiguousarray(full[:, : H * d]).reshape(T, H, d), device, w, 1e-6, cos, sin, x_view=q)
    _check(np.ascontiguousarray(full[:, H * d: 2 * H * d]).reshape(T, H, d), device, w, 1e-6, cos, sin, x_view=k)


def test_qk_prep_qkv_workload_rows(device):
    """The QKV workload's q at full width (M = 32760 tokens, 40 heads of 128) through the
    GPU, checked on a sample of tokens against the oracle."""
    rng = np.random.default_rng(43)
    T, H, d = 32760, 40, 128
    xt = torch.randn(T, H, d, device=device).to(torch.bfloat16)
    w = O.bf16_encode(1 + 0.1 * rng.standard_normal(d, dtype=np.float32))
    theta = torch.rand(T, d // 2, device=device) * 6.28
    cos = torch.cat([theta.cos(), theta.cos()], 1)
    sin = torch.cat([theta.sin(), theta.sin()], 1)
    out = vdn_fp8.qk_prep(xt, from_bits(w, device), 1e-6, cos, sin)
    torch.cuda.synchronize()
    rows = np.sort(rng.choice(T, 256, replace=False))
    x = bits(xt[rows])
    want, terms = O.qk_prep(x, w, 1e-6, cos[rows].cpu().numpy(), sin[rows].cpu().numpy(), return_terms=True)
    got = bits(out[rows])
    gv, wv = O.bf16_decode(got).astype(np.float64), O.bf16_decode(want).astype(np.float64)
    assert np.all(np.abs(gv - wv) <= _ulp(np.maximum(np.abs(wv), terms)))
    assert np.mean(got == want) >= 0.99


def test_qkv_shares_one_quantization(device):
    """softmax_attention.qkv on fp8 projections: q/k/v equal the three forward_quantized
    calls on one quantization of x (bit for bit), q/k the qk_prep of the raw projections."""
    import torch.nn as nn
    from vdn_fp8 import softmax_attention as SA
    T, H, d = 300, 8, 128
    C = H * d
    g = torch.Generator().manual_seed(5)
    lins = []
    for _ in range(3):
        l = nn.Linear(C, C, dtype=torch.bfloat16)
        with torch.no_grad():
            l.weight.copy_((0.02 * torch.randn(C, C, generator=g)).to(torch.bfloat16))
            l.bias.copy_((0.01 * torch.randn(C, generator=g)).to(torch.bfloat16))
        lins.append(vdn_fp8.Fp8Linear(l.to(device)))
    nq, nk = nn.RMSNorm(d, eps=1e-6, dtype=torch.bfloat16).to(device), nn.RMSNorm(d, eps=1e-5, dtype=torch.bfloat16).to(device)
    with torch.no_grad():
        nq.weight.copy_((1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16))
        nk.weight.copy_((1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16))
    x = torch.randn(T, C, generator=g).to(torch.bfloat16).to(device)
    th = torch.rand(T, d // 2, generator=g) * 6.28
    cos = torch.cat([th.cos(), th.cos()], 1).to(device)
    sin = torch.cat([th.sin(), th.sin()], 1).to(device)
    with torch.no_grad():
        q, k, v, (qr, kr, vr) = SA.qkv(x, *lins, H, nq, nk, (cos, sin))
        xq, xs = vdn_fp8.quantize_rows(x)
        want = [l.forward_quantized(xq, xs).unflatten(-1, (H, d)) for l in lins]
        wq = vdn_fp8.qk_prep(want[0], nq.weight, nq.eps, cos, sin)
        wk = vdn_fp8.qk_prep(want[1], nk.weight, nk.eps, cos, sin)
    torch.cuda.synchronize()
    assert q.shape == k.shape == v.shape == (T, H, d)
    assert torch.equal(qr, want[0]) and torch.equal(kr, want[1]) and torch.equal(v, want[2]) and vr is v
    assert torch.equal(q, wq) and torch.equal(k, wk)


def test_qk_prep_large_output(device):
    """q of the QKV workload at full size (an output beyond the last-level cache:
    non-temporal stores) equals the same tokens done in small batches (cached stores)."""
    T, H, d = 32760, 40, 128
    print(f"qk_prep large T={T} H={H} d={d}", flush=True)
    g = torch.Generator(device=device).manual_seed(9)
    q = torch.randn(T, H, d, device=device, generator=g).to(torch.bfloat16)
    w = (1 + 0.05 * torch.randn(d, device=device, generator=g)).to(torch.bfloat16)
    th = torch.rand(T, d // 2, device=device, generator=g) * 6.28
    cs, sn = torch.cat([th.cos(), th.cos()], 1), torch.cat([th.sin(), th.sin()], 1)
    out = vdn_fp8.qk_prep(q, w, 1e-6, cs, sn)
    for t0 in range(0, T, 8192):
        ob = vdn_fp8.qk_prep(q[t0:t0 + 8192], w, 1e-6, cs[t0:t0 + 8192], sn[t0:t0 + 8192])
        assert torch.equal(out[t0:t0 + 8192].view(torch.int16), ob.view(torch.int16)), f"tokens {t0}.. differ"
