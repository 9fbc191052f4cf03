"""The shared QKV quantization (HybridAttention._qkv's fp8 branch,
hybrid_attention.py:118-124) against the oracle, and the row-separability invariant the
fused QKV benchmark rests on.

- `softmax_attention.qkv` quantizes x once (codes and scales bit-exact with the oracle)
  and its raw q / k / v are each within the GEMM tolerance of the oracle's dequantized
  matmul of that projection (rel-L2 <= 1e-3, max-abs <= 2e-2 or the rounding chain).
- Per-output-channel scales are row-local, so requantizing the row concatenation
  Wq;Wk;Wv gives exactly the concatenation of the three requantizations (codes and
  scales, bit for bit), at the QKV workload's [15360, 5120] and at H3's [3 x 7168, 5376].
- The fused GEMM over those codes gives, bit for bit, the three projections' outputs
  concatenated: every output of the fused product is computed by the same arithmetic in
  the same order as in the separate product (the K-block order of an output depends
  only on K and on its tile's parity, and each projection is a multiple of 512 wide)."""
import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle as O
import vdn_fp8
from conftest import bits, codes
from test_gpu_gemm import MAX_ABS, REL_L2, bf16_ulp
from vdn_fp8 import workloads

pytestmark = pytest.mark.gpu


def _lin(w, b, device):
    lin = nn.Linear(w.shape[1], w.shape[0], bias=b is not None, dtype=torch.bfloat16, device="meta")
    lin.weight = nn.Parameter(w.to(device), requires_grad=False)
    lin.bias = nn.Parameter(b.to(device), requires_grad=False) if b is not None else None
    return vdn_fp8.Fp8Linear(lin)


def test_qkv_raw_projections_against_the_oracle(device):
    from vdn_fp8 import softmax_attention as SA
    T, H, d = 700, 8, 128
    C = H * d
    g = torch.Generator().manual_seed(21)
    x = torch.randn(T, C, generator=g).to(torch.bfloat16)
    ws = [(0.02 * torch.randn(C, C, generator=g)).to(torch.bfloat16) for _ in range(3)]
    bs = [(0.01 * torch.randn(C, generator=g)).to(torch.bfloat16) for _ in range(3)]
    lins = [_lin(w, b, device) for w, b in zip(ws, bs)]
    nq = nn.RMSNorm(d, eps=1e-6, dtype=torch.bfloat16).to(device)
    nk = nn.RMSNorm(d, eps=1e-6, dtype=torch.bfloat16).to(device)
    with torch.no_grad():
        q, k, v, (qr, kr, vr) = SA.qkv(x.to(device), *lins, H, nq, nk)
    torch.cuda.synchronize()
    qx, sx = O.quantize_rows(bits(x))                        # the one shared quantization
    for name, lin, raw, w, b in zip("qkv", lins, (qr, kr, vr), ws, bs):
        wq, wsc = O.quantize_weight(bits(w))
        assert np.array_equal(codes(lin.weight_fp8), wq), name
        want = O.dequant_linear(qx, sx, wq, wsc, bias=bits(b))
        mid = O.dequant_linear(qx, sx, wq, wsc)
        got = O.bf16_decode(bits(raw.reshape(T, C)))
        bound = np.maximum(MAX_ABS, bf16_ulp(mid) + bf16_ulp(want))
        rel, mx = O.rel_l2(got, want), O.max_abs(got, want)
        print(f"{name}: rel_l2={rel:.3e} max_abs={mx:.3e}", flush=True)
        assert rel <= REL_L2 and np.all(np.abs(got - want) <= bound), name


@pytest.mark.parametrize("case", ["dit_qkv", "h3"])
def test_fused_qkv_equals_three_projections(device, case):
    if case == "dit_qkv":
        x, w, b = workloads.dit_qkv()
        parts = 3
    else:
        g = torch.Generator().manual_seed(31)
        M, C, hid = 13107, 7168, 5376
        x = torch.randn(M, hid, generator=g).to(torch.bfloat16)
        w = (0.02 * torch.randn(3 * C, hid, generator=g)).to(torch.bfloat16)
        b = (0.01 * torch.randn(3 * C, generator=g)).to(torch.bfloat16)
        parts = 3
    print(f"fused QKV {case}: X {tuple(x.shape)} W {tuple(w.shape)}", flush=True)
    N = w.shape[0]
    n = N // parts
    fused = _lin(w, b, device)
    sep = [_lin(w[i * n:(i + 1) * n], b[i * n:(i + 1) * n], device) for i in range(parts)]
    # row separability of the weight quantization
    assert torch.equal(fused.weight_fp8.view(torch.uint8),
                       torch.cat([s.weight_fp8.view(torch.uint8) for s in sep], 0))
    assert torch.equal(fused.weight_scale, torch.cat([s.weight_scale for s in sep], 1))
    # one quantization of x shared by every product
    xq, xs = vdn_fp8.quantize_rows(x.to(device))
    out = fused.forward_quantized(xq, xs)
    outs = [s.forward_quantized(xq, xs) for s in sep]
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        same = torch.equal(out[:, i * n:(i + 1) * n].view(torch.int16), o.view(torch.int16))
        assert same, f"projection {i}: {(out[:, i * n:(i + 1) * n] != o).sum().item()} outputs differ"
