"""What the reference's own arithmetic contract gives against the float64 oracle, on the
benchmark configs' data (CPU only).

The reference's GEMM is torch._scaled_mm with fp32 accumulation (fp8_linear.py:272-276):
the e4m3 products are exact in binary32 and summed in binary32, in an order the library
picks, then scaled and rounded to bf16, then the bf16 bias add and the epilogue round
again. Restated here with numpy binary32 (BLAS sgemm: another fp32 summation order) at the
reference's rounding points, on sampled rows of the QKV (cfg2), FFN-down + gate and
attention-out + gate (cfg4) workloads, and compared with the float64 oracle at the same
rounding points.

What this pins: binary32 summation order alone flips very few GEMM-output roundings
(<= 1e-3 of them; measured 5e-5 on the QKV rows), every output of the contract lies within
the per-element bound the GPU tests apply, max(2e-2, the rounding chain), and rel-L2 stays far
below 1e-3. Where a flip lands at |v| >= 2 (one bf16 step is 2^-6 there, doubled by the
gate) even the fp32 contract exceeds max-abs 2e-2; on these sampled rows that happens on the
gated FFN-down rows and not on the QKV rows (too few flips at large |v|). The GPU kernel's
matrix cores accumulate with less precision than binary32 (their flip rate is set against
this one in the GPU tests), so its outputs rely on that per-element bound more often.
"""
import numpy as np
import pytest

import oracle as O
from vdn_fp8 import workloads

MAX_ABS = 2e-2
ROW_STEP = 256          # one row of every 256-row tile


def _u16(t):
    import torch
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _bf16(v):
    """binary32 -> bf16 (round to nearest even) -> float64, as torch's cast does."""
    return O.bf16_decode(O.bf16_encode(np.asarray(v, np.float32))).astype(np.float64)


def _ulp(v):
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def _contract_fp32(qx, sx, qw, sw, bias=None, gate=None):
    """The reference's sequence in binary32: exact e4m3 products summed in binary32
    (sgemm), x scale_a x scale_b, bf16; + bias in binary32, bf16; x gate, bf16."""
    a = O.e4m3_decode(qx).astype(np.float32)
    b = O.e4m3_decode(qw).astype(np.float32)
    acc = a @ b.T                                     # binary32 accumulation
    v = (acc * np.asarray(sx, np.float32)[:, None]) * np.asarray(sw, np.float32)[None, :]
    mid = _bf16(v)
    out = mid
    if bias is not None:
        out = _bf16(out.astype(np.float32) + O.bf16_decode(bias).astype(np.float32)[None, :])
    if gate is not None:
        out = _bf16(out.astype(np.float32) * O.bf16_decode(gate).astype(np.float32)[None, :])
    return mid, out


def _compare(name, x_bits, w_bits, bias=None, gate=None):
    rows = x_bits[::ROW_STEP]
    qx, sx = O.quantize_rows(rows)
    qw, sw = O.quantize_weight(w_bits)
    mid32, got = _contract_fp32(qx, sx, qw, sw, bias, gate)
    want = O.dequant_linear(qx, sx, qw, sw, bias=bias, epilogue="gate" if gate is not None else "none",
                            gate=gate)
    mid64 = O.dequant_linear(qx, sx, qw, sw)
    err = np.abs(got - want)
    above = err > MAX_ABS
    same = float(np.mean(got == want))
    rel = O.rel_l2(got, want)
    # the GPU tests' per-element bound: one rounding step at the GEMM output, one more at
    # the bias add, scaled by the gate, plus the gate's own rounding
    chain = _ulp(mid64) + (_ulp(O.dequant_linear(qx, sx, qw, sw, bias=bias)) if bias is not None else 0.0)
    slope = 1.0 if gate is None else max(1.0, float(np.max(np.abs(O.bf16_decode(gate)))))
    bound = np.maximum(MAX_ABS, chain if gate is None else slope * chain + _ulp(want))
    worst = float(np.max(err / bound))
    vmag = np.abs(want[above])
    print(f"{name}: fp32 contract vs float64 oracle over {got.size} outputs: rel_l2={rel:.3e} "
          f"max_abs={err.max():.4f} identical={same:.5f} above_2e-2={int(above.sum())}"
          + (f" |v| in [{vmag.min():.3g}, {vmag.max():.3g}]" if above.any() else "")
          + f" worst/bound={worst:.2f}", flush=True)
    # how often binary32 summation order alone flips the first rounding (the GEMM output)
    flips = float(np.mean(mid32 != mid64))
    print(f"{name}: GEMM-output roundings flipped by binary32 summation: {flips:.2e}", flush=True)
    return dict(rel=rel, max_abs=float(err.max()), above=int(above.sum()), same=same, worst=worst,
                vmin=float(vmag.min()) if above.any() else None, flips=flips)


@pytest.fixture(scope="module")
def cfg4():
    (xd, wd), (xo, wo), g = workloads.dit_ffn_down_attn_out()
    return _u16(xd), _u16(wd), _u16(xo), _u16(wo), _u16(g)


FP32_FLIPS_MAX = 1e-3


def test_qkv_contract_within_the_chain_bound():
    x, w, b = (_u16(t) for t in workloads.dit_qkv())
    r = _compare("cfg2 QKV + bias", x, w, bias=b)
    assert r["rel"] <= 1e-3 and r["worst"] <= 1.0, r
    assert r["flips"] <= FP32_FLIPS_MAX, r


def test_ffn_down_and_attn_out_contract_within_the_chain_bound(cfg4):
    xd, wd, xo, wo, g = cfg4
    res = {}
    for name, xb, wb in (("cfg4 FFN-down + gate", xd, wd), ("cfg4 attn-out + gate", xo, wo)):
        r = res[name] = _compare(name, xb, wb, gate=g)
        assert r["rel"] <= 1e-3 and r["worst"] <= 1.0, r
        assert r["flips"] <= FP32_FLIPS_MAX, r
    # a flip at |v| >= 2 under the gate (up to 2) exceeds 2e-2 even in the fp32 contract
    r = res["cfg4 FFN-down + gate"]
    if r["above"]:
        assert r["max_abs"] > MAX_ABS and r["vmin"] >= 1.0, r
