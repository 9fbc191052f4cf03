"""The LoRA workload end to end: merge, convert, then one DiT block's four fp8 linears on
its own input X [32760, 5120] (seed 5), in the reference's order -- merge_lora_state,
then convert_linear_to_fp8, then the forwards (assemble.py:124,166-175;
fused_block.py:93-111).

Checked against the oracle chain on one row of every 256-row tile:
- the merged QKV weight within one bf16 ulp of the oracle's merge, and the fused
  merge + requantize codes and scales bit-exact with the oracle's quantization of that
  merged weight (the merged weight is written once for the comparison; the fused
  conversion itself never writes it);
- X's codes and scales bit-exact; the QKV (+ bias), attention-out (+ gate) and FFN-up
  (+ GELU) outputs within the GEMM tolerance of the oracle's dequantized matmul;
- the FFN-up output, quantized again on the GPU, bit-exact with the oracle's codes of the
  same rows, and the FFN-down (+ gate) output within tolerance of the oracle's matmul of
  those codes;
- every output of the four linears identical to the reference's own call on this part
  (torch._scaled_mm on the same codes, then its bias add and epilogue) or one rounding
  chain apart."""
import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle as O
import vdn_fp8
from conftest import bits, codes, from_bits
from test_gpu_gemm import MAX_ABS, REL_L2, _tile_rows, _vs_reference_call, bf16_ulp, reference_call
from vdn_fp8 import workloads

pytestmark = pytest.mark.gpu


def _lin(w, b, device, lora=None):
    lin = nn.Linear(w.shape[1], w.shape[0], bias=b is not None, dtype=torch.bfloat16, device="meta")
    lin.weight = nn.Parameter(w.to(device), requires_grad=False)
    lin.bias = nn.Parameter(b.to(device), requires_grad=False) if b is not None else None
    return vdn_fp8.Fp8Linear(lin, lora=lora)


def _within(name, got, want, mid, b_bits=None, slope=None):
    chain = bf16_ulp(mid[0]) + (bf16_ulp(mid[1]) if b_bits is not None else 0.0)
    bound = chain if slope is None else slope * chain + bf16_ulp(want)
    bound = np.maximum(MAX_ABS, bound)
    err = np.abs(got - want)
    rel = O.rel_l2(got, want)
    above = err > MAX_ABS
    print(f"{name}: rel_l2={rel:.3e} max_abs={float(err.max()):.3e} identical={np.mean(got == want):.5f} "
          f"above_2e-2={int(above.sum())}/{got.size}"
          + (f" |v| in [{np.abs(want[above]).min():.3g}, {np.abs(want[above]).max():.3g}]" if above.any() else ""),
          flush=True)
    assert rel <= REL_L2 and np.all(err <= bound), name


def test_lora_block_chain(device):
    blk = workloads.dit_block()
    x = blk["x"]
    M = x.shape[0]
    rows = _tile_rows(M, 55)
    lora = (blk["a"].to(device), blk["b"].to(device), blk["lora_scale"])
    # merge, then convert: the fused conversion, and the merged weight written once for the check
    qkv = _lin(blk["w0"], blk["qkv_bias"], device, lora=lora)
    merged = torch.empty_like(blk["w0"], device=device)
    q2, s2 = vdn_fp8.requantize_weight(blk["w0"].to(device), lora=lora, merged_out=merged)
    torch.cuda.synchronize()
    assert torch.equal(q2.view(torch.uint8), qkv.weight_fp8.view(torch.uint8))
    assert torch.equal(s2.reshape(1, -1), qkv.weight_scale)
    gm = bits(merged)
    want_m = O.lora_merge(bits(blk["w0"]), bits(blk["a"]), bits(blk["b"]), blk["lora_scale"])
    gv, wv, w0 = (O.bf16_decode(t).astype(np.float64) for t in (gm, want_m, bits(blk["w0"])))
    tol = bf16_ulp(np.maximum(np.maximum(np.abs(w0), np.abs(wv - w0)), np.abs(wv)))
    assert np.all(np.abs(gv - wv) <= tol)
    print(f"merged weight: {np.mean(gm != want_m):.2e} of values one ulp off the oracle's merge", flush=True)
    wq_qkv, ws_qkv = O.quantize_weight(gm)
    assert np.array_equal(codes(qkv.weight_fp8), wq_qkv)
    assert np.array_equal(qkv.weight_scale.cpu().numpy().ravel().view(np.uint32), ws_qkv.view(np.uint32))

    out_l = _lin(blk["w_out"], None, device)
    up_l = _lin(blk["w_up"], blk["b_up"], device)
    dn_l = _lin(blk["w_down"], None, device)
    gate = blk["gate"].to(device)
    xd = x.to(device)
    qx, sx = vdn_fp8.quantize_rows(xd)
    y_qkv = qkv.forward_quantized(qx, sx)
    y_out = out_l.forward_quantized(qx, sx, epilogue="gate", gate=gate)
    h = up_l.forward_quantized(qx, sx, epilogue="gelu_tanh")
    qh, sh = vdn_fp8.quantize_rows(h)
    y_dn = dn_l.forward_quantized(qh, sh, epilogue="gate", gate=gate)
    torch.cuda.synchronize()

    oq, os_ = O.quantize_rows(bits(x[rows]))
    assert np.array_equal(codes(qx[rows]), oq)
    assert np.array_equal(sx[rows].cpu().numpy().ravel().view(np.uint32), os_.view(np.uint32))
    g_bits = bits(blk["gate"])
    for name, lin, y, bias, epi in (("qkv", qkv, y_qkv, blk["qkv_bias"], "none"),
                                    ("attn-out + gate", out_l, y_out, None, "gate"),
                                    ("ffn-up + gelu", up_l, h, blk["b_up"], "gelu_tanh")):
        wq, ws = codes(lin.weight_fp8), lin.weight_scale.cpu().numpy().ravel()
        b_bits = bits(bias) if bias is not None else None
        want = O.dequant_linear(oq, os_, wq, ws, bias=b_bits, epilogue=epi, gate=g_bits if epi == "gate" else None)
        mid = [O.dequant_linear(oq, os_, wq, ws), O.dequant_linear(oq, os_, wq, ws, bias=b_bits)]
        slope = None if epi == "none" else (1.13 if epi == "gelu_tanh" else
                                            max(1.0, float(np.abs(O.bf16_decode(g_bits)).max())))
        _within(name, O.bf16_decode(bits(y[rows])), want, mid, b_bits, slope)
    # the FFN-down input: the GPU's own GELU output, quantized again
    hq, hs = O.quantize_rows(bits(h[rows]))
    assert np.array_equal(codes(qh[rows]), hq)
    assert np.array_equal(sh[rows].cpu().numpy().ravel().view(np.uint32), hs.view(np.uint32))
    wq, ws = codes(dn_l.weight_fp8), dn_l.weight_scale.cpu().numpy().ravel()
    want = O.dequant_linear(hq, hs, wq, ws, epilogue="gate", gate=g_bits)
    mid = [O.dequant_linear(hq, hs, wq, ws), O.dequant_linear(hq, hs, wq, ws)]
    _within("ffn-down + gate", O.bf16_decode(bits(y_dn[rows])), want, mid, None,
            max(1.0, float(np.abs(O.bf16_decode(g_bits)).max())))
    # every output of the four linears against the reference's own call on this part
    # (torch._scaled_mm on the same codes, then its bias add and epilogue)
    for name, lin, y, q_, s_, epi in (("qkv", qkv, y_qkv, qx, sx, "none"),
                                      ("attn-out + gate", out_l, y_out, qx, sx, "gate"),
                                      ("ffn-up + gelu", up_l, h, qx, sx, "gelu_tanh"),
                                      ("ffn-down + gate", dn_l, y_dn, qh, sh, "gate")):
        rc = reference_call(q_, s_, lin, epi, gate if epi == "gate" else None)
        if rc is not None:
            print(name, end=": ", flush=True)
            _vs_reference_call(y, rc)
            del rc
