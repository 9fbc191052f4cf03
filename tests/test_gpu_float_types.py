"""GPU parity of the path for models that do not run in bf16: float16 / float32 rows into
the activation and SwiGLU quantizers, float16 / float32 weights into the rowwise weight
quantizer, and a float16 / float32 GEMM output (the reference's quantizers load any float
type and compute in binary32, fp8_linear.py:66-99; its weight branch divides in the
weight's own type, :262-267; `forward` passes out_dtype=rows.dtype, :279-283).

Codes and scales are compared bit for bit with the oracle (any two NaN codes count as
equal); SwiGLU codes within one step (sigmoid is transcendental); the GEMM's output within
the parity bounds (max-abs 2e-2, rel-L2 1e-3) of the oracle's float64 product rounded to
the output type, and against the reference's own torch._scaled_mm call with the same
out_dtype on the same codes."""
import numpy as np
import pytest
import torch

import oracle as O
import vdn_fp8
from conftest import codes, same_codes

pytestmark = pytest.mark.gpu

FLOATS = [torch.float32, torch.float16]


def _np(t):
    return t.detach().cpu().numpy()


def _cases(dtype, device):
    """Ordinary rows, rows scaled over many binades (float16 rows whose weight scale
    rounds to a subnormal or to zero), zeros, inf / NaN, the type's range ends, and a K
    that is not a multiple of 64."""
    g = torch.Generator().manual_seed(21)
    x = torch.randn(64, 200, generator=g) * torch.logspace(-7, 3, 64).reshape(-1, 1)
    x[3, 5], x[4, 7], x[6, 2] = float("nan"), float("inf"), -0.0
    x[5] = 0.0
    yield x.to(dtype)
    yield (torch.rand(16, 512, generator=g) * torch.finfo(dtype).max).to(dtype)
    yield (torch.randn(8, 256, generator=g) * torch.finfo(dtype).tiny).to(dtype)
    yield (torch.randn(1000, 5120, generator=g) * 2).to(dtype)
    yield (torch.randn(33, 136, generator=g)).to(dtype)


@pytest.mark.parametrize("dtype", FLOATS)
def test_quantize_rows_float_bit_exact(device, dtype):
    for x in _cases(dtype, device):
        print(f"quantize_rows {dtype} {tuple(x.shape)}", flush=True)
        q, s = vdn_fp8.quantize_rows(x.to(device))
        want_q, want_s = O.quantize_rows_float(_np(x))
        assert same_codes(codes(q), want_q).all()
        assert np.array_equal(_np(s).reshape(-1).view(np.uint32), want_s.view(np.uint32))


@pytest.mark.parametrize("dtype", FLOATS)
def test_requantize_weight_float_bit_exact(device, dtype):
    nan_codes = 0
    for w in _cases(dtype, device):
        w = torch.nan_to_num(w, nan=1.0, posinf=2.0)
        print(f"requantize_weight {dtype} {tuple(w.shape)}", flush=True)
        q, s = vdn_fp8.requantize_weight(w.to(device))
        want_q, want_s = O.quantize_weight_float(_np(w))
        got = codes(q)
        assert same_codes(got, want_q).all()
        assert np.array_equal(_np(s).view(np.uint32), want_s.view(np.uint32))
        nan_codes += int(((got & 0x7F) == 0x7F).sum())
    if dtype == torch.float16:
        assert nan_codes > 0      # quotients far above 448 (subnormal scales) give NaN, as torch's cast


@pytest.mark.parametrize("dtype", FLOATS)
def test_swiglu_quantize_float_within_one_code(device, dtype):
    g = torch.Generator().manual_seed(22)
    for M, K in ((64, 384), (257, 2048)):
        h = (torch.randn(M, 2 * K, generator=g) * 3).to(dtype)
        q, s = vdn_fp8.swiglu_quantize(h.to(device))
        want_q, want_s = O.swiglu_quantize_rows_float(_np(h))
        np.testing.assert_allclose(_np(s).reshape(-1), want_s, rtol=1e-6)
        got = codes(q).astype(int)
        assert np.max(np.abs(got - want_q.astype(int))) <= 1
        assert np.mean(got != want_q) < 1e-3


def _linear(N, K, dtype, device, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    lin = torch.nn.Linear(K, N, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
        if bias:
            lin.bias.copy_(torch.randn(N, generator=g) * 0.1)
    return lin.to(device=device, dtype=dtype)


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("M,N,K", [(300, 520, 512), (1000, 1536, 1024), (300, 520, 400)])
def test_fp8_linear_float_model(device, dtype, M, N, K):
    """Fp8Linear on a float16 / float32 Linear, fed rows of that type: the weight codes
    bit-exact with the oracle, the activation codes too, the output (of the rows' type)
    within the parity bounds of the oracle and of the reference's own
    torch._scaled_mm(out_dtype=that type) + bias on the same codes. K = 400 takes the
    kernel for K not a multiple of 256."""
    print(f"Fp8Linear {dtype} [{M}, {N}, {K}]", flush=True)
    lin = _linear(N, K, dtype, device, seed=M + N)
    f = vdn_fp8.Fp8Linear(lin)
    wq, ws = O.quantize_weight_float(_np(lin.weight))
    assert same_codes(codes(f.weight_fp8), wq).all()
    assert np.array_equal(_np(f.weight_scale).reshape(-1).view(np.uint32), ws.view(np.uint32))
    g = torch.Generator().manual_seed(K)
    x = (torch.randn(M, K, generator=g)).to(dtype).to(device)
    out = f(x)
    assert out.dtype == dtype and out.shape == (M, N)
    qx, sx = vdn_fp8.quantize_activation(x)
    want_qx, want_sx = O.quantize_rows_float(_np(x))
    assert same_codes(codes(qx), want_qx).all()
    np_dtype = np.float16 if dtype == torch.float16 else np.float32
    want = O.dequant_linear_typed(want_qx, want_sx, wq, ws, bias=_np(lin.bias).astype(np_dtype), out_dtype=np_dtype)
    got = _np(out).astype(np.float64)
    want = want.astype(np.float64)
    assert np.max(np.abs(got - want)) <= 2e-2
    assert O.rel_l2(got, want) <= 1e-3
    # the reference's own call on the same codes
    try:
        ref = torch._scaled_mm(qx, f.weight_fp8.t(), scale_a=sx, scale_b=f.weight_scale, out_dtype=dtype,
                               use_fast_accum=True) + lin.bias
    except (RuntimeError, ValueError) as e:   # hipBLASLt's rowwise path writes bf16 only on some shapes
        print(f"torch._scaled_mm refused out_dtype={dtype}: {str(e).splitlines()[0][:160]}", flush=True)
        return
    r = _np(ref).astype(np.float64)
    assert np.max(np.abs(got - r)) <= 2e-2
    assert O.rel_l2(got, r) <= 1e-3


def test_fp32_output_split_k(device):
    """A shape whose last round of tiles splits along K (K >= 8192, 260 tiles on 256 CUs):
    the binary32 output through the split-K reduction, rows of every m-tile checked
    against the oracle (so the split tiles are covered)."""
    M, N, K = 3328, 5120, 8192
    print(f"binary32 output split-K [{M}, {N}, {K}]", flush=True)
    lin = _linear(N, K, torch.float32, device, seed=5, bias=False)
    f = vdn_fp8.Fp8Linear(lin)
    assert vdn_fp8.fp8_linear.gemm_workspace_bytes(M, N, K, device) > 0
    g = torch.Generator().manual_seed(6)
    x = torch.randn(M, K, generator=g).to(device)
    qx, sx = vdn_fp8.quantize_rows(x)
    out = f.forward_quantized(qx, sx, out_dtype=torch.float32)
    rows = np.concatenate([np.arange(0, M, 256), np.arange(255, M, 256)])
    want = O.dequant_linear_typed(codes(qx)[rows], _np(sx).reshape(-1)[rows], codes(f.weight_fp8),
                                  _np(f.weight_scale).reshape(-1), out_dtype=np.float32)
    got = _np(out)[rows].astype(np.float64)
    assert np.max(np.abs(got - want)) <= 2e-2
    assert O.rel_l2(got, want.astype(np.float64)) <= 1e-3


def test_float_output_refuses_the_bf16_epilogues(device):
    lin = _linear(256, 256, torch.float32, device, seed=7)
    f = vdn_fp8.Fp8Linear(lin)
    qx, sx = vdn_fp8.quantize_rows(torch.randn(16, 256, device=device))
    with pytest.raises(ValueError, match="bfloat16"):
        f.forward_quantized(qx, sx, out_dtype=torch.float32, epilogue="gelu_tanh")
    with pytest.raises(ValueError, match="float64"):
        vdn_fp8.quantize_rows(torch.randn(4, 64, device=device, dtype=torch.float64))


def test_bf16_rows_through_a_float32_linear(device):
    """bf16 rows into a float32 Linear: the reference's forward gives out_dtype bf16 from
    _scaled_mm, then `out + bias` promotes to float32; the same here."""
    lin = _linear(512, 512, torch.float32, device, seed=8)
    f = vdn_fp8.Fp8Linear(lin)
    x = torch.randn(64, 512, device=device).to(torch.bfloat16)
    out = f(x)
    assert out.dtype == torch.float32
    qx, sx = vdn_fp8.quantize_rows(x)
    plain = f.forward_quantized(qx, sx, out_dtype=torch.bfloat16, epilogue=None)
    assert torch.equal(out, plain)
    f.bias = None
    want = f.forward_quantized(qx, sx) + lin.bias
    assert torch.equal(out, want)

