"""GPU parity of the GELU(tanh) row quantizer (vdn_fp8_gelu_quantize_rows): a GELU FFN's
down-projection input, quantize_rows (fp8_linear.py:110-117) of bf16(gelu_tanh(h)).

Against the GEMM path it replaces, bit for bit: the up projection with the "gelu_tanh"
epilogue, then quantize_rows, gives the same codes and scales as the up projection with
its bias alone, then gelu_quantize (the same GELU on the same bf16 value). Against the
oracle (the textbook GELU in float64): the kernel's GELU is an approximation within a few
binary32 ulps, so a bf16 rounding of it can land one step from the oracle's; codes within
one step, rows whose maximum rounded the same way with the same scale."""
import numpy as np
import pytest
import torch

import oracle as O
import vdn_fp8
from conftest import codes, same_codes

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K", [(300, 512, 1024), (1000, 13824, 1024), (257, 5120, 512), (64, 16384, 256),
                                   (33, 2056, 512)])
def test_gelu_quantize_equals_the_gemm_epilogue_path(device, M, N, K):
    """quantize_rows(up(x) with the GELU epilogue) == gelu_quantize(up(x) with its bias
    alone), codes and scales bit for bit; N = 13824 and 16384 take four waves per row,
    N = 512 and 2056 one."""
    print(f"gelu_quantize vs GEMM GELU epilogue [{M}, {N}, {K}]", flush=True)
    g = torch.Generator(device=device).manual_seed(N + M)
    lin = torch.nn.Linear(K, N, bias=True, device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(0.05 * torch.randn(N, K, device=device, generator=g))
        lin.bias.copy_(0.5 * torch.randn(N, device=device, generator=g))
    f = vdn_fp8.Fp8Linear(lin)
    qx, sx = vdn_fp8.quantize_rows(torch.randn(M, K, device=device, generator=g).to(torch.bfloat16))
    q1, s1 = vdn_fp8.quantize_rows(f.forward_quantized(qx, sx, epilogue="gelu_tanh"))
    q2, s2 = vdn_fp8.gelu_quantize(f.forward_quantized(qx, sx))
    torch.cuda.synchronize()
    assert torch.equal(q1.view(torch.uint8), q2.view(torch.uint8))
    assert torch.equal(s1.view(torch.int32), s2.view(torch.int32))


def _gelu_cases():
    rng = np.random.default_rng(51)
    x = (rng.standard_normal((200, 1024)) * np.logspace(-3, 1.5, 200).reshape(-1, 1)).astype(np.float32)
    x[3] = 0.0
    x[4] = -0.0
    x[5, :7] = [-10.0, -4.0, -1e-30, 1e-30, 3.0, 60.0, -60.0]
    yield x
    yield (rng.standard_normal((33, 13824)) * 3).astype(np.float32)
    yield (rng.standard_normal((9, 4104)) * 0.5).astype(np.float32)


def test_gelu_quantize_against_the_oracle(device):
    for x in _gelu_cases():
        print(f"gelu_quantize vs oracle {x.shape}", flush=True)
        hb = O.bf16_encode(x)
        h = torch.from_numpy(hb.view(np.int16)).view(torch.bfloat16).to(device)
        q, s = vdn_fp8.gelu_quantize(h)
        want_q, want_s = O.gelu_quantize_rows(hb)
        got_s = s.cpu().numpy().reshape(-1)
        got_q = codes(q)
        same_s = got_s.view(np.uint32) == want_s.view(np.uint32)
        assert np.mean(same_s) >= 0.97
        # a row maximum that rounded the other way moves the scale by one bf16 step of the maximum
        assert np.all(np.abs(got_s / want_s - 1.0) <= 2.0 ** -7)
        d = np.abs(got_q[same_s].astype(int) - want_q[same_s].astype(int))
        assert np.all((d <= 1) | same_codes(got_q[same_s], want_q[same_s]))
        assert np.mean(d != 0) < 1e-3
        # zero and signed-zero rows: scale 1e-12, codes +0 / -0
        if x.shape == (200, 1024):
            assert got_s[3] == np.float32(1e-12) and np.all(got_q[3] == 0) and np.all(got_q[4] == 0x80)


def test_gelu_quantize_refuses_wide_rows(device):
    h = torch.zeros(2, 16392, device=device, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="16384"):
        vdn_fp8.gelu_quantize(h)
