"""The GEMM against the reference's own forward_quantized call on the same codes:
torch._scaled_mm(x_fp8, weight_fp8.t(), scale_a=x_scale [M, 1], scale_b=weight_scale [1, N],
out_dtype=bf16, use_fast_accum=True) + bias (fp8_linear.py:272-276), which torch runs through
hipBLASLt on this part.

Both are fp8 GEMMs with fp32 accumulation in an unspecified order, rounded to bf16 at the
same points, so each output may sit one rounding step of the chain (GEMM output, bias add)
away from the reference's on either side: per element within max(2e-2, 2 x that chain),
rel-L2 <= 1e-3 over the output. If torch refuses rowwise scales the test is skipped with
its message."""
import numpy as np
import pytest
import torch

import oracle as O
import vdn_fp8
from conftest import bits, from_bits

pytestmark = pytest.mark.gpu


def _ulp(v):
    return torch.exp2(torch.floor(torch.log2(v.abs().clamp_min(2.0 ** -126))) - 7)


@pytest.mark.parametrize("M,N,K", [(4096, 3072, 5120), (1000, 1024, 1024)])
def test_gemm_matches_torch_scaled_mm(device, M, N, K):
    print(f"scaled_mm M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + N + K)
    x = from_bits(O.bf16_encode(rng.standard_normal((M, K), dtype=np.float32)), device)
    lin = torch.nn.Linear(K, N, bias=True, device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(from_bits(O.bf16_encode(rng.standard_normal((N, K), dtype=np.float32) * 0.02), device))
        lin.bias.copy_(from_bits(O.bf16_encode(rng.standard_normal(N, dtype=np.float32) * 0.01), device))
    f = vdn_fp8.Fp8Linear(lin)
    qx, sx = vdn_fp8.quantize_rows(x)
    ours = f.forward_quantized(qx, sx)
    try:
        mm = torch._scaled_mm(qx, f.weight_fp8.t(), scale_a=sx, scale_b=f.weight_scale,
                              out_dtype=torch.bfloat16, use_fast_accum=True)
    except RuntimeError as e:
        pytest.skip(f"torch._scaled_mm refuses rowwise scales here: {str(e).splitlines()[0][:200]}")
    ref = (mm + f.bias).float()
    torch.cuda.synchronize()
    got = ours.float()
    chain = _ulp(mm.float()) + _ulp(ref)
    bound = (2 * chain).clamp_(min=2e-2)
    err = (got - ref).abs()
    worst = float((err / bound).max())
    rel = float(torch.linalg.vector_norm(got - ref) / torch.linalg.vector_norm(ref))
    same = float((got == ref).float().mean())
    print(f"vs torch._scaled_mm: rel_l2={rel:.3e} max_abs={float(err.max()):.3e} identical={same:.5f} "
          f"worst/bound={worst:.2f}", flush=True)
    assert rel <= 1e-3 and worst <= 1.0, (rel, worst)
    # and torch's output is itself within the GEMM tolerance of the oracle on sampled rows
    rows = np.arange(0, M, 97)
    want = O.dequant_linear(qx.view(torch.uint8).cpu().numpy()[rows], sx.cpu().numpy().reshape(-1)[rows],
                            f.weight_fp8.view(torch.uint8).cpu().numpy(), f.weight_scale.cpu().numpy().reshape(-1),
                            bias=bits(f.bias.detach()))
    sel = torch.from_numpy(rows).to(device)
    tv = O.bf16_decode(bits((mm + f.bias)[sel]))
    ov = O.bf16_decode(bits(ours[sel]))
    print(f"vs the oracle on sampled rows: torch rel_l2={O.rel_l2(tv, want):.3e} max_abs={O.max_abs(tv, want):.3e} "
          f"identical={np.mean(tv == want):.5f}; ours rel_l2={O.rel_l2(ov, want):.3e} "
          f"max_abs={O.max_abs(ov, want):.3e} identical={np.mean(ov == want):.5f}", flush=True)
    assert O.rel_l2(tv, want) <= 1e-3
