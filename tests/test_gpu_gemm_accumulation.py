"""How precisely the GEMM's matrix cores accumulate, measured through the C ABI.

X rows hold e4m3 codes c_k and repeat them (x[k + K/2] = x[k]); W rows hold codes d_k and
their negations (w[k + K/2] = -w[k]). Every exact dot product is then zero while its partial
sums grow to half the sum of |products| S and back, so with unit scales the bf16 output is
the accumulation's own error, measured against S. A binary32 accumulation sequence errs by
a few units of 2^-24 of its partial sums; the same codes summed by torch's binary32 matmul
give the comparison. The test reports the distribution and bounds its maximum: that
maximum is the error scale the GEMM parity tests' rounding-flip rates follow from."""
import numpy as np
import pytest
import torch

import vdn_fp8._lib as L

pytestmark = pytest.mark.gpu

# bound on max |error| / S of the fp8 matrix-core accumulation (checked here, used to
# derive the GEMM parity tests' identical-output floors)
MFMA_REL_ERR_MAX = 2.0 ** -15


def _codes(g, rows, cols, device):
    v = torch.randn(rows, cols, generator=g, device=device)
    return (v * (448.0 / v.abs().amax(1, keepdim=True))).to(torch.float8_e4m3fn).view(torch.uint8)


@pytest.mark.parametrize("M,N,K", [(2048, 2048, 5120), (1024, 1024, 13824), (512, 512, 1024)])
def test_accumulation_error_scale(device, M, N, K):
    print(f"accumulation M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=device).manual_seed(K)
    h = K // 2
    x = _codes(g, M, h, device).repeat(1, 2).contiguous()
    w = _codes(g, N, h, device)
    w = torch.cat([w, w ^ 0x80], 1).contiguous()            # e4m3 negation: the sign bit
    ones_x = torch.ones(M, device=device)
    ones_w = torch.ones(N, device=device)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=device)
    lib = L.load()
    st = torch.cuda.current_stream(device).cuda_stream
    L.check(lib.vdn_fp8_gemm(x.data_ptr(), ones_x.data_ptr(), w.data_ptr(), ones_w.data_ptr(), M, N, K, K, K,
                             None, L.EPI_NONE, None, None, 0, 0, None, 0, out.data_ptr(), N, st), "gemm")
    xf = x.view(torch.float8_e4m3fn).float()
    wf = w.view(torch.float8_e4m3fn).float()
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        S = xf.abs() @ wf.abs().t()
        f32 = xf @ wf.t()                                    # binary32 accumulation (library order)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    torch.cuda.synchronize()
    rel = (out.float().abs() / S).flatten()
    rel32 = (f32.abs() / S).flatten()
    q = torch.tensor([0.5, 0.99, 0.999], device=device)
    qs, qs32 = torch.quantile(rel[:1 << 24], q), torch.quantile(rel32[:1 << 24], q)
    frac_zero = float((out == 0).float().mean())
    print(f"|err|/S matrix cores: max={float(rel.max()):.3e} (2^{np.log2(max(float(rel.max()), 1e-30)):.1f}) "
          f"median={float(qs[0]):.2e} p99={float(qs[1]):.2e} p99.9={float(qs[2]):.2e} exact={frac_zero:.4f}; "
          f"binary32 library: max={float(rel32.max()):.3e} median={float(qs32[0]):.2e} p99.9={float(qs32[2]):.2e}",
          flush=True)
    assert float(rel.max()) <= MFMA_REL_ERR_MAX
