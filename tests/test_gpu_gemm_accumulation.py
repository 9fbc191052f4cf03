"""How the fp8 matrix cores add, measured through the C ABI with unit scales (the bf16
output is then the accumulator itself, rounded once), and set against the reference's own
call on this part (torch._scaled_mm with fast accumulation, hipBLASLt).

Known answers: inside one fp8 MFMA instruction (v_mfma_f32_16x16x128_f8f6f4 here: 128
products of one K step; the 32 x 32 x 64 form behaves the same on its 64) the products are
aligned to the largest of them before they are summed, and bits below that alignment are
dropped. A cancelling pair of large products next to many small ones loses
part of the small ones' sum (448^2 pairs with 62 products of 2^-9: 0.109 instead of 0.121),
while the same small products alone sum exactly, as do exact small integers. hipBLASLt
gives the same results on the same codes: it is the instruction's arithmetic, not this
kernel's. This is what makes ~1% of the bf16 outputs of a real GEMM round differently from
a float64 (or binary32) sum of the same products, in both.

Across K steps the accumulator adds exactly for these magnitudes: X rows repeat their
codes (x[k + K/2] = x[k]) against W rows holding codes and their negations, so every exact
dot product is zero while its partial sums grow to half the sum of |products| S and back;
the output is then within 2^-15 S of zero (measured ~2^-27; binary32 library matmul
~2^-25)."""
import numpy as np
import pytest
import torch

import oracle as O
import vdn_fp8._lib as L

pytestmark = pytest.mark.gpu

# bound on max |output| / S of the mirrored sums (the accumulation across K steps)
MFMA_REL_ERR_MAX = 2.0 ** -15


def _codes(g, rows, cols, device):
    v = torch.randn(rows, cols, generator=g, device=device)
    return (v * (448.0 / v.abs().amax(1, keepdim=True))).to(torch.float8_e4m3fn).view(torch.uint8)


def _gemm(x, w):
    """bf16 x @ w^T of e4m3 codes (uint8 tensors on the GPU) with unit scales."""
    M, K = x.shape
    N = w.shape[0]
    dev = x.device
    ones_x, ones_w = torch.ones(M, device=dev), torch.ones(N, device=dev)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    L.check(L.load().vdn_fp8_gemm(x.data_ptr(), ones_x.data_ptr(), w.data_ptr(), ones_w.data_ptr(), M, N, K, K, K,
                                  None, L.EPI_NONE, None, None, 0, 0, None, 0, out.data_ptr(), N,
                                  torch.cuda.current_stream(dev).cuda_stream), "gemm")
    return out


def _scaled_mm(x, w):
    M, N = x.shape[0], w.shape[0]
    try:
        return torch._scaled_mm(x.view(torch.float8_e4m3fn), w.view(torch.float8_e4m3fn).t(),
                                scale_a=torch.ones(M, 1, device=x.device), scale_b=torch.ones(1, N, device=x.device),
                                out_dtype=torch.bfloat16, use_fast_accum=True)
    except RuntimeError as e:
        print(f"torch._scaled_mm refused: {str(e).splitlines()[0][:160]}", flush=True)
        return None


def _dec(c):
    return float(O.e4m3_decode(np.array([c], np.uint8))[0])


@pytest.mark.parametrize("big,small", [(0x7E, 0x01), (0x7E, 0x08), (0x70, 0x20), (0x60, 0x01), (None, 0x01),
                                       (None, 0x20)])
def test_matrix_core_alignment_known_answers(device, big, small):
    """One K step of 64 products: a cancelling pair big x big, big x -big (or none) and 62
    products 1.0 x small, then a K step of zeros. Without the pair the sum is exact; with it,
    the small products lose the bits below the pair's alignment -- in this kernel and in
    hipBLASLt alike."""
    M = N = 256
    K = 128
    x = torch.zeros(M, K, dtype=torch.uint8, device=device)
    w = torch.zeros(N, K, dtype=torch.uint8, device=device)
    x[:, 2:64] = 0x38
    w[:, 2:64] = small
    if big is not None:
        x[:, 0] = big
        x[:, 1] = big
        w[:, 0] = big
        w[:, 1] = big | 0x80
    exact = 62 * _dec(small)
    got = _gemm(x, w)
    ref = _scaled_mm(x, w)
    torch.cuda.synchronize()
    g = float(got[0, 0])
    print(f"big={big} small={_dec(small):.6g}: ours {g:.8g}, exact {exact:.8g}"
          + ("" if ref is None else f", hipBLASLt {float(ref[0, 0]):.8g}"), flush=True)
    assert torch.all(got == got[0, 0])
    if big is None:
        assert g == exact                                   # small products alone: exact
    else:
        assert 0.85 * exact <= g <= exact                   # bits below the alignment dropped
    if ref is not None:
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("M,N,K", [(2048, 2048, 5120), (1024, 1024, 13824), (512, 512, 1024)])
def test_accumulation_across_k_steps(device, M, N, K):
    print(f"accumulation M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=device).manual_seed(K)
    h = K // 2
    x = _codes(g, M, h, device).repeat(1, 2).contiguous()
    w = _codes(g, N, h, device)
    w = torch.cat([w, w ^ 0x80], 1).contiguous()            # e4m3 negation: the sign bit
    out = _gemm(x, w)
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
    print(f"|out|/S matrix cores: max={float(rel.max()):.3e} (2^{np.log2(max(float(rel.max()), 1e-30)):.1f}) "
          f"median={float(qs[0]):.2e} p99={float(qs[1]):.2e} p99.9={float(qs[2]):.2e} exact={frac_zero:.4f}; "
          f"binary32 library: max={float(rel32.max()):.3e} median={float(qs32[0]):.2e} p99.9={float(qs32[2]):.2e}",
          flush=True)
    assert float(rel.max()) <= MFMA_REL_ERR_MAX
