"""GPU parity of the row quantizers (vdn_fp8_quantize_rows / _swiglu_quantize_rows)
against the oracle: codes and scales bit-exact (SwiGLU: within one code, sigmoid is
transcendental). Inputs are seeded; shapes cover the DiT widths, ragged tails, the
wide two-sweep path, edge rows (zeros, signed zeros, the 1e-12 floor, outliers,
non-finite values) and an exhaustive sweep over every (row max, element) bf16 pair."""
import numpy as np
import pytest
import torch

import oracle as O
import vdn_fp8
from conftest import bits, codes, from_bits, same_codes

pytestmark = pytest.mark.gpu


def _run(x_bits, device):
    x = from_bits(x_bits, device)
    y, s = vdn_fp8.quantize_rows(x)
    torch.cuda.synchronize()
    return codes(y), s.cpu().numpy().reshape(-1)


def _check(x_bits, device):
    gy, gs = _run(x_bits, device)
    wy, ws = O.quantize_rows(x_bits)
    assert np.array_equal(gs.view(np.uint32), ws.view(np.uint32)), "scales differ"
    bad = ~same_codes(gy, wy)
    assert not bad.any(), f"{bad.sum()} codes differ, first at {np.argwhere(bad)[0]}"


def _randn_bits(rng, M, K, std=1.0):
    return O.bf16_encode(rng.standard_normal((M, K), dtype=np.float32) * std)


@pytest.mark.parametrize("M,K", [(1, 8), (3, 24), (5, 512), (64, 1024), (3, 4096), (7, 4104), (17, 5120),
                                 (9, 5376), (5, 8192), (2, 8200), (33, 13824), (4, 14336), (6, 16384), (3, 16392),
                                 (2, 40000)])
def test_quantize_rows_shapes(device, M, K):
    print(f"quantize_rows M={M} K={K}", flush=True)
    rng = np.random.default_rng(M * 100003 + K)
    _check(_randn_bits(rng, M, K), device)


def test_quantize_rows_edge_rows(device):
    rng = np.random.default_rng(7)
    K = 1024
    rows = [
        np.zeros(K, np.float32),                                     # zero row -> scale 1e-12
        -np.zeros(K, np.float32),                                    # signed zeros -> 0x80
        rng.standard_normal(K).astype(np.float32) * 1e-14,           # below the floor
        rng.standard_normal(K).astype(np.float32) * 1e-38,           # bf16 subnormals
        rng.standard_normal(K).astype(np.float32) * 3e38,            # near bf16 max
        np.where(np.arange(K) == 5, 448.0, 1.0).astype(np.float32),  # one outlier
        np.where(np.arange(K) % 2, -1.0, 1.0).astype(np.float32) * 0.7,
    ]
    x = O.bf16_encode(np.stack(rows))
    _check(x, device)


@pytest.mark.parametrize("K,col", [(64, 3), (5120, 600), (5120, 5119)])
def test_quantize_rows_nonfinite(device, K, col):
    """A row with inf gets scale inf and signed-zero codes for its finite elements; a
    row with NaN gets a NaN scale and NaN codes (sign of NaN codes unspecified). At
    K = 5120 two waves share a row; column 600 lies in the second wave's chunks."""
    x = np.ones((3, K), np.float32)
    x[0, col] = np.inf
    x[1, col - 1] = -np.inf
    x[2, col - 2] = np.nan
    xb = O.bf16_encode(x)
    gy, gs = _run(xb, device)
    wy, ws = O.quantize_rows(xb)
    assert np.isinf(gs[0]) and np.isinf(gs[1]) and np.isnan(gs[2])
    assert np.all(same_codes(gy, wy))


def test_quantize_rows_real_activations(device):
    """Real DiT inputs with outlier channels (the reference's prompt-embedding cache)."""
    d = np.load(f"{__import__('conftest').GOLDEN_DIR}/prompt_rows.npz")
    _check(d["x"], device)


def test_quantize_rows_qkv_full(device):
    """The M=32760 x 5120 activation of the QKV workload (0.1% outlier channels), whole."""
    from vdn_fp8 import workloads
    x, _, _ = workloads.dit_qkv()
    _check(bits(x), device)


def test_quantize_rows_strided_output(device):
    """Leading dimensions larger than K through the C ABI."""
    import vdn_fp8._lib as L
    rng = np.random.default_rng(11)
    M, K, ldx, ldy = 10, 512, 640, 576
    xb = _randn_bits(rng, M, ldx)
    x = from_bits(xb, device)
    y = torch.full((M, ldy), 0x55, dtype=torch.uint8, device=device)
    s = torch.empty(M, dtype=torch.float32, device=device)
    st = torch.cuda.current_stream().cuda_stream
    L.check(L.load().vdn_fp8_quantize_rows(x.data_ptr(), M, K, ldx, y.data_ptr(), ldy, s.data_ptr(), st), "q")
    torch.cuda.synchronize()
    wy, ws = O.quantize_rows(np.ascontiguousarray(xb[:, :K]))
    yy = y.cpu().numpy()
    assert np.array_equal(yy[:, :K], wy)
    assert np.all(yy[:, K:] == 0x55), "wrote past K"
    assert np.array_equal(s.cpu().numpy(), ws)


def exhaustive_chunks(rows_per_chunk=2048):
    """Yields bf16 matrices that together hold every (row max a, element x) pair of
    finite bf16 values with |x| <= a. Each row max a gets 4 rows of K = 16328: the
    first 8 columns hold a itself, the rest one quarter of all 65280 finite bf16
    patterns (both signs), zeroed where |x| > a. K = 16328 keeps the quantizers on
    their register-resident path (2041 chunks of 8 per row)."""
    allbits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    cols = allbits[(allbits & 0x7FFF) < 0x7F80].reshape(4, -1)      # [4, 16320]
    colmag = cols & 0x7FFF
    per = rows_per_chunk // 4
    for a0 in range(0, 0x7F80, per):
        amax = np.arange(a0, min(a0 + per, 0x7F80), dtype=np.uint16)
        body = np.where(colmag[None, :, :] <= amax[:, None, None], cols[None, :, :], 0).astype(np.uint16)
        head = np.repeat(amax[:, None, None], 8, axis=2).repeat(4, axis=1)
        yield np.concatenate([head, body], axis=2).reshape(-1, 8 + cols.shape[1])


def test_quantize_rows_exhaustive(device):
    """Codes and scales equal the oracle's for every (row max, element) pair: this
    covers every quotient the activation quantizer can form from bf16 input, and with
    it the hardware e4m3 conversion on that domain."""
    for i, x in enumerate(exhaustive_chunks()):
        if i % 16 == 0:
            print(f"exhaustive activation chunk {i}", flush=True)
        _check(x, device)


@pytest.mark.parametrize("M,K", [(1, 8), (7, 512), (16, 5120), (5, 7168), (3, 14336), (257, 14336), (9, 6152)])
def test_swiglu_quantize(device, M, K):
    rng = np.random.default_rng(K + M)
    hb = _randn_bits(rng, M, 2 * K, 2.0)
    y, s = vdn_fp8.swiglu_quantize(from_bits(hb, device))
    torch.cuda.synchronize()
    gy, gs = codes(y), s.cpu().numpy().reshape(-1)
    wy, ws = O.swiglu_quantize_rows(hb)
    # sigmoid via a different exp: scales within 1e-6 relative, codes within one step
    np.testing.assert_allclose(gs, ws, rtol=1e-6, atol=0)
    gv = O.e4m3_decode(gy).astype(np.float64) * gs[:, None]
    wv = O.e4m3_decode(wy).astype(np.float64) * ws[:, None]
    diff = np.abs(gy.astype(np.int32) - wy.astype(np.int32))
    assert np.mean(gy != wy) < 1e-3, "more than 0.1% of codes differ"
    assert np.all((diff <= 1) | (np.abs(gv - wv) <= 0.07 * np.abs(wv) + 1e-30)), "a code is off by more than one step"


def test_quantize_rows_large_output(device):
    """An output beyond the last-level cache (>= 256 MiB of codes: the non-temporal store
    path) is bit-identical to quantizing the same rows in small batches (the cached store
    path), and sampled rows match the oracle."""
    M, K = 20000, 13824
    print(f"quantize_rows large M={M} K={K}", flush=True)
    g = torch.Generator(device=device).manual_seed(5)
    x = torch.randn(M, K, device=device, generator=g).to(torch.bfloat16)
    y, s = vdn_fp8.quantize_rows(x)
    for r0 in range(0, M, 4000):
        yb, sb = vdn_fp8.quantize_rows(x[r0:r0 + 4000])
        assert torch.equal(y[r0:r0 + 4000].view(torch.uint8), yb.view(torch.uint8)), f"rows {r0}.. differ"
        assert torch.equal(s[r0:r0 + 4000].view(torch.int32), sb.view(torch.int32))
    rows = torch.arange(3, M, 1999, device=device)
    xs = bits(x[rows])
    wy, ws = O.quantize_rows(xs)
    assert np.all(same_codes(codes(y[rows]), wy))
    assert np.array_equal(s[rows].cpu().numpy().reshape(-1).view(np.uint32), ws.view(np.uint32))


def test_swiglu_quantize_large_output(device):
    """SwiGLU at the H3 width with an output beyond the last-level cache (non-temporal
    stores) is bit-identical to the same rows in small batches (cached stores)."""
    M, K = 19000, 14336
    print(f"swiglu_quantize large M={M} K={K}", flush=True)
    g = torch.Generator(device=device).manual_seed(6)
    h = (2.0 * torch.randn(M, 2 * K, device=device, generator=g)).to(torch.bfloat16)
    y, s = vdn_fp8.swiglu_quantize(h)
    for r0 in range(0, M, 4000):
        yb, sb = vdn_fp8.swiglu_quantize(h[r0:r0 + 4000])
        assert torch.equal(y[r0:r0 + 4000].view(torch.uint8), yb.view(torch.uint8)), f"rows {r0}.. differ"
        assert torch.equal(s[r0:r0 + 4000].view(torch.int32), sb.view(torch.int32))
