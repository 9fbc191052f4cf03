"""GPU parity of the fused pre-norm + quantizer (vdn_fp8_norm_quantize_rows) against the
oracle.

The normed bf16 values (RMSNorm + AdaLN affine, one rounding) are within one bf16 ulp of
the oracle's float64 evaluation -- an ulp at the scale of the affine's terms, since
x*rstd*w*(1+scale) and shift can cancel and a binary32 evaluation (the reference's compiled
`pre` is one too) errs at that scale -- and identical almost everywhere (the binary32 sum of
squares and reciprocal square root may flip a rounding); the codes and scales are then
bit-exact with quantize_rows of the kernel's own normed values -- the a2 contract
(fp8_linear.py:132-135) applied to the pre-norm's output (fused_block.py:41-44)."""
import numpy as np
import pytest
import torch

import oracle as O
import vdn_fp8
from conftest import bits, codes, from_bits, same_codes

pytestmark = pytest.mark.gpu


def _ulp(v):
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def _check(x, device, w=None, sc=None, sh=None, idx=None, eps=1e-6, min_same=0.995):
    y, s, n = vdn_fp8.pre_quantize(
        from_bits(x, device), None if w is None else from_bits(w, device), eps,
        None if sc is None else from_bits(sc, device), None if sh is None else from_bits(sh, device),
        None if idx is None else torch.from_numpy(np.asarray(idx, np.int32)).to(device), return_normed=True)
    torch.cuda.synchronize()
    gn = bits(n)
    want, terms = O.norm_rows(x, w, eps, sc, sh, idx, return_terms=True)
    gv, wv = O.bf16_decode(gn).astype(np.float64), O.bf16_decode(want).astype(np.float64)
    tol = _ulp(np.maximum(np.abs(wv), terms))
    assert np.all(np.abs(gv - wv) <= tol), f"normed off by {np.max(np.abs(gv - wv) / tol):.2f} ulp"
    same = float(np.mean(gn == want))
    assert same >= min_same, same
    q, qs = O.quantize_rows(gn)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), qs.view(np.uint32))
    assert np.all(same_codes(codes(y), q))
    # without the normed output the codes are the same
    y2, s2 = vdn_fp8.pre_quantize(
        from_bits(x, device), None if w is None else from_bits(w, device), eps,
        None if sc is None else from_bits(sc, device), None if sh is None else from_bits(sh, device),
        None if idx is None else torch.from_numpy(np.asarray(idx, np.int32)).to(device))
    torch.cuda.synchronize()
    assert np.array_equal(codes(y2), codes(y)) and torch.equal(s2, s)


def _rand(rng, shape, std, mean=0.0):
    return O.bf16_encode((mean + rng.standard_normal(shape, dtype=np.float32) * std).astype(np.float32))


@pytest.mark.parametrize("M,K", [(1, 8), (7, 64), (300, 1024), (64, 5120), (33, 5376), (16, 13824), (5, 16384)])
def test_pre_quantize_plain(device, M, K):
    rng = np.random.default_rng(M + K)
    _check(_rand(rng, (M, K), 1.5), device)


@pytest.mark.parametrize("M,K,T", [(256, 5120, 1), (300, 5376, 6), (40, 7168, 3), (3, 2048, 2), (9, 14336, 4)])
def test_pre_quantize_weight_and_table(device, M, K, T):
    rng = np.random.default_rng(M * K + T)
    x = _rand(rng, (M, K), 1.0)
    w = _rand(rng, K, 0.1, 1.0)
    sc = _rand(rng, (T, K), 0.3)
    sh = _rand(rng, (T, K), 0.3)
    idx = rng.integers(-1, T + 1, M)          # out-of-range rows clamp into the table
    _check(x, device, w, sc, sh, idx)


@pytest.mark.parametrize("M,K,T,frames", [(4096, 5120, 21, True), (700, 4096, 3, True), (999, 3072, 7, True),
                                          (1000, 3072, 5, False), (5, 5120, 2, False), (2000, 5376, 4, True),
                                          (600, 7168, 3, True), (300, 6144, 3, False)])
def test_pre_quantize_frames(device, M, K, T, frames):
    """Table rows by frame (contiguous runs of tokens, the factors of a block's first and
    last rows then serve every row) and at random (rows whose table row neither serves)."""
    rng = np.random.default_rng(M + K + T)
    x = _rand(rng, (M, K), 1.0)
    w = _rand(rng, K, 0.1, 1.0)
    sc = _rand(rng, (T, K), 0.3)
    sh = _rand(rng, (T, K), 0.3)
    idx = np.arange(M) * T // M if frames else rng.integers(0, T, M)
    _check(x, device, w, sc, sh, idx)


def test_pre_quantize_dit_rows(device):
    """The QKV activation's shape with its outlier channels, eps of the H3 norms."""
    from vdn_fp8 import workloads
    x, _, _ = workloads.dit_qkv(M=4096)
    rng = np.random.default_rng(4)
    K = x.shape[1]
    _check(bits(x), device, _rand(rng, K, 0.05, 1.0), _rand(rng, (2, K), 0.2), _rand(rng, (2, K), 0.2),
           rng.integers(0, 2, x.shape[0]), eps=1e-6)


@pytest.mark.parametrize("K", [512, 5120, 7168])
def test_pre_quantize_zero_and_constant_rows(device, K):
    """Both kernels (one wave group per row up to 2048 elements, one wave per row with the
    factors in LDS for 2049-7168)."""
    x = np.zeros((4, K), np.float32)
    x[1] = 3.0
    x[2] = -1e-20
    x[3, ::7] = 65000.0
    _check(O.bf16_encode(x), device, eps=1e-6, min_same=1.0)
