"""Pins the CPU oracle (test infrastructure) before anything is compared with it.

Each check is independent of the oracle's own code: torch's CPU casts (the library
routines the reference's eager spellings call), a nearest-value brute force over the
256 e4m3 codes, known answers probed from torch, closed forms and invariants.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from conftest import same_codes

FP8 = torch.float8_e4m3fn


def torch_e4m3(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(FP8).view(torch.uint8).numpy()


def u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def from_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


# ---------------------------------------------------------------------------------
# e4m3 / bf16 element conversions
# ---------------------------------------------------------------------------------

def test_e4m3_all_bf16_values_match_torch():
    """Every bf16 pattern (all 65536), as binary32, encodes like torch's cast."""
    x = O.bf16_decode(np.arange(1 << 16, dtype=np.uint32).astype(np.uint16))
    assert np.all(same_codes(O.e4m3_encode(x), torch_e4m3(x)))


def test_e4m3_rounding_midpoints_match_torch():
    """Every midpoint between adjacent e4m3 values, and its binary32 neighbours: the
    inputs where a wrong tie rule or an off-by-one exponent shows."""
    vals = O.e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)   # 0 .. 448
    mids = np.concatenate([(vals[:-1] + vals[1:]) / 2, [464.0]]).astype(np.float32)
    near = np.concatenate([mids, np.nextafter(mids, 0), np.nextafter(mids, np.inf)])
    near = np.concatenate([near, -near])
    assert np.all(same_codes(O.e4m3_encode(near), torch_e4m3(near)))


def test_e4m3_random_fp32_match_torch():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    assert np.all(same_codes(O.e4m3_encode(x), torch_e4m3(x)))


def test_e4m3_brute_force_nearest():
    """Round to the nearest of the 126 positive finite codes, ties to the even code,
    magnitudes past the 448/NaN midpoint to NaN -- from the definition, on a dense
    sample of binary32 values."""
    table = O.e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)  # codes 0..0x7e
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(0, 470, 200_000), np.exp(rng.uniform(-25, 6.2, 200_000))]).astype(np.float32)
    xd = x.astype(np.float64)
    idx = np.searchsorted(table, xd)            # table[idx-1] < x <= table[idx]
    lo = np.clip(idx - 1, 0, 125)
    hi = np.clip(idx, 0, 126)
    dlo, dhi = xd - table[lo], table[hi] - xd
    pick = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi, np.where(lo % 2 == 0, lo, hi)))
    want = np.where(xd > 464.0, 0x7F, pick).astype(np.uint8)
    want = np.where(xd == table[hi], hi, want).astype(np.uint8)
    assert np.array_equal(O.e4m3_encode(x), want)


@pytest.mark.parametrize("v,code", [(448.0, 0x7E), (463.9, 0x7E), (464.0, 0x7E), (470.0, 0x7F), (480.0, 0x7F),
                                    (2.0 ** -9, 0x01), (2.0 ** -10, 0x00), (0.0013671875, 0x01), (1e-12, 0x00),
                                    (-0.0, 0x80), (-1e-5, 0x80), (1.0, 0x38), (-2.0, 0xC0), (2.0 ** -6, 0x08)])
def test_e4m3_known_answers(v, code):
    """Known answers probed from torch's CPU cast in this container."""
    assert O.e4m3_encode(np.array([v], np.float32))[0] == code


def test_e4m3_decode_table():
    c = np.arange(256, dtype=np.uint8)
    f = O.e4m3_decode(c)
    ref = torch.from_numpy(c.copy()).view(FP8).float().numpy()
    assert np.array_equal(np.isnan(f), np.isnan(ref))
    ok = ~np.isnan(f)
    assert np.array_equal(f[ok].view(np.uint32), ref[ok].view(np.uint32))


def test_bf16_encode_matches_torch():
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2 ** 32, size=1_000_000, dtype=np.uint64).astype(np.uint32)
    # add every exact tie and its neighbours in a few binades
    ties = (np.arange(1 << 16, dtype=np.uint32) << 16) | 0x8000
    x = np.concatenate([bits, ties, ties + 1, ties - 1]).view(np.float32)
    x = x[~np.isnan(x)]
    got = O.bf16_encode(x)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------------------------
# the quantizers against the reference's eager spellings in torch
# ---------------------------------------------------------------------------------

def rows_reference(x):
    """quantize_rows_reference (fp8_linear.py:132-135), torch CPU ops."""
    scale = (x.float().abs().amax(dim=1, keepdim=True) / 448.0).clamp_min(1e-12)
    return (x.float() / scale).to(FP8), scale


def weight_reference(w):
    """Rowwise branch of Fp8Linear.__init__ (fp8_linear.py:262-267), torch CPU ops."""
    scale = (w.abs().amax(dim=1, keepdim=True).float() / 448.0).clamp_min(1e-12)
    return (w / scale.to(w.dtype)).to(FP8), scale.reshape(1, -1)


def _rows_cases():
    g = torch.Generator().manual_seed(3)
    yield torch.randn(64, 1024, generator=g).to(torch.bfloat16)
    x = torch.randn(32, 5120, generator=g)
    x[:, torch.randperm(5120, generator=g)[:5]] *= 20
    yield x.to(torch.bfloat16)
    yield (torch.randn(8, 640, generator=g) * 1e-14).to(torch.bfloat16)          # below the floor
    yield (torch.randn(8, 640, generator=g) * 1e-38).to(torch.bfloat16)          # subnormals
    yield torch.zeros(2, 64, dtype=torch.bfloat16)
    yield -torch.zeros(2, 64, dtype=torch.bfloat16)
    yield (torch.rand(16, 2048, generator=g) * 3e38).to(torch.bfloat16)


@pytest.mark.parametrize("case", range(7))
def test_quantize_rows_matches_eager(case):
    x = list(_rows_cases())[case]
    q, s = O.quantize_rows(u16(x))
    rq, rs = rows_reference(x)
    assert np.array_equal(q, rq.view(torch.uint8).numpy())
    assert np.array_equal(s.view(np.uint32), rs.reshape(-1).numpy().view(np.uint32))


@pytest.mark.parametrize("case", range(7))
def test_quantize_weight_matches_eager(case):
    w = list(_rows_cases())[case]
    q, s = O.quantize_weight(u16(w))
    rq, rs = weight_reference(w)
    assert np.array_equal(q, rq.view(torch.uint8).numpy())
    assert np.array_equal(s.view(np.uint32), rs.reshape(-1).numpy().view(np.uint32))


def _float_cases(dtype):
    """Rows of float16 / float32 values: ordinary, scaled over many binades (float16 rows
    whose scale rounds to a float16 subnormal or to zero), signed zeros, inf / NaN, and
    values at the type's range ends."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(64, 200, generator=g) * torch.logspace(-7, 3, 64).reshape(-1, 1)
    x[3, 5], x[4, 7], x[6, 2] = float("nan"), float("inf"), -0.0
    x[5] = 0.0
    yield x.to(dtype)
    yield (torch.rand(16, 512, generator=g) * torch.finfo(dtype).max).to(dtype)
    yield (torch.randn(8, 256, generator=g) * torch.finfo(dtype).tiny).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_quantize_rows_float_matches_eager(dtype):
    """quantize_rows_reference on float16 / float32 rows: x.float() / scale, the cast."""
    for x in _float_cases(dtype):
        q, s = O.quantize_rows_float(x.numpy())
        rq, rs = rows_reference(x)
        assert np.array_equal(q, rq.view(torch.uint8).numpy())
        assert np.array_equal(s.view(np.uint32), rs.reshape(-1).numpy().view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_quantize_weight_float_matches_eager(dtype):
    """The rowwise branch of Fp8Linear.__init__ on float16 / float32 weights: the quotient
    in the weight's own type (for float16 rows with subnormal or zero scales, quotients
    far above 448: NaN codes, as torch's non-saturating cast gives)."""
    nan_codes = 0
    for w in _float_cases(dtype):
        w = torch.nan_to_num(w, nan=1.0, posinf=2.0)
        q, s = O.quantize_weight_float(w.numpy())
        rq, rs = weight_reference(w)
        assert np.array_equal(q, rq.view(torch.uint8).numpy())
        assert np.array_equal(s.view(np.uint32), rs.reshape(-1).numpy().view(np.uint32))
        nan_codes += int(((q & 0x7F) == 0x7F).sum())
    if dtype == torch.float16:
        assert nan_codes > 0          # the non-saturating cast is exercised


def test_quantize_weight_float16_rounding_matters():
    """A planted mistake must be caught: dividing by the binary32 scale (not its float16
    rounding) or skipping the float16 rounding of the quotient changes codes."""
    g = torch.Generator().manual_seed(12)
    w = (torch.randn(64, 1024, generator=g) * 0.05).to(torch.float16)
    rq, rs = weight_reference(w)
    no_scale_round = (w.float() / rs.reshape(-1, 1)).to(FP8)
    no_quot_round = (w.float() / rs.reshape(-1, 1).to(torch.float16).float()).to(FP8)
    assert (no_scale_round.view(torch.uint8) != rq.view(torch.uint8)).any()
    assert (no_quot_round.view(torch.uint8) != rq.view(torch.uint8)).any()


def test_swiglu_float_oracle_close_to_eager():
    """parity unpinned beyond tolerance, as for bf16 rows: SwiGLU + quantize on float32
    rows against torch's eager a * g * sigmoid(g) in binary32, codes within one step."""
    g = torch.Generator().manual_seed(13)
    h = torch.randn(32, 2 * 384, generator=g) * 3
    q, s = O.swiglu_quantize_rows_float(h.numpy())
    a, gt = h[:, :384], h[:, 384:]
    act = a * gt * torch.sigmoid(gt)
    rs = (act.abs().amax(dim=1) / 448.0).clamp_min(1e-12)
    rq = (act / rs[:, None]).to(FP8).view(torch.uint8).numpy()
    np.testing.assert_allclose(s, rs.numpy(), rtol=1e-6)
    assert np.mean(q != rq) < 1e-3
    assert np.max(np.abs(q.astype(int) - rq.astype(int))) <= 1


def test_dequant_linear_typed_closed_form():
    """One output by hand: codes 2.0 (0x40) and 0.5 (0x30), scales 0.25 and 4, K = 3:
    3 * 2 * 0.5 * 0.25 * 4 = 3, plus a bias of 0.5 in float16."""
    qx = np.full((1, 3), 0x40, np.uint8)
    qw = np.full((1, 3), 0x30, np.uint8)
    out = O.dequant_linear_typed(qx, [0.25], qw, [4.0], bias=np.array([0.5], np.float16), out_dtype=np.float16)
    assert out.dtype == np.float16 and float(out[0, 0]) == 3.5
    assert float(O.dequant_linear_typed(qx, [0.25], qw, [4.0])[0, 0]) == 3.0


def test_quantize_weight_double_rounding_matters():
    """A planted mistake must be caught: a single rounding (binary32 quotient straight
    to e4m3, skipping the bf16 round) differs from the reference's codes on ordinary
    weights, so the pinning above discriminates."""
    g = torch.Generator().manual_seed(4)
    w = (torch.randn(64, 2048, generator=g) * 0.02).to(torch.bfloat16)
    rq, rs = weight_reference(w)
    single = (w.float() / rs.reshape(-1, 1).to(torch.bfloat16).float()).to(FP8)
    assert (single.view(torch.uint8) != rq.view(torch.uint8)).any()


def test_quantize_rows_invariants():
    rng = np.random.default_rng(5)
    x = O.bf16_encode(rng.standard_normal((256, 512), dtype=np.float32) * rng.uniform(1e-3, 1e3, (256, 1)))
    q, s = O.quantize_rows(x)
    xf = O.bf16_decode(x)
    assert np.all(s >= np.float32(1e-12))
    mags = np.abs(xf).max(axis=1)
    arg = np.abs(xf).argmax(axis=1)
    # the row maximum maps to +-448
    assert np.all(q[np.arange(256), arg] & 0x7F == 0x7E)
    assert np.all(O.e4m3_decode(q) * np.sign(xf) >= 0)            # sign kept
    assert np.allclose(s, mags / 448.0, rtol=1e-7)


def test_swiglu_oracle_close_to_eager():
    """parity unpinned beyond tolerance: sigmoid is transcendental. Against torch's
    eager a * silu(g) in fp32: scales within 1e-6, codes within one step."""
    g = torch.Generator().manual_seed(6)
    h = (torch.randn(32, 2 * 1024, generator=g) * 2).to(torch.bfloat16)
    q, s = O.swiglu_quantize_rows(u16(h))
    a, gt = h.float().chunk(2, dim=1)
    act = a * gt * torch.sigmoid(gt)
    rs = (act.abs().amax(dim=1) / 448.0).clamp_min(1e-12)
    rq = (act / rs[:, None]).to(FP8).view(torch.uint8).numpy()
    np.testing.assert_allclose(s, rs.numpy(), rtol=1e-6)
    assert np.mean(q != rq) < 1e-3
    assert np.max(np.abs(q.astype(int) - rq.astype(int))) <= 1


# ---------------------------------------------------------------------------------
# LoRA merge
# ---------------------------------------------------------------------------------

def test_lora_merge_against_torch_fp32_matmul():
    g = torch.Generator().manual_seed(7)
    w = (torch.randn(96, 512, generator=g) * 0.02).to(torch.bfloat16)
    a = (torch.randn(32, 512, generator=g) * 0.05).to(torch.bfloat16)
    b = (torch.randn(96, 32, generator=g) * 0.05).to(torch.bfloat16)
    for scale in (1.0, 0.5):
        ref = w.clone()
        ref.add_(((b.float() @ a.float()) * scale).to(torch.bfloat16))
        got = O.lora_merge(u16(w), u16(a), u16(b), scale)
        d = np.abs(got.astype(np.int32) - u16(ref).astype(np.int32))
        assert np.mean(d != 0) < 1e-2          # fp32 summation order only
        gv, rv = O.bf16_decode(got), ref.float().numpy()
        assert np.max(np.abs(gv - rv)) <= 2.0 ** -14   # one bf16 ulp at the operands' scale


def test_lora_merge_exact_small_integers():
    """Brute force with a closed form: integer factors give exact sums; the merged
    weight is bf16(w + bf16(scale * (B @ A)))."""
    rng = np.random.default_rng(8)
    a = rng.integers(-3, 4, (8, 40)).astype(np.float32)
    b = rng.integers(-3, 4, (24, 8)).astype(np.float32)
    w = rng.integers(-50, 50, (24, 40)).astype(np.float32)
    got = O.bf16_decode(O.lora_merge(O.bf16_encode(w), O.bf16_encode(a), O.bf16_encode(b), 2.0))
    assert np.array_equal(got, w + 2.0 * (b @ a))


# ---------------------------------------------------------------------------------
# dequantized matmul and epilogues
# ---------------------------------------------------------------------------------

def test_dequant_linear_closed_form():
    """Identity-like weights: out = x * sx * sw exactly before rounding."""
    rng = np.random.default_rng(9)
    qx = O.e4m3_encode(rng.integers(-8, 9, (16, 32)).astype(np.float32))
    qw = O.e4m3_encode(np.eye(32, dtype=np.float32))
    sx = np.full(16, 0.5, np.float32)
    sw = np.full(32, 0.25, np.float32)
    out = O.dequant_linear(qx, sx, qw, sw, rounding="none")
    assert np.array_equal(out, O.e4m3_decode(qx).astype(np.float64) * 0.125)


def test_gelu_tanh_matches_torch():
    v = np.linspace(-8, 8, 10001)
    ref = torch.nn.functional.gelu(torch.from_numpy(v), approximate="tanh").numpy()
    np.testing.assert_allclose(O.gelu_tanh(v), ref, rtol=1e-12, atol=1e-14)


def test_gate_epilogue_matches_post_ref():
    """residual + gate.index_select(0, idx) * out (fused_block.py:47-49)."""
    rng = np.random.default_rng(10)
    qx = O.e4m3_encode(rng.standard_normal((12, 64)).astype(np.float32))
    qw = O.e4m3_encode(rng.standard_normal((16, 64)).astype(np.float32))
    sx, sw = np.ones(12, np.float32), np.full(16, 0.1, np.float32)
    gate = O.bf16_encode(rng.uniform(0, 2, (3, 16)).astype(np.float32))
    idx = rng.integers(0, 3, 12)
    res = O.bf16_encode(rng.standard_normal((12, 16)).astype(np.float32))
    base = O.dequant_linear(qx, sx, qw, sw, rounding="none")
    got = O.dequant_linear(qx, sx, qw, sw, epilogue="gate", gate=gate, gate_index=idx, residual=res, rounding="none")
    want = O.bf16_decode(res) + O.bf16_decode(gate)[idx] * base
    np.testing.assert_allclose(got, want, rtol=1e-12)


def test_reference_rounding_points():
    """rounding="reference" is bf16(bf16(matmul) + bias): planted single rounding
    differs from it somewhere, so the two spellings are distinguished."""
    rng = np.random.default_rng(11)
    qx = O.e4m3_encode(rng.standard_normal((64, 256)).astype(np.float32))
    qw = O.e4m3_encode(rng.standard_normal((64, 256)).astype(np.float32))
    sx, sw = np.full(64, 0.01, np.float32), np.full(64, 0.02, np.float32)
    bias = O.bf16_encode(rng.standard_normal(64).astype(np.float32))
    ref = O.dequant_linear(qx, sx, qw, sw, bias=bias)
    raw = O.dequant_linear(qx, sx, qw, sw, bias=bias, rounding="none")
    single = O.bf16_decode(O.bf16_encode(raw.astype(np.float32)))
    assert np.array_equal(ref, O.bf16_decode(O.bf16_encode(ref.astype(np.float32))))   # bf16 values
    assert np.any(ref != single)
    assert O.rel_l2(ref, raw) < 3e-3


# ---------------------------------------------------------------------------------
# the fused pre-norm (RMSNorm + AdaLN affine) feeding the quantizer
# ---------------------------------------------------------------------------------

def test_norm_rows_matches_torch_rms_norm():
    """Against torch's own F.rms_norm in float64, then the affine of _pre_ref."""
    import torch.nn.functional as F
    rng = np.random.default_rng(21)
    M, K, T = 37, 320, 3
    x = O.bf16_encode(rng.standard_normal((M, K), dtype=np.float32) * 2)
    w = O.bf16_encode(1 + 0.1 * rng.standard_normal(K, dtype=np.float32))
    sc = O.bf16_encode(0.2 * rng.standard_normal((T, K), dtype=np.float32))
    sh = O.bf16_encode(0.2 * rng.standard_normal((T, K), dtype=np.float32))
    idx = rng.integers(0, T, M)
    got = O.bf16_decode(O.norm_rows(x, w, 1e-6, sc, sh, idx)).astype(np.float64)
    xt = torch.from_numpy(O.bf16_decode(x).astype(np.float64))
    ref = F.rms_norm(xt, (K,), torch.from_numpy(O.bf16_decode(w).astype(np.float64)), float(np.float32(1e-6)))
    it = torch.from_numpy(idx)
    ref = ref * (1 + torch.from_numpy(O.bf16_decode(sc).astype(np.float64))[it]) \
        + torch.from_numpy(O.bf16_decode(sh).astype(np.float64))[it]
    want = ref.to(torch.float32).to(torch.bfloat16).to(torch.float64).numpy()
    assert np.mean(got == want) > 0.999 and np.max(np.abs(got - want)) <= np.max(np.abs(want)) * 2 ** -7


def test_norm_rows_closed_forms():
    """A constant row normalizes to sign(c) (eps = 0); the affine then applies exactly;
    with no weight and no table the result is x * rsqrt(mean(x^2) + eps)."""
    K = 64
    x = O.bf16_encode(np.array([[3.0] * K, [-0.5] * K], np.float32))
    w = O.bf16_encode(np.full(K, 2.0, np.float32))
    sc = O.bf16_encode(np.full((1, K), 0.5, np.float32))
    sh = O.bf16_encode(np.full((1, K), 0.25, np.float32))
    n = O.bf16_decode(O.norm_rows(x, w, 0.0, sc, sh))
    assert np.all(n[0] == 2.0 * 1.5 + 0.25) and np.all(n[1] == -2.0 * 1.5 + 0.25)
    x2 = O.bf16_encode(np.array([[1.0, -1.0, 2.0, -2.0] * 16], np.float32))
    n2 = O.bf16_decode(O.norm_rows(x2, None, 0.0))
    r = 1 / np.sqrt(2.5)
    assert np.all(n2 == O.bf16_decode(O.bf16_encode((O.bf16_decode(x2) * r).astype(np.float32))))


def test_norm_quantize_is_quantize_of_normed():
    rng = np.random.default_rng(22)
    x = O.bf16_encode(rng.standard_normal((9, 256), dtype=np.float32))
    q, s, n = O.norm_quantize_rows(x)
    q2, s2 = O.quantize_rows(n)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def _rms_norm_torch64(x_bits, w_bits, eps):
    import torch.nn.functional as F
    xt = torch.from_numpy(O.bf16_decode(x_bits).astype(np.float64))
    wt = None if w_bits is None else torch.from_numpy(O.bf16_decode(w_bits).astype(np.float64))
    return F.rms_norm(xt, (xt.shape[-1],), wt, float(np.float32(eps))).numpy()


def _bits64(v):
    return O.bf16_encode(np.asarray(v, np.float64).astype(np.float32))


def test_qk_prep_identity_rotation_is_rms_norm():
    """cos = 1, sin = 0: the pass is torch's F.rms_norm (float64), rounded once."""
    rng = np.random.default_rng(31)
    T, H, d = 7, 3, 128
    x = O.bf16_encode(rng.standard_normal((T, H, d), dtype=np.float32) * 3)
    w = O.bf16_encode(1 + 0.1 * rng.standard_normal(d, dtype=np.float32))
    ones, zeros = np.ones((T, d), np.float32), np.zeros((T, d), np.float32)
    got = O.qk_prep(x, w, 1e-6, ones, zeros)
    want = _bits64(_rms_norm_torch64(x, w, 1e-6))
    assert np.mean(got == want) > 0.999
    assert np.array_equal(O.qk_prep(x, w, 1e-6), got)          # no tables: no rotation


def test_qk_prep_quarter_turn_and_pass_through():
    """cos = 0, sin = 1 on the first R channels: out[i] = -n[i + R/2], out[i + R/2] = n[i];
    channels past R are the plain RMSNorm."""
    rng = np.random.default_rng(32)
    T, H, d, R = 5, 4, 128, 64
    x = O.bf16_encode(rng.standard_normal((T, H, d), dtype=np.float32))
    n = _rms_norm_torch64(x, None, 1e-6)
    got = O.bf16_decode(O.qk_prep(x, None, 1e-6, np.zeros((T, R), np.float32), np.ones((T, R), np.float32)))
    h = R // 2
    want = n.copy()
    want[..., :h] = -n[..., h:R]
    want[..., h:R] = n[..., :h]
    assert np.mean(got == O.bf16_decode(_bits64(want))) > 0.999


def test_qk_prep_is_complex_rotation():
    """With the usual table layout (cos[i] = cos[i + R/2]), each pair (n[i], n[i + R/2])
    is multiplied by the complex number c + i s: an independent formulation."""
    rng = np.random.default_rng(33)
    T, H, d = 6, 5, 128
    x = O.bf16_encode(rng.standard_normal((T, H, d), dtype=np.float32) * 0.5)
    w = O.bf16_encode(1 + 0.05 * rng.standard_normal(d, dtype=np.float32))
    theta = rng.uniform(-np.pi, np.pi, (T, d // 2))
    cos = np.concatenate([np.cos(theta), np.cos(theta)], 1).astype(np.float32)
    sin = np.concatenate([np.sin(theta), np.sin(theta)], 1).astype(np.float32)
    got = O.bf16_decode(O.qk_prep(x, w, 1e-6, cos, sin)).astype(np.float64)
    n = _rms_norm_torch64(x, w, 1e-6)
    c = O.bf16_decode(O.bf16_encode(cos[:, : d // 2])).astype(np.float64)[:, None, :]
    s = O.bf16_decode(O.bf16_encode(sin[:, : d // 2])).astype(np.float64)[:, None, :]
    z = (n[..., : d // 2] + 1j * n[..., d // 2:]) * (c + 1j * s)
    want = np.concatenate([z.real, z.imag], -1)
    want_b = O.bf16_decode(_bits64(want)).astype(np.float64)
    assert np.mean(got == want_b) > 0.995
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
    assert np.all(np.abs(got - want) <= ulp)


def test_gated_residual_matches_torch_binary32():
    """The compiled `post` evaluates residual + gate * branch in binary32 (the product of
    two bf16 values is exact there) and rounds to bf16 once: torch's own binary32
    arithmetic and casts give the same bits as the oracle's float64 restatement."""
    rng = np.random.default_rng(51)
    M, N, T = 64, 96, 3
    r = O.bf16_encode(rng.standard_normal((M, N), dtype=np.float32))
    b = O.bf16_encode(rng.standard_normal((M, N), dtype=np.float32) * 5)
    g = O.bf16_encode(rng.uniform(0, 2, (T, N)).astype(np.float32))
    idx = rng.integers(0, T, M)
    t = lambda a: torch.from_numpy(O.bf16_decode(a).astype(np.float32))
    want = (t(r) + t(g)[torch.from_numpy(idx)] * t(b)).to(torch.bfloat16)
    want = want.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.gated_residual(r, g, idx, b), want)
    # the product is exact in binary32: no rounding before the sum
    prod = O.bf16_decode(g).astype(np.float64)[idx] * O.bf16_decode(b).astype(np.float64)
    assert np.array_equal(prod, prod.astype(np.float32).astype(np.float64))
