"""GPU parity of the weight requantizer (vdn_fp8_requantize_weight) against the oracle.

Without LoRA: codes and fp32 scales bit-exact with the rowwise branch of
Fp8Linear.__init__ (fp8_linear.py:262-267), including an exhaustive sweep over every
(row max, element) bf16 pair. With LoRA: the merged weight within one bf16 ulp of the
oracle's merge (the reference's fp32 summation order is unspecified), and the codes
bit-exact with the oracle's quantization of the kernel's own merged weight."""
import numpy as np
import pytest
import torch

import oracle as O
import vdn_fp8
from conftest import bits, codes, from_bits, same_codes
from test_gpu_quantize import exhaustive_chunks

pytestmark = pytest.mark.gpu


def _requant(w_bits, device, lora=None, merged=False):
    w = from_bits(w_bits, device)
    out = torch.empty_like(w) if merged else None
    q, s = vdn_fp8.requantize_weight(w, lora=lora, merged_out=out)
    torch.cuda.synchronize()
    return codes(q), s.cpu().numpy(), (bits(out) if merged else None)


def _check_plain(w_bits, device):
    gq, gs, _ = _requant(w_bits, device)
    wq, ws = O.quantize_weight(w_bits)
    assert np.array_equal(gs.view(np.uint32), ws.view(np.uint32)), "scales differ"
    bad = ~same_codes(gq, wq)
    assert not bad.any(), f"{bad.sum()} codes differ, first at {np.argwhere(bad)[0]}"


@pytest.mark.parametrize("N,K", [(1, 8), (7, 40), (64, 1024), (100, 5120), (16, 13824), (3, 16392)])
def test_requant_plain_shapes(device, N, K):
    rng = np.random.default_rng(N * 7919 + K)
    _check_plain(O.bf16_encode(rng.standard_normal((N, K), dtype=np.float32) * 0.02), device)


def test_requant_plain_exhaustive(device):
    """Every (row max, element) pair through the weight path's double rounding."""
    for i, w in enumerate(exhaustive_chunks()):
        if i % 16 == 0:
            print(f"exhaustive weight chunk {i}", flush=True)
        _check_plain(w, device)


def test_requant_qkv_weight_full(device):
    from vdn_fp8 import workloads
    _, w, _ = workloads.dit_qkv(M=8)
    _check_plain(bits(w), device)


def _lora_case(rng, N, K, r, std_w=0.02, std_ab=0.01):
    w = O.bf16_encode(rng.standard_normal((N, K), dtype=np.float32) * std_w)
    a = O.bf16_encode(rng.standard_normal((r, K), dtype=np.float32) * std_ab)
    b = O.bf16_encode(rng.standard_normal((N, r), dtype=np.float32) * std_ab)
    return w, a, b


def _bf16_ulp(v):
    """The bf16 ulp at |v| (float64 in, float64 out; 2^-133 for zero/subnormals)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def _check_lora(w, a, b, scale, device, max_mismatch=2e-3):
    lora = (from_bits(a, device), from_bits(b, device), scale)
    gq, gs, gm = _requant(w, device, lora=lora, merged=True)
    want_m = O.lora_merge(w, a, b, scale)
    # merged weight: exact almost everywhere; elsewhere one bf16 ulp at the scale of the
    # operands (W and the update), because a one-ulp flip of bf16(delta) -- fp32
    # summation order -- survives a cancelling add unchanged.
    gv, wv, w0 = (O.bf16_decode(t).astype(np.float64) for t in (gm, want_m, w))
    tol = _bf16_ulp(np.maximum(np.maximum(np.abs(w0), np.abs(wv - w0)), np.abs(wv)))
    err = np.abs(gv - wv)
    assert np.all(err <= tol), f"merged weight off by {np.max(err / tol):.2f} ulp"
    assert np.mean(gm != want_m) <= max_mismatch, f"{np.mean(gm != want_m):.2e} of merged values differ"
    # codes: bit-exact given the kernel's merged weight
    wq, ws = O.quantize_weight(gm)
    assert np.array_equal(gs.view(np.uint32), ws.view(np.uint32))
    assert np.all(same_codes(gq, wq))


@pytest.mark.parametrize("N,K,r", [(16, 256, 64), (40, 1024, 16), (33, 4096, 64), (64, 5120, 128),
                                   (17, 6144, 32), (20, 8192, 96), (18, 14336, 64), (5, 16384, 8),
                                   # odd ranks (2-byte B rows), partial column stripes, one row,
                                   # partial row tiles
                                   (24, 2048, 5), (70, 1280, 33), (9, 272, 19), (130, 4112, 64),
                                   (1, 5120, 64), (200, 768, 127),
                                   # one-pass row groups of 28 rows with a short last group, and
                                   # two rounds of 18-row groups over uneven workgroups
                                   (6999, 2048, 32), (9000, 1024, 64)])
def test_requant_lora_shapes(device, N, K, r):
    print(f"lora requant N={N} K={K} r={r}", flush=True)
    rng = np.random.default_rng(N + K + r)
    w, a, b = _lora_case(rng, N, K, r)
    _check_lora(w, a, b, 1.0, device)


def test_requant_lora_scale(device):
    rng = np.random.default_rng(3)
    w, a, b = _lora_case(rng, 48, 2048, 64, std_ab=0.05)
    _check_lora(w, a, b, 0.25, device)


def test_requant_lora_workload(device):
    """Base QKV weight [15360, 5120] + rank-64 LoRA (alpha 64), whole."""
    from vdn_fp8 import workloads
    w0, a, b, scale, _ = workloads.dit_lora(M=8)
    _check_lora(bits(w0), bits(a), bits(b), scale, device)


@pytest.mark.parametrize("r", [64, 19])
def test_requant_lora_edge_rows(device, r):
    """Rows with inf / NaN in W or in the LoRA factors, zero and negative-zero rows,
    subnormal rows, a row whose merge overflows bf16, and rows the update dominates:
    the scales and codes bit-exact with the oracle's quantization of the kernel's own
    merged weight, the merged weight within one bf16 ulp (same class where not finite)."""
    rng = np.random.default_rng(77 + r)
    N, K = 40, 1024
    w = rng.standard_normal((N, K), dtype=np.float32) * 0.02
    a = rng.standard_normal((r, K), dtype=np.float32) * 0.01
    b = rng.standard_normal((N, r), dtype=np.float32) * 0.01
    w[0, 5] = np.inf
    w[1, 700] = np.nan
    w[2], b[2] = 0.0, 0.0
    w[3], b[3] = -0.0, 0.0
    w[4], b[4] = 1e-39, 0.0
    w[5, 100], b[5] = 3.38e38, 3e37
    b[6, 3] = np.inf
    b[7, 0] = np.nan
    w[8], b[8] = -300.0, 0.0
    b[10] = 5.0
    w[11, 1023] = -np.inf
    w, a, b = (O.bf16_encode(t) for t in (w, a, b))
    lora = (from_bits(a, device), from_bits(b, device), 1.0)
    gq, gs, gm = _requant(w, device, lora=lora, merged=True)
    want_m = O.lora_merge(w, a, b, 1.0)
    gv, wv, w0 = (O.bf16_decode(t).astype(np.float64) for t in (gm, want_m, w))
    fin = np.isfinite(wv)
    assert np.array_equal(np.isnan(gv), np.isnan(wv)), "NaN positions differ"
    assert np.array_equal(gv[np.isinf(wv)], wv[np.isinf(wv)]), "infinities differ"
    with np.errstate(invalid="ignore", over="ignore"):
        tol = _bf16_ulp(np.maximum(np.maximum(np.abs(w0), np.abs(wv - w0)), np.abs(wv)))
    assert np.all(np.abs(gv - wv)[fin] <= tol[fin])
    wq, ws = O.quantize_weight(gm)
    same_scale = (gs.view(np.uint32) == ws.view(np.uint32)) | (np.isnan(gs) & np.isnan(ws))
    assert same_scale.all(), f"scales differ in rows {np.flatnonzero(~same_scale)}"
    bad = ~same_codes(gq, wq)
    assert not bad.any(), f"{bad.sum()} codes differ, rows {np.unique(np.argwhere(bad)[:, 0])}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_requant_lora_float_factors(device, dtype):
    """fp16 / fp32 adapter factors (external LoRA files): the reference's fp32 update
    bf16((B @ A) * scale) added in bf16 (lora.py:91-92), then the requantization; the
    merged weight within one bf16 ulp of a float64 restatement, the codes bit-exact with
    the oracle's quantization of the kernel's merged weight; merge_into the same."""
    from vdn_fp8.lora import merge_into
    rng = np.random.default_rng(31)
    N, K, r, scale = 96, 1024, 16, 0.5
    w = O.bf16_encode(rng.standard_normal((N, K), dtype=np.float32) * 0.02)
    a = (rng.standard_normal((r, K)) * 0.05).astype(np.float32)
    b = (rng.standard_normal((N, r)) * 0.05).astype(np.float32)
    at, bt = torch.from_numpy(a).to(dtype), torch.from_numpy(b).to(dtype)
    a64, b64 = at.double().numpy(), bt.double().numpy()
    d16 = O.bf16_encode(((b64 @ a64) * scale).astype(np.float32))
    want = O.bf16_encode(O.bf16_decode(w) + O.bf16_decode(d16))
    w0 = O.bf16_decode(w).astype(np.float64)
    wv = O.bf16_decode(want).astype(np.float64)
    tol = _bf16_ulp(np.maximum(np.maximum(np.abs(w0), np.abs(wv - w0)), np.abs(wv)))
    gq, gs, gm = _requant(w, device, lora=(at.to(device), bt.to(device), scale), merged=True)
    assert np.all(np.abs(O.bf16_decode(gm).astype(np.float64) - wv) <= tol)
    assert np.mean(gm != want) <= 2e-3
    wq, ws = O.quantize_weight(gm)
    assert np.array_equal(gs.view(np.uint32), ws.view(np.uint32))
    assert np.all(same_codes(gq, wq))
    wt = from_bits(w, device)
    merge_into(wt, at, bt, scale)          # factors on the host: moved by merge_into
    torch.cuda.synchronize()
    assert np.array_equal(bits(wt), gm)


def test_merge_only_in_place(device):
    """merge_lora_state's in-place update (wq = NULL): W' written over W."""
    from vdn_fp8.lora import merge_into
    rng = np.random.default_rng(9)
    w, a, b = _lora_case(rng, 64, 5120, 64)
    wt = from_bits(w, device)
    merge_into(wt, from_bits(a, device), from_bits(b, device), 1.0)
    torch.cuda.synchronize()
    got = bits(wt)
    want = O.lora_merge(w, a, b, 1.0)
    gv, wv, w0 = (O.bf16_decode(t).astype(np.float64) for t in (got, want, w))
    tol = _bf16_ulp(np.maximum(np.maximum(np.abs(w0), np.abs(wv - w0)), np.abs(wv)))
    assert np.all(np.abs(gv - wv) <= tol)
    assert np.mean(got != want) <= 2e-3
