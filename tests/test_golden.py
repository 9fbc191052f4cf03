"""The oracle reproduces the committed golden fixtures (written from torch's eager
spellings of the reference functions by tests/golden/make_golden.py), and the
seeded workload generator still draws the same bits (sha256 of the inputs)."""
import hashlib
import json
import os

import numpy as np

import oracle as O
from conftest import GOLDEN_DIR, bits


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_prompt_rows_codes_and_scales():
    d = np.load(os.path.join(GOLDEN_DIR, "prompt_rows.npz"))
    q, s = O.quantize_rows(d["x"])
    assert np.array_equal(q, d["codes"])
    assert np.array_equal(s.view(np.uint32), d["scale"].view(np.uint32))


def test_single_linear_workload():
    from vdn_fp8 import workloads
    g = json.load(open(os.path.join(GOLDEN_DIR, "single.json")))
    x, w, b = workloads.dit_single()
    assert sha(bits(x)) == g["x"] and sha(bits(w)) == g["w"] and sha(bits(b)) == g["bias"], \
        "torch's CPU generator drew different inputs"
    qx, sx = O.quantize_rows(bits(x))
    qw, sw = O.quantize_weight(bits(w))
    assert sha(qx) == g["x_codes"] and sha(sx) == g["x_scale"]
    assert sha(qw) == g["w_codes"] and sha(sw) == g["w_scale"]
    out = O.dequant_linear(qx, sx, qw, sw, bias=bits(b), rounding="none")
    np.testing.assert_allclose(out.sum(), g["out_sum"], rtol=1e-9)
    np.testing.assert_allclose((out * out).sum(), g["out_sumsq"], rtol=1e-9)
    np.testing.assert_allclose(out[0, :8], g["out_first_row_head"], rtol=1e-9)


def test_lora_small():
    d = np.load(os.path.join(GOLDEN_DIR, "lora_small.npz"))
    merged = O.lora_merge(d["w"], d["a"], d["b"], float(d["scale"]))
    ulps = np.abs(merged.astype(np.int32) - d["merged"].astype(np.int32))
    assert np.mean(ulps != 0) < 1e-2 and ulps.max() <= 1
    q, s = O.quantize_weight(d["merged"])
    assert np.array_equal(q, d["codes"])
    assert np.array_equal(s.view(np.uint32), d["w_scale"].view(np.uint32))


import pytest


@pytest.mark.parametrize("name", ["dit_qkv", "dit_ffn_up", "dit_ffn_down_attn_out", "dit_lora"])
def test_full_size_draws_are_pinned(name):
    """Every full-size configuration draw (cfg2-5) still has the committed sha256: the
    benchmark and the parity tests run on exactly these inputs."""
    from vdn_fp8 import workloads
    assert workloads.draw_digests(name) == workloads.DRAW_SHA256[name], \
        "torch's CPU generator drew different inputs"


def test_single_draw_pin_matches_golden():
    from vdn_fp8 import workloads
    g = json.load(open(os.path.join(GOLDEN_DIR, "single.json")))
    assert workloads.DRAW_SHA256["dit_single"] == {"x": g["x"], "w": g["w"], "bias": g["bias"]}
