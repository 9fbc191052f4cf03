"""The HIP quantizers divide by the row scale as q0 = x * RN(1/s), then one
remainder fma correction. tests/native/division_check.c proves, exhaustively over
every (row max, element) bf16 pair, that this yields the same e4m3 code (and, for
the weight path, the same bf16-then-e4m3 code) as the IEEE quotient -- and that on the
weight path, where both operands are bf16, the single product x * RN(1/s) already
rounds to the same bf16 value as the IEEE quotient (what the weight kernels use)."""
import os
import shutil
import subprocess

import pytest

from conftest import ROOT

SRC = os.path.join(ROOT, "tests", "native", "division_check.c")
ORACLE_C = os.path.join(ROOT, "oracle", "fp8_oracle.c")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_reciprocal_fma_division_is_exact_on_codes(tmp_path):
    exe = tmp_path / "division_check"
    subprocess.run(["gcc", "-O2", "-std=gnu99", "-ffp-contract=off", "-fopenmp", SRC, ORACLE_C, "-o", str(exe),
                    "-lm", "-lpthread"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "code mismatches: activation 0, weight 0" in r.stdout
    assert "weight path, single multiply: bf16 mismatches 0" in r.stdout
