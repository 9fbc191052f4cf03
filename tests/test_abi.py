"""The C-ABI library (no GPU needed): it loads, exports every symbol that
include/vdn_fp8.h declares, reports its ABI version, and rejects contract
violations with EINVAL before launching anything."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "vdn_fp8.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(vdn_fp8_\w+)\s*\(", text)))


def test_header_declares_the_abi():
    names = declared_symbols()
    assert {"vdn_fp8_quantize_rows", "vdn_fp8_swiglu_quantize_rows", "vdn_fp8_gelu_quantize_rows",
            "vdn_fp8_requantize_weight",
            "vdn_fp8_gemm", "vdn_fp8_norm_quantize_rows", "vdn_fp8_qk_prep", "vdn_fp8_gated_residual",
            "vdn_fp8_last_error",
            "vdn_fp8_abi_version"} <= set(names)


def test_library_exports_every_declared_symbol():
    import vdn_fp8._lib as L
    lib = L.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    bound = {n for n, _, _ in L.EXPORTS}
    assert bound == set(declared_symbols())


def test_abi_version():
    import vdn_fp8._lib as L
    m = re.search(r"#define VDN_FP8_ABI_VERSION (\d+)", open(HEADER).read())
    assert L.load().vdn_fp8_abi_version() == int(m.group(1)) == L.ABI_VERSION


def test_constants_match_header():
    import vdn_fp8._lib as L
    text = open(HEADER).read()
    for name, value in (("VDN_FP8_OK", L.OK), ("VDN_FP8_EINVAL", L.EINVAL), ("VDN_FP8_ELAUNCH", L.ELAUNCH),
                        ("VDN_FP8_EPI_NONE", L.EPI_NONE), ("VDN_FP8_EPI_GELU_TANH", L.EPI_GELU_TANH),
                        ("VDN_FP8_EPI_GATE", L.EPI_GATE), ("VDN_FP8_EPI_F32", L.EPI_F32),
                        ("VDN_FP8_DTYPE_BF16", L.DTYPE_BF16), ("VDN_FP8_DTYPE_F16", L.DTYPE_F16),
                        ("VDN_FP8_DTYPE_F32", L.DTYPE_F32)):
        assert int(re.search(rf"#define {name} (\d+)", text).group(1)) == value


FAKE = 1 << 20        # never dereferenced: every call below fails validation first


@pytest.mark.parametrize("call,needle", [
    (lambda l: l.vdn_fp8_quantize_rows(FAKE, 4, 12, 12, FAKE, 12, FAKE, None), "multiples of 8"),
    (lambda l: l.vdn_fp8_quantize_rows(FAKE, -1, 8, 8, FAKE, 8, FAKE, None), "negative"),
    (lambda l: l.vdn_fp8_quantize_rows(None, 4, 8, 8, FAKE, 8, FAKE, None), "null"),
    (lambda l: l.vdn_fp8_quantize_rows(FAKE + 8, 4, 8, 8, FAKE, 8, FAKE, None), "aligned"),
    (lambda l: l.vdn_fp8_swiglu_quantize_rows(FAKE, 4, 8, 8, FAKE, 8, FAKE, None), "2K"),
    (lambda l: l.vdn_fp8_norm_quantize_rows(FAKE, 4, 8, 8, None, 1e-6, FAKE, None, 8, None, 1, FAKE, 8, FAKE,
                                            None, 8, None), "together"),
    (lambda l: l.vdn_fp8_norm_quantize_rows(FAKE, 4, 8, 8, None, -1.0, None, None, 0, None, 0, FAKE, 8, FAKE,
                                            None, 8, None), "eps"),
    (lambda l: l.vdn_fp8_norm_quantize_rows(FAKE, 4, 8, 8, FAKE, 1e-6, FAKE, FAKE, 8, None, 0, FAKE, 8, FAKE,
                                            None, 8, None), "table"),
    (lambda l: l.vdn_fp8_norm_quantize_rows(FAKE, 4, 16392, 16392, None, 1e-6, None, None, 0, None, 0, FAKE,
                                            16392, FAKE, None, 16392, None), "16384"),
    (lambda l: l.vdn_fp8_requantize_weight(FAKE, 4, 8, 8, FAKE, None, 4, 1.0, FAKE, 8, FAKE, None, None), "together"),
    (lambda l: l.vdn_fp8_requantize_weight(FAKE, 4, 32, 32, FAKE, FAKE, 200, 1.0, FAKE, 32, FAKE, None, None), "rank"),
    (lambda l: l.vdn_fp8_requantize_weight(FAKE, 4, 24, 24, FAKE, FAKE, 8, 1.0, FAKE, 24, FAKE, None, None), "K % 16"),
    (lambda l: l.vdn_fp8_gemm(FAKE, FAKE, FAKE, FAKE, 4, 4, 24, 32, 32, None, 0, None, None, 0, 0, None, 0, FAKE, 4, None), "multiple of 16"),
    (lambda l: l.vdn_fp8_gemm(FAKE, FAKE, FAKE, FAKE, 4, 6, 32, 32, 32, None, 0, None, None, 0, 0, None, 0, FAKE, 8, None), "multiple of 4"),
    (lambda l: l.vdn_fp8_gemm(FAKE, FAKE, FAKE, FAKE, 4, 4, 32, 32, 32, None, 7, None, None, 0, 0, None, 0, FAKE, 4, None), "epilogue"),
    (lambda l: l.vdn_fp8_gemm(FAKE, FAKE, FAKE, FAKE, 4, 4, 32, 32, 32, None, 2, None, None, 0, 0, None, 0, FAKE, 4, None), "gate"),
    (lambda l: l.vdn_fp8_gemm(FAKE, FAKE, FAKE, FAKE, 4, 4, 32, 16, 32, None, 0, None, None, 0, 0, None, 0, FAKE, 4, None), "ldx"),
    (lambda l: l.vdn_fp8_qk_prep(FAKE, 4, 2, 96, 192, None, 1e-6, None, None, 0, 0, 0, FAKE, 192, None), "head dim"),
    (lambda l: l.vdn_fp8_qk_prep(FAKE, 4, 2, 128, 256, None, 1e-6, FAKE, FAKE, 72, 72, 0, FAKE, 256, None), "multiple of 16"),
    (lambda l: l.vdn_fp8_qk_prep(FAKE, 4, 2, 128, 256, None, 1e-6, None, None, 128, 128, 0, FAKE, 256, None), "tables"),
    (lambda l: l.vdn_fp8_qk_prep(FAKE, 4, 2, 128, 128, None, 1e-6, None, None, 0, 0, 0, FAKE, 256, None), "H * d"),
    (lambda l: l.vdn_fp8_qk_prep(FAKE, 4, 200, 128, 25600, None, 1e-6, None, None, 0, 0, 0, FAKE, 25600, None), "16384"),
    (lambda l: l.vdn_fp8_qk_prep(FAKE + 8, 4, 2, 128, 256, None, 1e-6, None, None, 0, 0, 0, FAKE, 256, None), "aligned"),
    (lambda l: l.vdn_fp8_qk_prep(FAKE, 4, 2, 128, 256, None, -1.0, None, None, 0, 0, 0, FAKE, 256, None), "eps"),
    (lambda l: l.vdn_fp8_norm_quantize_rows(FAKE, 4, 8, 8, None, 1e-6, None, None, 0, None, 0, None, 8, None,
                                            None, 8, None), "only when normed"),
    (lambda l: l.vdn_fp8_norm_quantize_rows(FAKE, 4, 8, 8, None, 1e-6, None, None, 0, None, 0, FAKE, 8, None,
                                            FAKE, 8, None), "together"),
    (lambda l: l.vdn_fp8_gated_residual(FAKE, 8, FAKE, 8, None, 1, FAKE, 8, FAKE, 8, 4, 12, None), "multiples of 8"),
    (lambda l: l.vdn_fp8_gated_residual(FAKE, 8, FAKE, 8, None, 0, FAKE, 8, FAKE, 8, 4, 8, None), ">= 1 row"),
    (lambda l: l.vdn_fp8_gated_residual(FAKE, 8, None, 8, None, 1, FAKE, 8, FAKE, 8, 4, 8, None), "null"),
    (lambda l: l.vdn_fp8_gated_residual(FAKE + 8, 8, FAKE, 8, None, 1, FAKE, 8, FAKE, 8, 4, 8, None), "aligned"),
    (lambda l: l.vdn_fp8_quantize_rows_typed(FAKE, 5, 4, 8, 8, FAKE, 8, FAKE, None), "dtype"),
    (lambda l: l.vdn_fp8_quantize_rows_typed(FAKE, 2, 4, 12, 12, FAKE, 12, FAKE, None), "multiples of 8"),
    (lambda l: l.vdn_fp8_quantize_rows_typed(FAKE + 8, 1, 4, 8, 8, FAKE, 8, FAKE, None), "aligned"),
    (lambda l: l.vdn_fp8_quantize_rows_typed(FAKE, 2, -1, 8, 8, FAKE, 8, FAKE, None), "negative"),
    (lambda l: l.vdn_fp8_swiglu_quantize_rows_typed(FAKE, 2, 4, 8, 8, FAKE, 8, FAKE, None), "ldx >= 16"),
    (lambda l: l.vdn_fp8_requantize_weight_typed(None, 1, 4, 8, 8, FAKE, 8, FAKE, None), "null"),
    (lambda l: l.vdn_fp8_gelu_quantize_rows(FAKE, 4, 16392, 16392, FAKE, 16392, FAKE, None), "16384"),
    (lambda l: l.vdn_fp8_gelu_quantize_rows(FAKE, 4, 12, 12, FAKE, 12, FAKE, None), "multiples of 8"),
    (lambda l: l.vdn_fp8_gelu_quantize_rows(FAKE, 4, 16, 8, FAKE, 16, FAKE, None), "ldh, ldy >= K"),
    (lambda l: l.vdn_fp8_gelu_quantize_rows(FAKE + 8, 4, 8, 8, FAKE, 8, FAKE, None), "aligned"),
    (lambda l: l.vdn_fp8_gelu_quantize_rows(None, 4, 8, 8, FAKE, 8, FAKE, None), "null"),
    (lambda l: l.vdn_fp8_gelu_quantize_rows(FAKE, -1, 8, 8, FAKE, 8, FAKE, None), "negative"),
    (lambda l: l.vdn_fp8_gemm(FAKE, FAKE, FAKE, FAKE, 4, 4, 32, 32, 32, FAKE, 3, None, None, 0, 0, None, 0, FAKE, 4, None), "binary32"),
    (lambda l: l.vdn_fp8_gemm(FAKE, FAKE, FAKE, FAKE, 4, 4, 32, 32, 32, None, 3, None, None, 0, 0, None, 0, FAKE + 8, 4, None), "binary32"),
])
def test_contract_violations_are_einval(call, needle):
    import vdn_fp8._lib as L
    lib = L.load()
    assert call(lib) == L.EINVAL
    assert needle in lib.vdn_fp8_last_error().decode()


def test_empty_problems_are_no_ops():
    import vdn_fp8._lib as L
    lib = L.load()
    assert lib.vdn_fp8_quantize_rows(None, 0, 8, 8, None, 8, None, None) == L.OK
    assert lib.vdn_fp8_gelu_quantize_rows(None, 0, 8, 8, None, 8, None, None) == L.OK
    assert lib.vdn_fp8_gemm(None, None, None, None, 0, 16, 32, 32, 32, None, 0, None, None, 0, 0, None, 0, None, 16, None) == L.OK
    assert lib.vdn_fp8_requantize_weight(None, 0, 8, 8, None, None, 0, 1.0, None, 8, None, None, None) == L.OK
    assert lib.vdn_fp8_norm_quantize_rows(None, 0, 8, 8, None, 1e-6, None, None, 0, None, 0, None, 8, None,
                                          None, 8, None) == L.OK
    assert lib.vdn_fp8_qk_prep(None, 0, 2, 128, 256, None, 1e-6, None, None, 0, 0, 0, None, 256, None) == L.OK
    assert lib.vdn_fp8_gated_residual(None, 8, None, 8, None, 1, None, 8, None, 8, 0, 8, None) == L.OK
    for dt in (L.DTYPE_F16, L.DTYPE_F32):
        assert lib.vdn_fp8_quantize_rows_typed(None, dt, 0, 8, 8, None, 8, None, None) == L.OK
        assert lib.vdn_fp8_swiglu_quantize_rows_typed(None, dt, 0, 8, 16, None, 8, None, None) == L.OK
        assert lib.vdn_fp8_requantize_weight_typed(None, dt, 0, 8, 8, None, 8, None, None) == L.OK


def test_check_raises_reference_exception_types():
    import vdn_fp8._lib as L
    lib = L.load()
    lib.vdn_fp8_quantize_rows(FAKE, 4, 12, 12, FAKE, 12, FAKE, None)
    with pytest.raises(ValueError):
        L.check(L.EINVAL, "quantize_rows")
    with pytest.raises(L.Fp8LibraryError):
        L.check(L.ELAUNCH, "gemm")


def test_build_info_matches_the_sources():
    import vdn_fp8._lib as L
    from vdn_fp8 import build as B
    info = L.build_info()
    assert info == B.source_manifest()
    assert set(info["sources"]) == set(B.SOURCES + B.HEADERS + B.PUBLIC_HEADERS)


def test_stale_library_is_refused(tmp_path):
    """A library whose embedded manifest differs from the sources beside it does not load:
    checked in a fresh process against a copy of the sources with one kernel file changed."""
    import shutil
    import subprocess
    import sys
    from vdn_fp8 import build as B
    shutil.copytree(B.CSRC, tmp_path / "csrc")
    shutil.copytree(B.INCLUDE, tmp_path / "include")
    with open(tmp_path / "csrc" / "gemm.hip", "a") as f:
        f.write("\n// changed\n")
    code = ("import sys; sys.path.insert(0, %r)\n"
            "import vdn_fp8._lib as L\n"
            "try:\n    L.load()\nexcept RuntimeError as e:\n    print('REFUSED', e)\n" % os.path.join(ROOT, "vdn-minimax-h3_amd"))
    env = dict(os.environ, VDN_FP8_SOURCE_DIR=str(tmp_path))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert "REFUSED" in r.stdout and "gemm.hip" in r.stdout, r.stdout + r.stderr


def test_library_from_another_compiler_is_refused(tmp_path):
    """The manifest records the compiler's identity: with another hipcc installed (a
    stand-in script on HIPCC reporting another version) the same library does not load."""
    import subprocess
    import sys
    fake = tmp_path / "hipcc"
    fake.write_text("#!/bin/sh\necho 'HIP version: 0.0.0-other'\necho 'AMD clang version 0.0.0 (other)'\n")
    fake.chmod(0o755)
    code = ("import sys; sys.path.insert(0, %r)\n"
            "import vdn_fp8._lib as L\n"
            "try:\n    L.load()\nexcept RuntimeError as e:\n    print('REFUSED', e)\n" % os.path.join(ROOT, "vdn-minimax-h3_amd"))
    env = dict(os.environ, HIPCC=str(fake))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert "REFUSED" in r.stdout and "compiler" in r.stdout, r.stdout + r.stderr
