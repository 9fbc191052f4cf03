"""ctypes binding of libvdnfp8.so (include/vdn_fp8.h).

The library is required: there is no CPU or torch fallback for any entry point.
Loading fails loudly when the shared library is missing, was built for another ABI
version, or was built from sources other than the ones beside it (its embedded
source manifest, vdn_fp8_build_info, must match the csrc/ and include/ files on disk,
the build flags and, where hipcc is installed, the compiler's identity).
"""
import ctypes
import json
import os

from .build import CSRC, INCLUDE, LIB_PATH, compiler_id, source_manifest

ABI_VERSION = 5

OK, EINVAL, ELAUNCH = 0, 1, 2
EPI_NONE, EPI_GELU_TANH, EPI_GATE, EPI_F32 = 0, 1, 2, 3
DTYPE_BF16, DTYPE_F16, DTYPE_F32 = 0, 1, 2

_lib = None
_build_info = None

# (name, restype, argtypes) of every exported symbol, in header order.
_P, _I64, _F32, _I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
EXPORTS = (
    ("vdn_fp8_quantize_rows", _I32, [_P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    ("vdn_fp8_gelu_quantize_rows", _I32, [_P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    ("vdn_fp8_swiglu_quantize_rows", _I32, [_P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    ("vdn_fp8_norm_quantize_rows", _I32, [_P, _I64, _I64, _I64, _P, _F32, _P, _P, _I64, _P, _I64, _P, _I64, _P,
                                          _P, _I64, _P]),
    ("vdn_fp8_requantize_weight", _I32, [_P, _I64, _I64, _I64, _P, _P, _I64, _F32, _P, _I64, _P, _P, _P]),
    ("vdn_fp8_quantize_rows_typed", _I32, [_P, _I32, _I64, _I64, _I64, _P, _I64, _P, _P]),
    ("vdn_fp8_swiglu_quantize_rows_typed", _I32, [_P, _I32, _I64, _I64, _I64, _P, _I64, _P, _P]),
    ("vdn_fp8_requantize_weight_typed", _I32, [_P, _I32, _I64, _I64, _I64, _P, _I64, _P, _P]),
    ("vdn_fp8_gemm", _I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I32, _P, _P, _I64, _I64,
                            _P, _I64, _P, _I64, _P]),
    ("vdn_fp8_gemm_workspace_size", _I32, [_I64, _I64, _I64, _P]),
    ("vdn_fp8_gemm_ws", _I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I32, _P, _P, _I64, _I64,
                               _P, _I64, _P, _I64, _P, _I64, _P]),
    ("vdn_fp8_gemm_noalloc", _I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I32, _P, _P, _I64, _I64,
                                    _P, _I64, _P, _I64, _P]),
    ("vdn_fp8_qk_prep", _I32, [_P, _I64, _I64, _I64, _I64, _P, _F32, _P, _P, _I64, _I64, _I32, _P, _I64, _P]),
    ("vdn_fp8_gated_residual", _I32, [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P]),
    ("vdn_fp8_last_error", ctypes.c_char_p, []),
    ("vdn_fp8_abi_version", _I32, []),
    ("vdn_fp8_build_info", ctypes.c_char_p, []),
)


class Fp8LibraryError(RuntimeError):
    """A launch the HIP runtime refused (status ELAUNCH)."""


def _check_sources(lib, path):
    """Refuse a library whose embedded source manifest differs from the sources on
    disk. The sources looked at are the package's csrc/ and include/, or
    VDN_FP8_SOURCE_DIR (a directory holding csrc/ and include/) for a library built
    from another tree."""
    info = json.loads(lib.vdn_fp8_build_info().decode())
    src_root = os.environ.get("VDN_FP8_SOURCE_DIR")
    csrc, include = (os.path.join(src_root, "csrc"), os.path.join(src_root, "include")) if src_root \
        else (CSRC, INCLUDE)
    # the compiler is compared where one is installed (a machine without hipcc cannot
    # rebuild, and checks the sources and flags alone)
    compiler = compiler_id() or info.get("compiler", "unknown")
    try:
        want = source_manifest(csrc, include, compiler)
    except FileNotFoundError as e:
        raise RuntimeError(f"cannot check {path} against its sources ({e}); the fp8 library ships with "
                           "its csrc/ and include/ trees") from None
    if info.get("digest") != want["digest"]:
        stale = sorted(f for f, h in want["sources"].items() if info.get("sources", {}).get(f) != h)
        if not stale and info.get("flags") != want["flags"]:
            stale = ["build flags"]
        if not stale and info.get("compiler") != want["compiler"]:
            stale = [f"compiler ({info.get('compiler')!r}, installed {want['compiler']!r})"]
        raise RuntimeError(
            f"{path} was built from other sources than {csrc} / {include} "
            f"(differs in: {', '.join(stale) or 'manifest'}): rebuild it (python "
            f"vdn-minimax-h3_amd/vdn_fp8/build.py, or __graft_entry__.build())")
    return info


def load(path=None):
    """Load (once) and return the library handle; raises if it is absent or stale."""
    global _lib, _build_info
    if _lib is not None:
        return _lib
    path = path or os.environ.get("VDN_FP8_LIB", LIB_PATH)
    if not os.path.exists(path):
        raise RuntimeError(
            f"libvdnfp8.so not found at {path}: build it first (python "
            f"vdn-minimax-h3_amd/vdn_fp8/build.py, or __graft_entry__.build()). "
            "The fp8 path has no fallback.")
    lib = ctypes.CDLL(path)
    version = lib.vdn_fp8_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI {version}, expected {ABI_VERSION}: rebuild it")
    for name, res, args in EXPORTS:
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    _build_info = _check_sources(lib, path)
    _lib = lib
    return lib


def build_info():
    """The loaded library's source manifest (see vdn_fp8.build.source_manifest)."""
    load()
    return _build_info


def check(status, what):
    """Turn a C status into the reference's exception types."""
    if status == OK:
        return
    msg = load().vdn_fp8_last_error().decode(errors="replace")
    if status == EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise Fp8LibraryError(f"{what}: {msg}")
