"""ctypes binding of libvdnfp8.so (include/vdn_fp8.h).

The library is required: there is no CPU or torch fallback for any entry point.
Loading fails loudly when the shared library is missing or was built for another
ABI version.
"""
import ctypes
import os

from .build import LIB_PATH

ABI_VERSION = 1

OK, EINVAL, ELAUNCH = 0, 1, 2
EPI_NONE, EPI_GELU_TANH, EPI_GATE = 0, 1, 2

_lib = None

# (name, restype, argtypes) of every exported symbol, in header order.
_P, _I64, _F32, _I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
EXPORTS = (
    ("vdn_fp8_quantize_rows", _I32, [_P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    ("vdn_fp8_swiglu_quantize_rows", _I32, [_P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    ("vdn_fp8_norm_quantize_rows", _I32, [_P, _I64, _I64, _I64, _P, _F32, _P, _P, _I64, _P, _I64, _P, _I64, _P,
                                          _P, _I64, _P]),
    ("vdn_fp8_requantize_weight", _I32, [_P, _I64, _I64, _I64, _P, _P, _I64, _F32, _P, _I64, _P, _P, _P]),
    ("vdn_fp8_gemm", _I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I32, _P, _P, _I64, _I64,
                            _P, _I64, _P, _I64, _P]),
    ("vdn_fp8_qk_prep", _I32, [_P, _I64, _I64, _I64, _I64, _P, _F32, _P, _P, _I64, _I64, _I32, _P, _I64, _P]),
    ("vdn_fp8_gated_residual", _I32, [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P]),
    ("vdn_fp8_last_error", ctypes.c_char_p, []),
    ("vdn_fp8_abi_version", _I32, []),
)


class Fp8LibraryError(RuntimeError):
    """A launch the HIP runtime refused (status ELAUNCH)."""


def load(path=None):
    """Load (once) and return the library handle; raises if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or os.environ.get("VDN_FP8_LIB", LIB_PATH)
    if not os.path.exists(path):
        raise RuntimeError(
            f"libvdnfp8.so not found at {path}: build it first (python "
            f"vdn-minimax-h3_amd/vdn_fp8/build.py, or __graft_entry__.build()). "
            "The fp8 path has no fallback.")
    lib = ctypes.CDLL(path)
    for name, res, args in EXPORTS:
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    if lib.vdn_fp8_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI {lib.vdn_fp8_abi_version()}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def check(status, what):
    """Turn a C status into the reference's exception types."""
    if status == OK:
        return
    msg = load().vdn_fp8_last_error().decode(errors="replace")
    if status == EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise Fp8LibraryError(f"{what}: {msg}")
