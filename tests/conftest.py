"""Shared test setup: import paths, the `gpu` marker, and small helpers.

CPU tests (`-m "not gpu"`) pin the oracle and exercise the host-side contract; GPU
tests (`-m gpu`) run the HIP library through its C ABI and compare with the oracle.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "vdn-minimax-h3_amd")
ORACLE_DIR = os.path.join(ROOT, "oracle")
GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")
for p in (PKG_DIR, ORACLE_DIR, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def gpu_available():
    import torch
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    return torch.device("cuda:0")


def bits(t):
    """bf16 torch tensor (any device) -> numpy uint16 bit patterns."""
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def codes(t):
    """float8_e4m3fn torch tensor -> numpy uint8 codes."""
    import torch
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def from_bits(a, device=None):
    """numpy uint16 bit patterns -> bf16 torch tensor."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
    return t.to(device) if device is not None else t


def same_codes(got, want):
    """Bit equality of e4m3 codes, treating any two NaN codes as equal."""
    got = np.asarray(got, np.uint8)
    want = np.asarray(want, np.uint8)
    nan = lambda c: (c & 0x7F) == 0x7F
    return (got == want) | (nan(got) & nan(want))
