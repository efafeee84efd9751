"""Test configuration: the `gpu` marker, import paths, and shared helpers.

CPU tests (`-m "not gpu"`) pin the oracle and exercise host logic and the C
ABI's exports; GPU tests (`-m gpu`) run the HIP kernels through the C ABI and
compare against the oracle.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def lib():
    """The loaded libmira_rocm.so (GPU tests: initialised on device 0)."""
    from mira_amd import _lib as L
    lib = L.load()
    if gpu_available():
        L.check(lib.mr_init(0), "mr_init")
    return lib


def bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    """Same dtype, shape and bit pattern (so +0 and -0 differ); every NaN counts as one
    canonical NaN, since NaN payloads are not part of any result's meaning."""
    a, b = np.asarray(a), np.asarray(b)
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    if a.dtype.kind == "f":
        ui = {2: np.uint16, 4: np.uint32, 8: np.uint64}[a.dtype.itemsize]
        an, bn = np.isnan(a), np.isnan(b)
        return bool(np.array_equal(an, bn) and np.array_equal(a[~an].view(ui), b[~bn].view(ui)))
    return bool(np.array_equal(a, b))
