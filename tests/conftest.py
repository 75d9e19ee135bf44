"""Shared pytest configuration.

Tests marked ``gpu`` run the HIP library on a ROCm device and compare it
with the oracle (the CPU restatement under oracle/).  Everything else runs
on the CPU: the oracle against the reference-generated golden vectors and
known-answer tests, host-side logic, and the C ABI's exported symbols.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a ROCm GPU and libsuffixgpu_amd.so")


def golden(name: str):
    return np.load(GOLDEN / f"{name}.npz")


@pytest.fixture(scope="session")
def gpu():
    """The ROCm device; fails (not skips) when the HIP library is absent."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from suffixgpu_amd import _lib
    _lib.lib()
    return torch.device("cuda", 0)
