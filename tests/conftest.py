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


def keys_by_definition(corpus: torch.Tensor, sa: torch.Tensor,
                       keys: torch.Tensor, width: int = 32,
                       rows: int = 1 << 18) -> None:
    """Key row r holds corpus[sa[r] + j] for j < width, -1 at or past the
    end: checked with torch gathers on the device, in slices of ranks."""
    import torch
    n = corpus.shape[0]
    kv = keys.view(n, width)
    j = torch.arange(width, device=corpus.device, dtype=torch.int64)
    for r0 in range(0, n, rows):
        pos = sa[r0:r0 + rows].to(torch.int64).unsqueeze(1) + j
        want = torch.where(pos < n, corpus[pos.clamp(max=n - 1)],
                           torch.full_like(pos, -1, dtype=torch.int32))
        bad = (kv[r0:r0 + rows] != want).any(dim=1)
        if bool(bad.any()):
            r = r0 + int(bad.nonzero()[0, 0])
            raise AssertionError(f"key row {r} differs from its definition")
