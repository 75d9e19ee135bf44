"""Register and scratch budget of the step kernels, from the compiler's
resource report (hipcc cross-compiles for gfx950 without a GPU).

Two 512-thread workgroups of the fused step share a CU only while it needs
at most 128 VGPRs (4 waves per SIMD); spilling to scratch would put every
step on the slow path.  Both happened once by accident, so they are
checked here.  The fused step kernel's launches past twice the CU count
size every role for three workgroups per CU, which needs at most 80 VGPRs
(6 waves per SIMD)."""

from __future__ import annotations

import re
import shutil
import subprocess

import pytest

from suffixgpu_amd import build

HIPCC = build.HIPCC


def _resources(src: str, tmp_path) -> dict[str, dict[str, int]]:
    cmd = [HIPCC, *build.COMMON, "-c", str(build.CSRC / src), "-o",
           str(tmp_path / "k.o"), "-Rpass-analysis=kernel-resource-usage"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    out: dict[str, dict[str, int]] = {}
    name = None
    for line in res.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            out[name] = {}
            continue
        m = re.search(r"remark:\s+(VGPRs|ScratchSize \[bytes/lane\]|"
                      r"Occupancy \[waves/SIMD\]): (\d+)", line)
        if m and name:
            out[name][m.group(1).split()[0]] = int(m.group(2))
    return out


@pytest.mark.skipif(shutil.which(HIPCC) is None and
                    not __import__("os").path.exists(HIPCC),
                    reason="needs hipcc")
@pytest.mark.parametrize("src,kernel", [("step.hip", "k_step"),
                                        ("local.hip", "k_local"),
                                        ("global.hip", "k_global")])
def test_step_kernels_fit_two_workgroups_per_cu(src, kernel, tmp_path):
    res = _resources(src, tmp_path)
    found = {k: v for k, v in res.items() if kernel in k}
    assert found, f"no {kernel} in the resource report"
    for name, r in found.items():
        assert r["ScratchSize"] == 0, (name, r)
        assert r["VGPRs"] <= 128, (name, r)
        assert r["Occupancy"] >= 4, (name, r)
        if kernel == "k_step":
            assert r["VGPRs"] <= 80 and r["Occupancy"] >= 6, (name, r)


@pytest.mark.skipif(shutil.which(HIPCC) is None and
                    not __import__("os").path.exists(HIPCC),
                    reason="needs hipcc")
def test_sa_local_round_fits_two_workgroups_per_cu(tmp_path):
    """The suffix-array build's local round (1024 threads, 24 KiB of LDS):
    at most 64 VGPRs (eight waves per SIMD) and no scratch.  A cross-lane
    read feeding its sort decision once pushed it to 128 VGPRs with 376
    bytes of scratch per lane."""
    res = _resources("sa_build.hip", tmp_path)
    found = {k: v for k, v in res.items() if "k_sa_local" in k}
    assert found, "no k_sa_local in the resource report"
    for name, r in found.items():
        assert r["ScratchSize"] == 0, (name, r)
        assert r["VGPRs"] <= 64, (name, r)
        assert r["Occupancy"] >= 8, (name, r)
