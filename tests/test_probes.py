"""The standalone measurement programs that profiles/ cites build for gfx950 (no GPU needed).

csrc/hbm_ceiling_probe.hip (the HBM streaming ceilings, profiles/hbm_ceilings.txt)
and csrc/launch_cost_probe.hip (the host's cost of a launch against its kernel-argument
bytes, profiles/launch_floor.txt) are not part of libiekv.so; each profile gives the
hipcc command that builds it, and this test runs exactly that command.
"""
from __future__ import annotations

import shutil
import subprocess

import pytest

from conftest import ROOT

PROBES = {
    "hbm_ceiling_probe": "profiles/hbm_ceilings.txt",
    "launch_cost_probe": "profiles/launch_floor.txt",
}


@pytest.mark.parametrize("probe", sorted(PROBES))
def test_the_measurement_program_builds_as_its_profile_says(tmp_path, probe):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not shutil.which(hipcc):
        pytest.skip("hipcc is not installed")
    source = f"inference-engine_amd/csrc/{probe}.hip"
    profile = (ROOT / PROBES[probe]).read_text()
    assert source in profile, f"{PROBES[probe]} no longer gives the command for {source}"
    exe = tmp_path / probe
    out = subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                          "-target-feature", "-Xclang", "-packed-fp32-ops", str(ROOT / source),
                          "-o", str(exe)], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-3000:]
    assert exe.stat().st_size > 0
