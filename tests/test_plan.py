"""The kv_move launch planning (inference-engine_amd/csrc/kv_plan.h) checked on the CPU.

tests/plan_check.cpp includes the header the kernels use and checks it
exhaustively: the XCD-grouped workgroup order is a bijection, every workgroup
order visits each (array unit, run, chunk) once, plans respect the dispatch
limit, chunk and tile-group rules, a simulation of every launch and
workgroup of small plans moves every vector of every tile exactly once, and
the copies of a scattered restore (image_runs) merge exactly the images that
are adjacent within one allocation, over fixed and random layouts; the device
addresses of direct host transfers (image_views), the launch and staging-slot
splits of the host pipelines, and the pool-overlap test (spans_cross) hold at
the 70B-share workload's numbers and on random layouts; each kind of launch
takes the chunk size its rule gives it (launch_chunk).
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


# Optimised, then with AddressSanitizer and UndefinedBehaviorSanitizer: any report
# (an access outside an object, a signed overflow, a misaligned load) ends the run
# with a non-zero status. CPU-only code: g++, no GPU code involved.
BUILDS = {"optimised": ["-O2"],
          "sanitized": ["-O1", "-g", "-fsanitize=address,undefined",
                        "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]}


@pytest.mark.parametrize("build", list(BUILDS))
def test_the_launch_plan_covers_every_tile_once(tmp_path, build):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    exe = tmp_path / "plan_check"
    subprocess.run([gxx, "-std=c++17", *BUILDS[build], "-Wall", "-Wextra", "-Werror",
                    "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    str(ROOT / "tests" / "plan_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True, timeout=300)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0 and out.stdout.strip().endswith("plan ok"), \
        (out.stdout[-3000:] + out.stderr[-3000:])
