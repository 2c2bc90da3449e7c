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
takes the chunk size its rule gives it (launch_chunk). Thirteen mistakes planted one
at a time in a copy of the header (seven in the launch planning, six in the host-address
arithmetic) each make it fail.
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


# Mistakes planted one at a time in a copy of kv_plan.h: each is a plausible slip in
# the planning the kernels rely on, and plan_check must fail on every one of them.
# (name, the header's text, the same text with the mistake)
MISTAKES = [
    ("xcd remainder dropped",
     "return x * q + (x < rem ? x : rem) + i / kXcds;",
     "return x * q + i / kXcds;"),
    ("diagonal taken modulo the units",
     "pl.r = static_cast<int>((static_cast<int64_t>(pl.r) + pl.a) % runs);",
     "pl.r = static_cast<int>((static_cast<int64_t>(pl.r) + pl.a) % n_units);"),
    ("no halving of the split at the dispatch limit",
     "  while (pl->parts > 1 && pl->total_runs * n_arrays * pl->parts > kMaxGrid) pl->parts /= 2;\n",
     ""),
    ("tile group not capped at the array count",
     "return static_cast<int>(group < n_arrays ? group : n_arrays);",
     "return static_cast<int>(group);"),
    ("unit count truncated",
     "pl->units = (n_arrays + pl->group - 1) / pl->group;",
     "pl->units = n_arrays / pl->group;"),
    ("unpack chunk rule with a strict comparison",
     "tile_bytes >= pool_chunk ? pool_chunk",
     "tile_bytes > pool_chunk ? pool_chunk"),
    ("launch grid without the chunk factor",
     "return static_cast<uint32_t>(runs * pl.units * pl.parts);",
     "return static_cast<uint32_t>(runs * pl.units);"),
    # The host-address arithmetic of the host-memory transfers.
    ("a copy run past its first image's allocation",
     "static_cast<int64_t>(len + 1) * image_bytes <= space)",
     "space >= 0)"),
    ("a looked-up allocation reused for an image that runs past its end",
     "if (!(have && p >= lo && p + static_cast<uint64_t>(bytes) <= hi)) {",
     "if (!(have && p >= lo && p < hi)) {"),
    ("an image longer than the rest of its allocation accepted",
     "if (!span.mapped || span.room < bytes) return false;",
     "if (!span.mapped) return false;"),
    ("two staging slots when the buffer holds one image",
     "*n_slots = fit >= 2 ? 2 : 1;",
     "*n_slots = 2;"),
    ("more images per launch than the argument block holds",
     "  if (per > max_images) per = max_images;\n",
     ""),
    # The request queue's claims.
    ("a descriptor's claims not capped",
     "  if (k < least_k) k = least_k;\n",
     ""),
    ("the last claim of a block dropped",
     "c.per_block = (units + k - 1) / k;",
     "c.per_block = units / k;"),
    ("claims never larger than one unit for a big request",
     "if (k > max_k) k = max_k;",
     "if (k > 1) k = 1;"),
    ("queue tile groups for tiles that do not divide the wave",
     "tile_vecs * vec_bytes >= chunk_bytes || kQueueWave % tile_vecs)",
     "tile_vecs * vec_bytes >= chunk_bytes)"),
    ("claims spanning two blocks",
     "  if (k > units) k = units;\n",
     ""),
    ("touching pools counted as overlapping",
     "if (reach[1 - s.owner] > s.lo) return true;",
     "if (reach[1 - s.owner] >= s.lo) return true;"),
]


@pytest.mark.parametrize("name,right,wrong", MISTAKES, ids=[m[0] for m in MISTAKES])
def test_each_planted_mistake_fails_the_check(tmp_path, name, right, wrong):
    """The check has teeth: with any one of these mistakes in the header, plan_check
    names a failure instead of printing "plan ok"."""
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    header = (ROOT / "inference-engine_amd" / "csrc" / "kv_plan.h").read_text()
    assert header.count(right) == 1, f"{name}: the header no longer holds {right!r}"
    (tmp_path / "inference-engine_amd" / "csrc").mkdir(parents=True)
    (tmp_path / "tests").mkdir()
    (tmp_path / "inference-engine_amd" / "csrc" / "kv_plan.h").write_text(
        header.replace(right, wrong))
    shutil.copy(ROOT / "tests" / "plan_check.cpp", tmp_path / "tests" / "plan_check.cpp")
    exe = tmp_path / "plan_check"
    subprocess.run([gxx, "-std=c++17", "-O2", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    str(tmp_path / "tests" / "plan_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True, timeout=300)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert out.returncode != 0 and not out.stdout.strip().endswith("plan ok"), \
        f"{name}: plan_check passed with the mistake planted"
