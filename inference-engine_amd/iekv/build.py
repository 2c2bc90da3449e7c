"""Build libiekv.so (the HIP kernels and their C-ABI) in-tree for gfx950.

The library is compiled with hipcc straight from ``csrc/kv_handoff.hip`` into
``iekv/libiekv.so`` next to this file, so it travels with the source tree and
is the file ``iekv._native`` loads. Run ``python -m iekv.build`` (with
``inference-engine_amd`` on ``sys.path``) or call :func:`build`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR.parent / "csrc"
REPO_ROOT = PACKAGE_DIR.parent.parent
INCLUDE_DIR = REPO_ROOT / "include"
LIBRARY = PACKAGE_DIR / "libiekv.so"
SOURCES = [SOURCE_DIR / "kv_handoff.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: install ROCm or put hipcc on PATH")
    return found


def command(output: Path = LIBRARY) -> list[str]:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # Packed FP32 instructions stay disabled in every HIP build here.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        f"-I{INCLUDE_DIR}",
        *[str(s) for s in SOURCES],
        "-o", str(output),
    ]


def build(verbose: bool = False) -> Path:
    """Compile libiekv.so; raises RuntimeError with the compiler output on failure."""
    tmp = LIBRARY.with_name(LIBRARY.name + f".tmp{os.getpid()}")
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        tmp.unlink(missing_ok=True)
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
