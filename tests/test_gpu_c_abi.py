"""The handoff driven from plain C through include/iekv.h, with no Python in the data path (GPU).

tests/c_abi_handoff.c (built by __graft_entry__.build() against the in-tree
libiekv.so) allocates two pools in one HIP allocation, runs a direct copy with
device ids, one with host ids, and a pack -> unpack, then checks every byte; then
offloads to and restores from host memory, pinned (read and written by the move
kernel directly) and pageable (the staged pipelines), checking every byte again.
"""
from __future__ import annotations

import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu


def test_a_c_program_hands_off_through_the_c_abi(gpu):
    exe = ROOT / "tests" / "c_abi_handoff"
    if not exe.exists():
        pytest.fail(f"{exe} is not built (run __graft_entry__.build())")
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, (out.returncode, out.stdout, out.stderr)
    assert out.stdout.startswith("c-abi handoff ok")
