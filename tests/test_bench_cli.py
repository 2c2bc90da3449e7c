"""bench.py's command-line refusals (CPU): each happens before any GPU is touched."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.parametrize("args,message", [
    (["--gpus", "2"], "measures one GPU"),
    (["--legs", "write_kv,gather_context"], "needs one handoff leg"),
    (["--config", "cfg2", "--tp", "4"], "does not divide"),
    (["--config", "cfg9"], "unknown workload"),
    (["--config", "cfg5", "--slack", "3"], "fixed pool sizes"),
    (["--ab", "streams=0,2"], "--ab takes"),
    (["--ab", "width=4"], "--ab takes"),
    (["--config", "cfg5", "--ab", "slack=64,engine"], "--ab takes"),
    (["--ab", "direct_chunk=4096,3000"], "--ab takes"),
    (["--ab", "direct_chunk=32"], "--ab takes"),
    (["--ab", "pack_order=0,3"], "--ab takes"),
    (["--ab", "unroll=0"], "--ab takes"),
])
def test_the_bench_refuses_before_touching_a_gpu(args, message):
    out = subprocess.run([sys.executable, "bench.py", *args], cwd=ROOT, capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 2 and message in out.stderr, out.stderr[-2000:]
