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
    (["--ab", "pack_order=0,8"], "--ab takes"),
    (["--ab", "unroll=0"], "--ab takes"),
    (["--streams", "9"], "--streams must be"),
])
def test_the_bench_refuses_before_touching_a_gpu(args, message):
    out = subprocess.run([sys.executable, "bench.py", *args], cwd=ROOT, capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 2 and message in out.stderr, out.stderr[-2000:]


def test_requests_overlap_on_two_streams_only_up_to_the_size_limit():
    """Workloads whose median request moves at most 512 MiB each way alternate their
    requests over two streams; larger requests run on one."""
    import bench
    from iekv import workloads

    def streams(cfg, tp=1):
        return bench.request_streams(workloads.make(cfg, 0, None, tp=tp))

    assert bench.OVERLAP_MAX_REQUEST_BYTES == 512 << 20
    assert [streams(c) for c in ("cfg1", "cfg2", "cfg3", "cfg4")] == [2, 2, 2, 2]
    assert streams("cfg3", 2) == streams("cfg3", 8) == 2
    assert streams("cfg5") == streams("cfg5", 2) == streams("cfg5", 4) == 1  # 2.5 GiB .. 640 MiB
    assert streams("cfg5", 8) == 2                                           # 320 MiB
