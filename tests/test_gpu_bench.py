"""bench.py end to end on the small workload (GPU): the JSON line's fields and every leg verified.

Each case runs bench.py in a child process on cfg1 (72.5 MB payload) with a
short timed pass, then reads its one JSON line. The second case measures one
rank's share at tp=4 (2 KiB tiles, moved two to a workgroup).
"""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
LEGS = ["direct", "pack_unpack", "pack", "unpack", "batched", "copier", "copier_pack_unpack",
        "requests",
        "write_kv", "write_kv_per_layer", "gather_context", "gather_per_array",
        "host_roundtrip"]


def run_bench(*args):
    cmd = [sys.executable, "bench.py", "--config", "cfg1", "--steps", "2", "--warmup", "1",
           "--cpu-blocks", "64", "--cpu-seconds", "0.2", *args]
    print("running", " ".join(cmd[1:]), flush=True)
    out = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=240)
    assert out.returncode == 0, out.stderr[-3000:]
    return json.loads(out.stdout.strip().splitlines()[-1])


@pytest.mark.parametrize("tp", [1, 4])
def test_the_bench_line_keeps_its_contract(gpu, tp):
    line = run_bench("--legs", ",".join(LEGS), "--tp", str(tp))
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["steps"] == 2 and line["warmup"] == 1
    assert line["unit"] == "GB/s" and line["higher_is_better"] is True
    assert line["config"]["tp_share"] == tp
    assert line["config"]["tile_bytes"] == 8192 // tp
    assert set(line["verified"]) == set(LEGS) and all(line["verified"].values())
    # the value is the first handoff leg's 2P / step time
    assert line["config"]["leg"] == "direct"
    assert line["value"] == line["legs"]["direct"]["GBps"] > 0
    roof = line["roofline"]
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    assert roof["algorithmic_bytes_per_launch"] > 0
    # HBM traffic comes only from the committed PMC summary, which measured cfg3
    assert roof["traffic"] is None and "not measured" in roof["traffic_source"]
    assert line["dtype"] == "f32"
    cpu = line["cpu_baseline"]
    assert cpu["kind"] == "port" and cpu["cores"] == 1 and cpu["value"] > 0 and cpu["checked"]
    # one launch per request for write_kv and gather_context (every layer / array at once);
    # per request and layer, and per request and array, for their reference-granularity legs
    legs = line["legs"]
    assert legs["write_kv"]["launches_per_step"] == 64
    assert legs["write_kv_per_layer"]["launches_per_step"] == 64 * 4
    assert legs["gather_context"]["launches_per_step"] == 64
    assert legs["gather_per_array"]["launches_per_step"] == 64 * 8
    assert legs["batched"]["launches_per_step"] == 1
    assert legs["requests"]["launches_per_step"] == legs["direct"]["launches_per_step"] == 64
    # the host's time to issue a step: positive, and within the timed pass's wall time
    # (wall_s is rounded to milliseconds)
    for name, leg in legs.items():
        if "ms_per_step" in leg:
            assert 0 < leg["host_issue_ms_per_step"] <= 1000 * leg["wall_s"] + 1.0, name
    # the host tier's round trip: the whole block list each way, one call per block,
    # and the drop-in tier path (deferred evictions flushed 64 at a time, scattered
    # restores); the leg's verification covers the blocks the tier path restored
    host = legs["host_roundtrip"]
    assert host["d2h_GBps"] > 0 and host["h2d_GBps"] > 0
    assert host["one_call_per_block"]["blocks"] == min(1024, line["config"]["blocks"])
    tier = host["through_the_tier"]
    assert tier["blocks"] == host["one_call_per_block"]["blocks"]
    assert tier["evictions_per_flush"] == 64 and tier["d2h_GBps"] > 0 and tier["h2d_GBps"] > 0


@pytest.mark.parametrize("spec", ["pack_order=0,4", "direct_chunk=4096,8192", "streams=1,2"])
def test_in_process_ab_checks_every_leg(gpu, spec):
    """--ab prints one JSON line: one row per (round, value), every leg checked right
    after its run (unpack after direct included)."""
    line = run_bench("--ab", spec, "--rounds", "2", "--legs", "direct,unpack,pack,pack_unpack")
    key, _, raw = spec.partition("=")
    values = raw.split(",")
    assert line["ab"] == key and line["values"] == values and line["verified"] is True
    assert len(line["rows"]) == 2 * len(values)
    assert all("failed" not in row for row in line["rows"])
    assert set(line["mean"]) == set(values)
    for row in line["rows"]:
        assert all(row[leg] > 0 for leg in ("direct", "unpack", "pack", "pack_unpack"))


def test_the_bench_verifier_notices_one_wrong_byte(gpu):
    """Every figure the bench reports is followed by its tile check, so that check
    must notice the smallest error: after a correct direct handoff of the small
    workload, one flipped bit in the last byte of the last destination tile makes
    verify() fail, and flipping it back passes again; the same for one byte of the
    last packed staging image and verify_pack()."""
    import torch

    import bench
    from iekv import workloads

    w = workloads.make("cfg1", 0, None)
    legs = bench.Legs(w, gpu, 0, "paired", streams=1)
    T = w.shape.tile_bytes
    legs.direct()
    torch.cuda.synchronize()
    assert legs.verify()
    tiles = legs.dst_v[-1].view(torch.uint8).view(-1, T)
    last = int(legs.dst_all[-1])
    tiles[last, T - 1] ^= 1
    assert not legs.verify()
    tiles[last, T - 1] ^= 1
    assert legs.verify()
    legs.pack()
    torch.cuda.synchronize()
    assert legs.verify_pack()
    n = legs.src_ids[-1].numel()
    image = legs.stagings[0][:n * w.shape.block_bytes]
    image[-1] ^= 1
    assert not legs.verify_pack()
    image[-1] ^= 1
    assert legs.verify_pack()
