"""The synthetic benchmark workloads (CPU).

The sizes at seed 0 are pinned against figures computed independently of this
package when the benchmark was specified (blocks B, payload P = B x 2L x T, the
largest request, cfg4's skipped prefix references). Destination tables come
from the BlockManager's free list, so they are checked to be distinct ids in
range; a tensor-parallel share keeps the tables and divides the tile.
"""
from __future__ import annotations

import pytest

from iekv import workloads

# name: (tile bytes T, block bytes 2L*T, blocks B, payload P, largest request, skipped refs)
SIZES = {
    "cfg1": (8192, 65536, 1107, 72_548_352, 32, 0),
    "cfg2": (65536, 3 << 20, 94, 295_698_432, 2, 0),
    "cfg3": (32768, 2 << 20, 49534, 103_880_327_168, 508, 0),
    "cfg4": (32768, 2 << 20, 17803, 37_335_597_056, 256, 16384),
    "cfg5": (16384, 5 << 19, 16384, 42_949_672_960, 1024, 0),
}


@pytest.mark.parametrize("name", sorted(SIZES))
def test_workload_sizes_at_seed_0(name):
    w = workloads.make(name)
    tile, block, blocks, payload, largest, skipped = SIZES[name]
    assert (w.shape.tile_bytes, w.shape.block_bytes, w.num_blocks) == (tile, block, blocks)
    assert w.payload_bytes == payload
    assert max(len(t) for t in w.src_tables) == largest
    assert w.skipped_blocks == skipped


@pytest.mark.parametrize("name", sorted(SIZES))
def test_tables_are_distinct_ids_in_range(name):
    w = workloads.make(name)
    src = [b for t in w.src_tables for b in t]
    dst = [b for t in w.dst_tables for b in t]
    assert [len(t) for t in w.src_tables] == [len(t) for t in w.dst_tables]
    assert len(set(src)) == len(src) and len(set(dst)) == len(dst)
    assert 0 <= min(src) and max(src) < w.src_pool_blocks
    assert 0 <= min(dst) and max(dst) < w.dst_pool_blocks
    assert not set(dst) & set(w.resident_prefix)   # cfg4: the shared prefix never moves


@pytest.mark.parametrize("tp,tile", [(1, 32768), (2, 16384), (4, 8192), (8, 4096)])
def test_a_tensor_parallel_share_moves_the_same_blocks_with_smaller_tiles(tp, tile):
    full = workloads.make("cfg3")
    share = workloads.make("cfg3", tp=tp)
    assert share.shape.tile_bytes == tile
    assert share.shape.kv_heads == 8 // tp
    assert share.src_tables == full.src_tables and share.dst_tables == full.dst_tables
    assert share.payload_bytes * tp == full.payload_bytes
    assert share.name == ("cfg3" if tp == 1 else f"cfg3/tp{tp}")


def test_cfg4_runs_on_the_llama8b_engine_pools():
    """cfg4 is the cfg3 model, so by default its pools have cfg3's size."""
    cfg3, cfg4 = workloads.make("cfg3"), workloads.make("cfg4")
    assert workloads.llama8b_engine_blocks(0) == cfg3.src_pool_blocks == 49598
    assert cfg4.src_pool_blocks == cfg4.dst_pool_blocks == 49598
    assert cfg4.num_blocks == 17803


def test_a_tensor_parallel_degree_must_divide_the_kv_heads():
    with pytest.raises(ValueError, match="does not divide"):
        workloads.make("cfg3", tp=3)
    with pytest.raises(ValueError, match="does not divide"):
        workloads.make("cfg2", tp=4)          # two KV heads
    with pytest.raises(ValueError):
        workloads.make("cfg1", tp=0)


def test_slack_applies_to_cfg3_and_cfg4_only():
    assert workloads.make("cfg3", slack=0).src_pool_blocks == 49534
    dense = workloads.make("cfg4", slack=64)
    assert (dense.src_pool_blocks, dense.dst_pool_blocks) == (17867, 17996)
    with pytest.raises(ValueError, match="fixed pool sizes"):
        workloads.make("cfg5", slack=4)
    with pytest.raises(ValueError, match="unknown workload"):
        workloads.make("cfg9")
