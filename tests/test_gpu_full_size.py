"""The benchmark workloads at their full sizes, checked through size-independent properties (GPU).

For each configuration the whole handoff runs — half the requests through the
direct pool-to-pool kernel, half through pack -> unpack — and then:
* every destination tile equals its source tile (all 2L arrays, all blocks);
* every destination block outside the handoff is untouched, including the
  prefix blocks a prefix-sharing workload (cfg4) keeps resident and must skip;
* the source pool is unchanged (a checksum of per-array checksums).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DTYPE = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16,
         "fp8_e4m3": torch.float8_e4m3fn}


def checksum(arrays):
    """Sum over arrays of (array index + 1) x (sum of the array's bytes as int64)."""
    total = 0
    for i, t in enumerate(arrays):
        total += (i + 1) * int(t.view(torch.uint8).sum(dtype=torch.int64).item())
    return total


@pytest.mark.parametrize("name", ["cfg2", "cfg4", "cfg5", "cfg3", "cfg5/tp8"])
def test_full_size_handoff(gpu, name):
    """cfg5/tp8 is one tensor-parallel rank's share of cfg5: 2 KiB tiles in 160
    arrays, which the kernels move two to a workgroup."""
    from iekv import workloads
    from iekv.engine.copier import HipSlotCopier
    from iekv.engine.pools import allocate_pool

    base, _, tp = name.partition("/tp")
    w = workloads.make(base, tp=int(tp or 1))
    s = w.shape
    print(f"{name}: {w.num_requests} requests, {w.num_blocks} blocks, "
          f"{w.payload_bytes / 1e9:.1f} GB", flush=True)
    sk, sv = allocate_pool(w.src_pool_blocks, s.block_size, s.layers, s.kv_heads, s.head_dim,
                           dtype=DTYPE[s.dtype], device=gpu, zero=False)
    slab = sk[0]._base
    slab.view(torch.uint8).random_(0, 256, generator=torch.Generator(device=gpu).manual_seed(5))
    dk, dv = allocate_pool(w.dst_pool_blocks, s.block_size, s.layers, s.kv_heads, s.head_dim,
                           dtype=DTYPE[s.dtype], device=gpu, zero=True)
    src, dst = HipSlotCopier(sk, sv, s.block_size), HipSlotCopier(dk, dv, s.block_size)
    before = checksum(sk + sv)

    half = w.num_requests // 2
    for src_ids, dst_ids in zip(w.src_tables[:half], w.dst_tables[:half]):
        dst.copy_blocks(src, src_ids, dst_ids)
    for src_ids, dst_ids in zip(w.src_tables[half:], w.dst_tables[half:]):
        dst.write_blocks(dst_ids, src.read_blocks(src_ids))
    torch.cuda.synchronize()

    moved_src = torch.tensor(sum(w.src_tables, []), dtype=torch.long, device=gpu)
    moved_dst = torch.tensor(sum(w.dst_tables, []), dtype=torch.long, device=gpu)
    untouched = np.setdiff1d(np.arange(w.dst_pool_blocks), moved_dst.cpu().numpy())
    untouched_t = torch.from_numpy(untouched).to(gpu)
    if name == "cfg4":
        assert set(w.resident_prefix) <= set(untouched.tolist())
    T = s.tile_bytes
    for a, (s_arr, d_arr) in enumerate(zip(sk + sv, dk + dv)):
        s_tiles = s_arr.view(torch.uint8).view(-1, T)
        d_tiles = d_arr.view(torch.uint8).view(-1, T)
        for lo in range(0, moved_src.numel(), 8192):
            got = d_tiles.index_select(0, moved_dst[lo:lo + 8192])
            want = s_tiles.index_select(0, moved_src[lo:lo + 8192])
            assert torch.equal(got, want), f"{name}: array {a} differs near entry {lo}"
        if untouched.size:
            assert not d_tiles.index_select(0, untouched_t).any(), f"{name}: array {a} stray write"
    assert checksum(sk + sv) == before
    assert src.blocks_read == w.num_blocks and dst.blocks_written == w.num_blocks
    del sk, sv, dk, dv, slab, src, dst
    torch.cuda.empty_cache()


def test_full_size_host_round_trip_cfg4(gpu):
    """cfg4's round trip of the moved blocks through pinned host DRAM at workload size.

    All 17,803 unique blocks (37.3 GB) go to one pinned buffer with ONE
    iekv_offload and come back onto the decode worker's ids with ONE
    iekv_restore (the reference offloads one block per eviction,
    ie/core/block_manager.py:80-83, and restores one per tier hit, :159-167).
    Then every destination tile equals its source tile, the resident prefix and
    every other untouched destination block are still zero, the source pool is
    unchanged, and sampled host images equal their source tiles (so the host
    image itself, not only the round trip, is block-major in table order).
    """
    from iekv import _native, workloads
    from iekv.engine.copier import HOST_STAGING_BYTES
    from iekv.engine.pools import KVPool, allocate_pool

    w = workloads.make("cfg4")
    s = w.shape
    B, T = w.num_blocks, s.tile_bytes
    print(f"cfg4 host round trip: {B} blocks, {w.payload_bytes / 1e9:.1f} GB", flush=True)
    sk, sv = allocate_pool(w.src_pool_blocks, s.block_size, s.layers, s.kv_heads, s.head_dim,
                           dtype=DTYPE[s.dtype], device=gpu, zero=False)
    sk[0]._base.view(torch.uint8).random_(0, 256,
                                          generator=torch.Generator(device=gpu).manual_seed(6))
    dk, dv = allocate_pool(w.dst_pool_blocks, s.block_size, s.layers, s.kv_heads, s.head_dim,
                           dtype=DTYPE[s.dtype], device=gpu, zero=True)
    src, dst = KVPool(sk, sv, s.block_size), KVPool(dk, dv, s.block_size)
    before = checksum(sk + sv)
    src_ids = sum(w.src_tables, [])
    dst_ids = sum(w.dst_tables, [])
    d_src, d_dst = src.block_ids(src_ids), dst.block_ids(dst_ids, unique=True)
    host = torch.empty((B, s.n_arrays, T), dtype=torch.uint8, pin_memory=True)
    staging = torch.empty(2 * HOST_STAGING_BYTES, dtype=torch.uint8, device=gpu)
    stream, side = torch.cuda.current_stream(), torch.cuda.Stream()
    _native.call("iekv_offload", src.native.handle, d_src.data_ptr(), B, host.data_ptr(),
                 host.numel(), staging.data_ptr(), staging.numel(), stream.cuda_stream,
                 side.cuda_stream)
    _native.call("iekv_restore", dst.native.handle, d_dst.data_ptr(), B, host.data_ptr(),
                 host.numel(), staging.data_ptr(), staging.numel(), stream.cuda_stream,
                 side.cuda_stream)
    torch.cuda.synchronize()
    print("round trip done; checking every tile", flush=True)

    moved_src = d_src.long()
    moved_dst = d_dst.long()
    untouched = np.setdiff1d(np.arange(w.dst_pool_blocks), np.asarray(dst_ids))
    assert set(w.resident_prefix) <= set(untouched.tolist())
    untouched_t = torch.from_numpy(untouched).to(gpu)
    rng = np.random.default_rng(7)
    sample = np.unique(np.concatenate([[0, B - 1], rng.integers(0, B, 62)]))
    sample_t = torch.from_numpy(sample).to(gpu)
    host_sample = host[torch.from_numpy(sample)].to(gpu)          # [k, 2L, T]
    for a, (s_arr, d_arr) in enumerate(zip(sk + sv, dk + dv)):
        s_tiles = s_arr.view(torch.uint8).view(-1, T)
        d_tiles = d_arr.view(torch.uint8).view(-1, T)
        for lo in range(0, B, 8192):
            got = d_tiles.index_select(0, moved_dst[lo:lo + 8192])
            want = s_tiles.index_select(0, moved_src[lo:lo + 8192])
            assert torch.equal(got, want), f"array {a} differs near entry {lo}"
        assert not d_tiles.index_select(0, untouched_t).any(), f"array {a} stray write"
        want = s_tiles.index_select(0, moved_src.index_select(0, sample_t))
        assert torch.equal(host_sample[:, a], want), f"host image of array {a} differs"
    assert checksum(sk + sv) == before
    del host, host_sample, staging, sk, sv, dk, dv, src, dst
    torch.cuda.empty_cache()
    torch._C._host_emptyCache()      # give the pinned pages back before the next test
