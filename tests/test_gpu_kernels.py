"""HIP handoff kernels vs the NumPy oracle, byte for byte (GPU).

Every pool is filled with random BYTES (all bit patterns, NaN codes included),
and every comparison is on bytes: the handoff must be a bitwise copy of the
reference's NumPy slice copies for any KV dtype.
"""
from __future__ import annotations

import ctypes
import hashlib

import numpy as np
import pytest
import torch

from conftest import golden
from helpers import cfg1_inputs
from oracle.copier import LayeredSlotCopier, handoff, pack, packed_image

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16, torch.float8_e4m3fn, torch.int8,
          torch.uint8]


def allocate(num_blocks, bs, layers, heads, dim, dtype, device, seed):
    from iekv.engine.pools import allocate_pool

    k, v = allocate_pool(num_blocks, bs, layers, heads, dim, dtype=dtype, device=device,
                         zero=False)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    slab = k[0]._base if k[0]._base is not None else k[0]
    raw = slab.view(torch.uint8)
    raw.copy_(torch.randint(0, 256, raw.shape, dtype=torch.uint8, device=device, generator=gen))
    return k, v


def host_bytes(arrays):
    """Per-array uint8 copies [rows, bytes_per_row] on the host."""
    out = []
    for t in arrays:
        rows = t.shape[0]
        out.append(t.contiguous().view(torch.uint8).reshape(rows, -1).cpu().numpy().copy())
    return out


def oracle_of(k, v, bs):
    return LayeredSlotCopier(host_bytes(k), host_bytes(v), bs)


def assert_pool_equals(k, v, oracle):
    got = host_bytes(k) + host_bytes(v)
    want = list(oracle.k_caches) + list(oracle.v_caches)
    for a, (g, w) in enumerate(zip(got, want)):
        if not np.array_equal(g, w):
            rows = np.nonzero((g != w).any(axis=1))[0]
            raise AssertionError(f"array {a}: {rows.size} rows differ, first at row {rows[0]}")


def random_tables(rng, n_src, n_dst, count):
    src = [int(b) for b in rng.permutation(n_src)[:count]]
    dst = [int(b) for b in rng.permutation(n_dst)[:count]]
    return src, dst


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_direct_copy_matches_the_oracle(gpu, dtype):
    from iekv.engine.copier import HipSlotCopier

    bs, layers, heads, dim = 16, 3, 2, 16
    sk, sv = allocate(64, bs, layers, heads, dim, dtype, gpu, seed=1)
    dk, dv = allocate(80, bs, layers, heads, dim, dtype, gpu, seed=2)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(3)
    src_ids, dst_ids = random_tables(rng, 64, 80, 37)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    dst.copy_blocks(src, src_ids, dst_ids)
    torch.cuda.synchronize()
    handoff(src_o, dst_o, [src_ids], [dst_ids])
    assert_pool_equals(dk, dv, dst_o)
    assert_pool_equals(sk, sv, src_o)  # the source is untouched
    assert src.blocks_read == 37 and dst.blocks_written == 37
    # The consumers' [N, bs, H, D] view (ie/kernels/flash_backend.py:15-17) sees
    # each moved block at its new id.
    from iekv.engine.pools import paged_view

    for s_arr, d_arr in zip(sk + sv, dk + dv):
        got = paged_view(d_arr, bs).view(torch.uint8)[torch.tensor(dst_ids, device=gpu)]
        want = paged_view(s_arr, bs).view(torch.uint8)[torch.tensor(src_ids, device=gpu)]
        assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_pack_then_unpack_matches_the_oracle(gpu, dtype):
    from iekv.engine.copier import HipSlotCopier

    bs, layers, heads, dim = 16, 4, 2, 32
    sk, sv = allocate(50, bs, layers, heads, dim, dtype, gpu, seed=4)
    dk, dv = allocate(70, bs, layers, heads, dim, dtype, gpu, seed=5)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(6)
    src_ids, dst_ids = random_tables(rng, 50, 70, 29)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    packed = src.read_blocks(src_ids)
    dst.write_blocks(dst_ids, packed)
    torch.cuda.synchronize()
    payloads = pack(src_o, src_ids)
    assert np.array_equal(packed.data.cpu().numpy(), packed_image(payloads))
    for d, p in zip(dst_ids, payloads):
        dst_o.write_block(d, p)
    assert_pool_equals(dk, dv, dst_o)
    assert src.bytes_moved == src_o.bytes_moved
    assert dst.bytes_moved == dst_o.bytes_moved


@pytest.mark.parametrize("bs,heads,dim,dtype", [
    (1, 1, 1, torch.uint8),      # 1-byte tiles
    (3, 1, 5, torch.float16),    # 30-byte tiles (2-byte vectors)
    (1, 1, 1, torch.float32),    # 4-byte tiles
    (1, 1, 2, torch.float32),    # 8-byte tiles
    (5, 3, 3, torch.uint8),      # 45-byte tiles
    (2, 1, 24, torch.float32),   # 192 bytes: 16-byte vectors, odd array stride
])
def test_narrow_and_odd_tiles(gpu, bs, heads, dim, dtype):
    from iekv.engine.copier import HipSlotCopier

    layers = 2
    sk, sv = allocate(33, bs, layers, heads, dim, dtype, gpu, seed=7)
    dk, dv = allocate(41, bs, layers, heads, dim, dtype, gpu, seed=8)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(9)
    src_ids, dst_ids = random_tables(rng, 33, 41, 19)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    dst.write_blocks(dst_ids[:9], src.read_blocks(src_ids[:9]))
    dst.copy_blocks(src, src_ids[9:], dst_ids[9:])
    torch.cuda.synchronize()
    handoff(src_o, dst_o, [src_ids], [dst_ids])
    assert_pool_equals(dk, dv, dst_o)


RANDOM_CASES = 48


@pytest.mark.parametrize("case", range(RANDOM_CASES))
def test_random_tiles_and_launch_shapes_match_the_oracle(gpu, case):
    """Seeded random tile shapes (1 B to 96 KiB, every vector width, tiles that
    split into uneven chunk counts), random tables and a random launch shape
    (run, unroll, order, chunk, non-temporal); pack -> unpack for half the
    request and the direct copy for the rest, byte for byte against the oracle."""
    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    rng = np.random.default_rng(1000 + case)
    dtype = [torch.uint8, torch.float16, torch.bfloat16, torch.float32][rng.integers(4)]
    elem = torch.tensor([], dtype=dtype).element_size()
    while True:
        bs = int(rng.choice([1, 2, 3, 4, 8, 16, 32]))
        heads = int(rng.integers(1, 9))
        dim = int(rng.choice([1, 3, 8, 16, 24, 64, 96, 128]))
        if bs * heads * dim * elem <= 96 << 10:
            break
    layers = int(rng.integers(1, 4))
    n_src, n_dst = int(rng.integers(8, 48)), int(rng.integers(8, 48))
    count = int(rng.integers(2, min(n_src, n_dst) + 1))
    shape = (int(rng.choice([0, 1, 3])), int(rng.choice([1, 2, 4, 8, 16])), int(rng.integers(2)),
             int(rng.choice([0, 1, 2, 3, 4, 5, 6, 7])), int(rng.choice([0, 1, 2, 3, 4, 5, 6, 7])),
             int(rng.choice([0, 64, 256, 1024, 4096, 8192])))
    sk, sv = allocate(n_src, bs, layers, heads, dim, dtype, gpu, seed=2000 + case)
    dk, dv = allocate(n_dst, bs, layers, heads, dim, dtype, gpu, seed=3000 + case)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    src_ids, dst_ids = random_tables(rng, n_src, n_dst, count)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    # odd cases hand the ids over as device tensors, even cases as host lists
    ids_of = (lambda ids: torch.tensor(ids, dtype=torch.int32, device=gpu)) if case % 2 else list
    before = _native.get_launch()
    try:
        _native.set_launch(*shape)
        half = count // 2
        packed = src.read_blocks(ids_of(src_ids[:half]))
        dst.write_blocks(ids_of(dst_ids[:half]), packed)
        dst.copy_blocks(src, ids_of(src_ids[half:]), ids_of(dst_ids[half:]))
        torch.cuda.synchronize()
    finally:
        _native.set_launch(**before)
    label = (case, dtype, bs, heads, dim, layers, count, shape)
    assert np.array_equal(packed.data.cpu().numpy(),
                          packed_image(pack(oracle_of(sk, sv, bs), src_ids[:half]))), label
    handoff(src_o, dst_o, [src_ids], [dst_ids])
    assert_pool_equals(dk, dv, dst_o)


def test_every_launch_shape_is_bit_exact(gpu):
    """Pack, unpack and direct copy under every run / unroll / non-temporal /
    workgroup-order / chunk setting (order for the pool-writing launches,
    pack_order for the staging-writing ones; 3 and 7 the scattered order,
    plain and XCD-grouped; 4-7 are the XCD-grouped orders,
    here on grids of 8 to 19,712 workgroups, most not a multiple of the 8
    XCDs; chunks of 64 B to whole 32 KiB tiles)."""
    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    bs, layers, heads, dim = 16, 2, 8, 128   # 32 KiB tiles, like the Llama-3-8B shape
    sk, sv = allocate(96, bs, layers, heads, dim, torch.bfloat16, gpu, seed=10)
    dk, dv = allocate(90, bs, layers, heads, dim, torch.bfloat16, gpu, seed=12)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    rng = np.random.default_rng(11)
    src_ids = [int(b) for b in rng.permutation(96)[:77]]
    dst_ids = [int(b) for b in rng.permutation(90)[:77]]
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    want = packed_image(pack(src_o, src_ids))
    handoff(src_o, dst_o, [src_ids], [dst_ids])
    before = _native.get_launch()
    try:
        shapes = [(run, unroll, nt, order, chunk)
                  for run in (1, 3, 0, 64) for unroll in (1, 4, 8, 16) for nt in (0, 1)
                  for order in range(8) for chunk in (0, 4096)]
        shapes += [(0, unroll, 1, order, chunk) for unroll in (1, 2, 8) for order in (0, 3, 5)
                   for chunk in (64, 512, 1024, 16384, 32768, 1 << 20)]
        rows = np.concatenate([np.arange(b * bs, (b + 1) * bs) for b in dst_ids])
        dev = lambda ids: torch.tensor(ids, dtype=torch.int32, device=gpu)  # noqa: E731
        for shape in shapes:
            run, unroll, nt, order, chunk = shape
            _native.set_launch(run, unroll, nt, order, order, chunk)
            # device ids take the kernel that honours run_blocks (LDS-staged runs);
            # host lists take the kernel with the ids in its arguments
            for ids_of in (dev, list):
                packed = src.read_blocks(ids_of(src_ids))
                assert np.array_equal(packed.data.cpu().numpy(), want), (shape, ids_of)
                for t in dk + dv:
                    t.zero_()
                half = len(src_ids) // 2
                dst.write_blocks(ids_of(dst_ids[:half]), packed[:half])
                dst.copy_blocks(src, ids_of(src_ids[half:]), ids_of(dst_ids[half:]))
                torch.cuda.synchronize()
                got = host_bytes(dk) + host_bytes(dv)
                for g, w in zip(got, list(dst_o.k_caches) + list(dst_o.v_caches)):
                    assert np.array_equal(g[rows], w[rows]), (shape, ids_of)
    finally:
        _native.set_launch(**before)


@pytest.mark.parametrize("bs,heads,dim,dtype,layers", [
    (16, 1, 128, torch.uint8, 40),     # 2 KiB tiles, 80 arrays (the 70B share at tp=8)
    (16, 1, 64, torch.bfloat16, 5),    # 2 KiB tiles, 10 arrays
    (4, 1, 32, torch.float32, 3),      # 512 B tiles, 6 arrays: groups larger than the arrays
    (1, 1, 8, torch.float16, 7),       # 16 B tiles, 14 arrays
    (16, 1, 128, torch.bfloat16, 3),   # 4 KiB tiles: grouped only under larger chunks
    (2, 3, 8, torch.float32, 4),       # 192 B tiles: 12 vectors do not divide 256 lanes
    (3, 1, 5, torch.float16, 6),       # 30 B tiles (2-byte vectors)
])
def test_tiles_smaller_than_a_chunk_are_grouped_bit_exact(gpu, bs, heads, dim, dtype, layers):
    """A tile smaller than the chunk size is moved together with the same
    block's tiles in the next arrays by one workgroup (partial last groups
    included). Pack, unpack and direct copy, device and kernel-argument ids,
    under chunks that give 1 to 128 tiles per workgroup, against the oracle."""
    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    sk, sv = allocate(60, bs, layers, heads, dim, dtype, gpu, seed=50)
    dk, dv = allocate(50, bs, layers, heads, dim, dtype, gpu, seed=51)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    rng = np.random.default_rng(52)
    src_ids, dst_ids = random_tables(rng, 60, 50, 37)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    want = packed_image(pack(src_o, src_ids))
    handoff(src_o, dst_o, [src_ids], [dst_ids])
    source = host_bytes(sk) + host_bytes(sv)
    rows = np.concatenate([np.arange(b * bs, (b + 1) * bs) for b in dst_ids])
    dev = lambda ids: torch.tensor(ids, dtype=torch.int32, device=gpu)  # noqa: E731
    before = _native.get_launch()
    try:
        for chunk in (0, 1024, 4096, 8192, 65536):
            for unroll in (1, 4, 16):
                _native.set_launch(0, unroll, 1, -1, -1, chunk)
                for ids_of in (dev, list):
                    label = (chunk, unroll, ids_of)
                    packed = src.read_blocks(ids_of(src_ids))
                    assert np.array_equal(packed.data.cpu().numpy(), want), label
                    for t in dk + dv:
                        t.zero_()
                    dst.write_blocks(ids_of(dst_ids[:20]), packed[:20])
                    dst.copy_blocks(src, ids_of(src_ids[20:]), ids_of(dst_ids[20:]))
                    torch.cuda.synchronize()
                    got = host_bytes(dk) + host_bytes(dv)
                    for g, w in zip(got, list(dst_o.k_caches) + list(dst_o.v_caches)):
                        assert np.array_equal(g[rows], w[rows]), label
    finally:
        _native.set_launch(**before)
    assert all(np.array_equal(a, b) for a, b in zip(source, host_bytes(sk) + host_bytes(sv)))


@pytest.mark.parametrize("count", [1, 64, 66, 128, 130, 255, 256, 257, 600, 1300])
def test_host_ids_in_the_kernel_arguments_and_beyond(gpu, count):
    """Host id lists ride in the launches' kernel arguments (iekv_*_ids), 256 per
    launch: lists of 1 to 256 blocks in one launch, 257 and 300 in two; a longer
    one (650 of a 1300-block request) is uploaded and moved in one launch. A
    launch whose ids fill at most 64 words takes the kernels with the small id
    block: the first half of the request is packed and unpacked (one word per
    id: 32 and 33 ids small, 64 small, 65 large), the second half copied
    directly (two words per id: 32 small, 33, 64 and 65 large). All give the
    oracle's bytes."""
    from iekv.engine.copier import HipSlotCopier

    bs, layers, heads, dim = 4, 2, 2, 32
    sk, sv = allocate(1400, bs, layers, heads, dim, torch.bfloat16, gpu, seed=41)
    dk, dv = allocate(1350, bs, layers, heads, dim, torch.bfloat16, gpu, seed=42)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(43)
    src_ids, dst_ids = random_tables(rng, 1400, 1350, count)
    half = count // 2
    packed = src.read_blocks(src_ids[:half])
    dst.write_blocks(dst_ids[:half], packed)
    dst.copy_blocks(src, src_ids[half:], dst_ids[half:])
    torch.cuda.synchronize()
    handoff(src_o, dst_o, [src_ids], [dst_ids])
    assert_pool_equals(dk, dv, dst_o)
    assert len(packed) == half
    if half:
        assert np.array_equal(packed.data.cpu().numpy(),
                              packed_image(pack(oracle_of(sk, sv, bs), src_ids[:half])))


def test_a_split_that_would_overflow_the_dispatch_is_halved(gpu):
    """70,000 blocks x 4 arrays in 64-byte chunks of 4 KiB tiles would need
    17.9M workgroups (over the 2^32 - 1 work-item limit of one dispatch): the
    library halves the split to 32 chunks and moves every byte in one launch."""
    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    bs, layers, heads, dim = 16, 2, 2, 64   # 4 KiB uint8 tiles
    n = 70_000
    sk, sv = allocate(n + 16, bs, layers, heads, dim, torch.uint8, gpu, seed=21)
    dk, dv = allocate(n + 16, bs, layers, heads, dim, torch.uint8, gpu, seed=22)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    rng = np.random.default_rng(23)
    src_ids = rng.permutation(n + 16)[:n]
    dst_ids = rng.permutation(n + 16)[:n]
    before = _native.get_launch()
    try:
        _native.set_launch(0, 1, 1, 5, 0, 64)
        with _native.LaunchTimer(8) as timer:
            dst.copy_blocks(src, src_ids, dst_ids)
        assert len(timer.durations_ms) == 1
    finally:
        _native.set_launch(**before)
    torch.cuda.synchronize()
    s_ids = torch.as_tensor(src_ids, device=gpu)
    d_ids = torch.as_tensor(dst_ids, device=gpu)
    for s_arr, d_arr in zip(sk + sv, dk + dv):
        want = s_arr.view(-1, bs * heads * dim)
        got = d_arr.view(-1, bs * heads * dim)
        assert torch.equal(got[d_ids], want[s_ids])


@pytest.mark.parametrize("chunk,launches", [(0, 4), (4096, 2)])
def test_a_move_beyond_one_dispatch_spreads_over_launches(gpu, chunk, launches):
    """9M 16-byte tiles x 2 arrays with one tile per workgroup (chunk 0) exceed
    one dispatch (16,777,215 workgroups of 256 lanes): the library issues two
    launches per move over consecutive entry ranges, and pack keeps the staging
    layout. Under 4 KiB chunks one workgroup takes a block's tiles in both
    arrays, so each move fits one launch."""
    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    bs, layers, heads, dim = 1, 1, 1, 16    # 16-byte uint8 tiles
    n = 9_000_000
    sk, sv = allocate(n, bs, layers, heads, dim, torch.uint8, gpu, seed=31)
    dk, dv = allocate(n, bs, layers, heads, dim, torch.uint8, gpu, seed=32)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(33)
    src_ids = torch.randperm(n, device=gpu, generator=gen).to(torch.int32)
    dst_ids = torch.randperm(n, device=gpu, generator=gen).to(torch.int32)
    before = _native.get_launch()
    try:
        _native.set_launch(0, 0, -1, -1, -1, chunk)
        with _native.LaunchTimer(8) as timer:
            dst.copy_blocks(src, src_ids, dst_ids)
            packed = src.read_blocks(src_ids)
        assert len(timer.durations_ms) == launches
    finally:
        _native.set_launch(**before)
    torch.cuda.synchronize()
    s_ids, d_ids = src_ids.long(), dst_ids.long()
    for a, (s_arr, d_arr) in enumerate(zip(sk + sv, dk + dv)):
        want = s_arr.view(n, 16)[s_ids]
        assert torch.equal(d_arr.view(n, 16)[d_ids], want)
        assert torch.equal(packed.data[:, a], want)


@pytest.mark.parametrize("chunk", [-1, 0], ids=["grouped tiles", "whole tiles"])
def test_block_ids_at_the_top_of_the_int32_range(gpu, chunk):
    """A pool of INT32_MAX blocks, the largest iekv_pool_create takes (16-byte tiles,
    one layer's K and V: 64 GiB): ids next to the int32 limit address the last tiles
    of both arrays, 32 GiB into each, so every move path must form 64-bit offsets from
    32-bit ids. The direct copy with device ids and with host ids and pack -> unpack
    each move their tiles, under the default launch shape (a block's two tiles in one
    workgroup) and with whole tiles per workgroup; the neighbours of every destination
    tile keep their bytes."""
    from array import array

    from iekv import _native

    n, T, A = 2**31 - 1, 16, 2
    top = n - 1
    slab = torch.empty(A * n * T, dtype=torch.uint8, device=gpu)
    tiles = slab.view(A, n, T)
    pool = _native.Pool([slab.data_ptr(), slab.data_ptr() + n * T], T, n, gpu.index or 0)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(61)
    cases = {   # (sources, destinations), all within one pool and disjoint
        "device ids": ([top, top - 2, 3, top - 7], [top - 1, 0, top - 3, top - 5]),
        "host ids": ([top - 11, 9, top - 13], [top - 12, top - 4, 17]),
        "pack/unpack": ([top - 21, 25, top - 23], [top - 22, top - 6, 27]),
    }
    touched = sorted({b for src, dst in cases.values() for b in src + dst}
                     | {b + d for _, dst in cases.values() for b in dst for d in (-1, 1)
                        if 0 <= b + d < n})
    idx = torch.tensor(touched, dtype=torch.long, device=gpu)
    for a in range(A):
        tiles[a].index_copy_(0, idx, torch.randint(0, 256, (len(touched), T), dtype=torch.uint8,
                                                   device=gpu, generator=gen))
    before_tiles = tiles[:, idx].clone()
    stream = torch.cuda.current_stream().cuda_stream
    settings = _native.get_launch()
    print(f"int32-limit pool, chunk {chunk}", flush=True)
    try:
        if chunk >= 0:
            _native.set_launch(0, 0, -1, -1, -1, chunk)
        src, dst = cases["device ids"]
        s_dev = torch.tensor(src, dtype=torch.int32, device=gpu)
        d_dev = torch.tensor(dst, dtype=torch.int32, device=gpu)
        _native.call("iekv_copy_direct", pool.handle, pool.handle, s_dev.data_ptr(),
                     d_dev.data_ptr(), len(src), stream)
        src, dst = cases["host ids"]
        hs, hd = array("i", src), array("i", dst)
        _native.call("iekv_copy_direct_ids", pool.handle, pool.handle, hs.buffer_info()[0],
                     hd.buffer_info()[0], len(src), stream)
        src, dst = cases["pack/unpack"]
        staging = torch.empty(len(src) * A * T, dtype=torch.uint8, device=gpu)
        hs, hd = array("i", src), array("i", dst)
        _native.call("iekv_pack_ids", pool.handle, hs.buffer_info()[0], len(src),
                     staging.data_ptr(), staging.numel(), stream)
        _native.call("iekv_unpack_ids", pool.handle, hd.buffer_info()[0], len(dst),
                     staging.data_ptr(), staging.numel(), stream)
        torch.cuda.synchronize()
    finally:
        _native.set_launch(**settings)
    # Expected: every tile as it was, then each case's destinations from their sources.
    want = {b: before_tiles[:, i] for i, b in enumerate(touched)}
    for src, dst in cases.values():
        moved = {d: want[s] for s, d in zip(src, dst)}
        want.update(moved)
    got = tiles[:, idx]
    for i, b in enumerate(touched):
        assert torch.equal(got[:, i], want[b]), f"block {b} (top - {top - b})"
    assert torch.equal(staging.view(len(cases["pack/unpack"][0]), A, T),
                       before_tiles[:, [touched.index(s) for s in cases["pack/unpack"][0]]]
                       .transpose(0, 1))
    pool.close()
    del slab, tiles, staging
    torch.cuda.empty_cache()


@pytest.mark.parametrize("layout", ["descending", "irregular"])
def test_separately_allocated_layers_use_an_address_table(gpu, layout):
    """Per-layer caches that do not sit at equal steps in memory make the pool keep
    their base addresses in a device table that every kernel reads. The arrays here
    are views of one buffer at descending or irregular positions (tensors allocated
    one after another can land at equal steps by chance, and the library then keeps
    only a base and a stride). Direct copy, pack -> unpack and a round trip through
    pinned host memory between two such pools move the oracle's bytes."""
    from iekv.engine.copier import HipSlotCopier

    bs, heads, dim, n, L = 16, 2, 16, 40, 3
    order = {"descending": ([5, 4, 3, 2, 1, 0], [10, 8, 6, 4, 2, 0]),
             "irregular": ([0, 3, 1, 7, 4, 9], [8, 2, 5, 0, 11, 6])}[layout]

    def arrays(positions, seed):
        gen = torch.Generator(device=gpu).manual_seed(seed)
        buf = torch.randint(-128, 127, (max(positions) + 1, n * bs, heads, dim),
                            dtype=torch.int8, device=gpu, generator=gen)
        views = [buf[i] for i in positions]
        ptrs = [t.data_ptr() for t in views]
        steps = {b - a for a, b in zip(ptrs, ptrs[1:])}
        assert len(steps) > 1 or ptrs[1] < ptrs[0]      # the library's table rule
        return views[:L], views[L:]

    k, v = arrays(order[0], 47)
    dk, dv = arrays(order[1], 48)
    src = HipSlotCopier(k, v, bs, payload_location="host", defer_reads=False)
    dst = HipSlotCopier(dk, dv, bs)
    src_o, dst_o = oracle_of(k, v, bs), oracle_of(dk, dv, bs)
    src_ids, dst_ids = [5, 0, 39, 17], [1, 38, 2, 20]
    dst.copy_blocks(src, src_ids, dst_ids)
    packed = src.read_blocks([6, 9, 33], location="device")
    dst.write_blocks([10, 11, 12], packed)
    host = src.read_blocks([21, 3], location="host")
    dst.write_blocks([30, 31], host)
    torch.cuda.synchronize()
    handoff(src_o, dst_o, [src_ids, [6, 9, 33], [21, 3]], [dst_ids, [10, 11, 12], [30, 31]])
    assert_pool_equals(dk, dv, dst_o)
    assert np.array_equal(host.host_data().numpy(), packed_image(pack(src_o, [21, 3])))


def test_empty_requests_move_nothing(gpu):
    from iekv.engine.copier import HipSlotCopier

    sk, sv = allocate(8, 16, 2, 2, 16, torch.float16, gpu, seed=12)
    dk, dv = allocate(8, 16, 2, 2, 16, torch.float16, gpu, seed=13)
    before = host_bytes(dk) + host_bytes(dv)
    src, dst = HipSlotCopier(sk, sv, 16), HipSlotCopier(dk, dv, 16)
    packed = src.read_blocks([])
    assert len(packed) == 0
    dst.write_blocks([], packed)
    dst.copy_blocks(src, [], [])
    torch.cuda.synchronize()
    assert all(np.array_equal(a, b) for a, b in zip(before, host_bytes(dk) + host_bytes(dv)))


def test_bad_ids_raise_before_any_launch(gpu):
    from iekv.engine.copier import HipSlotCopier

    sk, sv = allocate(8, 16, 2, 2, 16, torch.float16, gpu, seed=14)
    src = HipSlotCopier(sk, sv, 16)
    dk, dv = allocate(8, 16, 2, 2, 16, torch.float16, gpu, seed=15)
    dst = HipSlotCopier(dk, dv, 16)
    before = host_bytes(dk)
    with pytest.raises(IndexError):
        src.read_blocks([0, 8])
    with pytest.raises(IndexError):
        dst.copy_blocks(src, [0], [-1])
    with pytest.raises(ValueError, match="distinct"):
        dst.copy_blocks(src, [0, 1], [3, 3])
    with pytest.raises(ValueError, match="disjoint"):
        src.copy_blocks(src, [0, 1], [1, 2])
    with pytest.raises(ValueError):
        dst.write_blocks([0, 1], src.read_blocks([2]))
    with pytest.raises(TypeError):
        dst.copy_blocks(src, [0.0], [1])                   # not truncated to block 0
    with pytest.raises(TypeError):
        dst.write_blocks(np.array([1.5]), src.read_blocks([2]))
    # A payload accepted by one copier is still checked by a copier of another layout.
    ok = src.read_blocks([3])
    dst.write_blocks([4], ok)
    ek, ev = allocate(8, 16, 2, 4, 16, torch.float16, gpu, seed=16)   # twice the tile
    other = HipSlotCopier(ek, ev, 16)
    with pytest.raises(ValueError, match="does not fit"):
        other.write_blocks([0], ok)
    torch.cuda.synchronize()
    after = host_bytes(dk)
    src_o = oracle_of(sk, sv, bs=16)
    for a, (b, g) in enumerate(zip(before, after)):
        want = b.copy()
        want[4 * 16:5 * 16] = (src_o.k_caches + src_o.v_caches)[a][3 * 16:4 * 16]
        assert np.array_equal(g, want)


def test_device_ids_outside_the_pool_are_skipped_by_the_kernel(gpu):
    from iekv.engine.copier import HipSlotCopier

    sk, sv = allocate(8, 16, 2, 2, 16, torch.float32, gpu, seed=16)
    dk, dv = allocate(8, 16, 2, 2, 16, torch.float32, gpu, seed=17)
    src, dst = HipSlotCopier(sk, sv, 16), HipSlotCopier(dk, dv, 16)
    src_o, dst_o = oracle_of(sk, sv, 16), oracle_of(dk, dv, 16)
    src_ids = torch.tensor([1, 9, 2], dtype=torch.int32, device=gpu)   # 9 is outside
    dst_ids = torch.tensor([4, 5, 6], dtype=torch.int32, device=gpu)
    dst.copy_blocks(src, src_ids, dst_ids)
    torch.cuda.synchronize()
    handoff(src_o, dst_o, [[1, 2]], [[4, 6]])
    assert_pool_equals(dk, dv, dst_o)


def test_single_block_protocol_and_reference_payload_structure(gpu):
    from iekv.engine.copier import HipSlotCopier

    bs, layers, heads, dim = 4, 3, 2, 8
    sk, sv = allocate(10, bs, layers, heads, dim, torch.float32, gpu, seed=18)
    dk, dv = allocate(10, bs, layers, heads, dim, torch.float32, gpu, seed=19)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    payload = src.read_block(7)
    k_tiles, v_tiles = payload
    assert len(k_tiles) == layers and len(v_tiles) == layers
    for l in range(layers):
        assert k_tiles[l].shape == (bs, heads, dim)
        assert torch.equal(k_tiles[l].view(torch.int32), sk[l][28:32].view(torch.int32))
        assert torch.equal(v_tiles[l].view(torch.int32), sv[l][28:32].view(torch.int32))
    dst.write_block(2, payload)
    # A reference-structured payload of plain tensors (and of NumPy arrays) also writes.
    dst.write_block(5, ([t.clone() for t in k_tiles], [t.clone() for t in v_tiles]))
    dst.write_block(9, ([t.cpu().numpy() for t in k_tiles], [t.cpu().numpy() for t in v_tiles]))
    torch.cuda.synchronize()
    for b in (2, 5, 9):
        for l in range(layers):
            assert torch.equal(dk[l][b * bs:(b + 1) * bs].view(torch.int32),
                               sk[l][28:32].view(torch.int32))
            assert torch.equal(dv[l][b * bs:(b + 1) * bs].view(torch.int32),
                               sv[l][28:32].view(torch.int32))
    assert src.blocks_read == 1 and dst.blocks_written == 3


@pytest.mark.parametrize("pinned", [True, False], ids=["pinned", "pageable"])
@pytest.mark.parametrize("staging_blocks", [1, 2, 5, 64])
def test_host_offload_and_restore_pipelines(gpu, staging_blocks, pinned):
    """Offload then restore through host memory. Pinned host buffers of at most
    64 MiB are written and read by the move kernel itself; pageable ones go
    through the staged pipelines (1 to 23 staging chunks)."""
    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    bs, layers, heads, dim = 16, 2, 4, 32
    sk, sv = allocate(60, bs, layers, heads, dim, torch.bfloat16, gpu, seed=20)
    dk, dv = allocate(60, bs, layers, heads, dim, torch.bfloat16, gpu, seed=21)
    src = HipSlotCopier(sk, sv, bs, payload_location="host")
    dst = HipSlotCopier(dk, dv, bs)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(22)
    src_ids, dst_ids = random_tables(rng, 60, 60, 23)
    block = src.pool.block_bytes
    staging = torch.empty(staging_blocks * block, dtype=torch.uint8, device=gpu)
    host = torch.empty((23, src.pool.n_arrays, src.pool.tile_bytes), dtype=torch.uint8,
                       pin_memory=pinned)
    ids = src.pool.block_ids(src_ids)
    stream = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    _native.call("iekv_offload", src.pool.native.handle, ids.data_ptr(), 23, host.data_ptr(),
                 host.numel(), staging.data_ptr(), staging.numel(), stream.cuda_stream,
                 side.cuda_stream)
    stream.synchronize()
    payloads = pack(src_o, src_ids)
    assert np.array_equal(host.numpy(), packed_image(payloads))
    d_ids = dst.pool.block_ids(dst_ids)
    _native.call("iekv_restore", dst.pool.native.handle, d_ids.data_ptr(), 23, host.data_ptr(),
                 host.numel(), staging.data_ptr(), staging.numel(), stream.cuda_stream,
                 side.cuda_stream)
    torch.cuda.synchronize()
    for d, p in zip(dst_ids, payloads):
        dst_o.write_block(d, p)
    assert_pool_equals(dk, dv, dst_o)


@pytest.mark.parametrize("bs,heads,dim,dtype", [
    (5, 3, 3, torch.uint8),        # 45-byte tiles: byte vectors, grouped per workgroup
    (2, 1, 24, torch.float32),     # 192-byte tiles
    (16, 2, 64, torch.float16),    # 4 KiB tiles: one staging chunk
    (64, 4, 64, torch.bfloat16),   # 32 KiB tiles: several chunks, whole tiles on reads
    (256, 2, 64, torch.float16)])  # 64 KiB tiles
def test_direct_host_transfers_of_every_tile_shape(gpu, bs, heads, dim, dtype):
    """Pinned images restored directly by the unpack kernel (which reads whole tiles,
    or groups of tiles smaller than the staging chunk) and offloaded directly by the
    pack kernel, one contiguous image and scattered images: bytes equal the oracle's."""
    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    layers = 3
    sk, sv = allocate(40, bs, layers, heads, dim, dtype, gpu, seed=70)
    dk, dv = allocate(40, bs, layers, heads, dim, dtype, gpu, seed=71)
    src = HipSlotCopier(sk, sv, bs, payload_location="host", defer_reads=False)
    dst = HipSlotCopier(dk, dv, bs)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(72)
    src_ids, dst_ids = random_tables(rng, 40, 40, 17)
    assert 17 * src.pool.block_bytes <= _native.HOST_DIRECT_MAX
    whole = src.read_blocks(src_ids)                       # one pinned image, direct
    single = [src.read_block(b) for b in src_ids[:9]]      # one buffer each
    torch.cuda.synchronize()
    payloads = pack(src_o, src_ids)
    assert np.array_equal(whole.host_data().numpy(), packed_image(payloads))
    dst.write_blocks(dst_ids, whole)                       # iekv_restore, direct
    dst.write_blocks(dst_ids[:9][::-1], single[::-1])      # iekv_restore_blocks, direct
    torch.cuda.synchronize()
    for d, p in zip(dst_ids, payloads):
        dst_o.write_block(d, p)
    for d, p in zip(dst_ids[:9][::-1], payloads[:9][::-1]):
        dst_o.write_block(d, p)
    assert_pool_equals(dk, dv, dst_o)


def test_pinned_restores_of_any_size_leave_the_staging_buffer_untouched(gpu):
    """A pinned image is restored by the unpack kernel itself at any size (72 MiB here,
    above IEKV_HOST_DIRECT_MAX_BYTES: two launches), scattered pinned images too (130,
    above IEKV_INLINE_IMAGES): the staging buffer keeps its sentinel bytes. A pageable
    image of the same blocks goes through it. Bytes equal the oracle's each time."""
    from iekv import _native
    from iekv.engine.pools import KVPool

    bs, layers, heads, dim = 16, 4, 8, 128     # 1 MiB block images
    sk, sv = allocate(150, bs, layers, heads, dim, torch.bfloat16, gpu, seed=74)
    dk, dv = allocate(150, bs, layers, heads, dim, torch.bfloat16, gpu, seed=75)
    src, dst = KVPool(sk, sv, bs), KVPool(dk, dv, bs)
    rng = np.random.default_rng(76)
    block = src.block_bytes
    staging = torch.full((4 * block,), 0xA5, dtype=torch.uint8, device=gpu)
    stream, side = torch.cuda.current_stream(), torch.cuda.Stream()
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    for n, memory, layout in ((72, "pinned", "one image"), (130, "pinned", "scattered"),
                              (72, "pageable", "one image")):
        src_ids, dst_ids = random_tables(rng, 150, 150, n)
        image = torch.from_numpy(packed_image(pack(src_o, src_ids)).reshape(-1).copy())
        host = image.pin_memory() if memory == "pinned" else image
        ids = dst.block_ids(dst_ids)
        if layout == "one image":
            _native.call("iekv_restore", dst.native.handle, ids.data_ptr(), n, host.data_ptr(),
                         host.numel(), staging.data_ptr(), staging.numel(), stream.cuda_stream,
                         side.cuda_stream)
        else:
            order = [int(i) for i in rng.permutation(n)]       # images out of order
            addresses = (ctypes.c_void_p * n)(*[host.data_ptr() + i * block for i in order])
            ids = dst.block_ids([dst_ids[i] for i in order])
            _native.call("iekv_restore_blocks", dst.native.handle, ids.data_ptr(), n, addresses,
                         staging.data_ptr(), staging.numel(), stream.cuda_stream,
                         side.cuda_stream)
        side.synchronize()
        torch.cuda.synchronize()
        untouched = bool((staging == 0xA5).all())
        assert untouched == (memory == "pinned"), (n, memory, layout)
        for d, p in zip(dst_ids, pack(src_o, src_ids)):
            dst_o.write_block(d, p)
        assert_pool_equals(dk, dv, dst_o)


@pytest.mark.parametrize("blocks,offset", [(72, 0), (16, 4096), (1, 0)],
                         ids=["72MiB-two-launches", "16MiB-interior", "1MiB"])
def test_pinned_host_transfers_on_either_side_of_the_direct_limit(gpu, blocks, offset):
    """1 MiB blocks to and from pinned host memory, always moved by the kernels
    themselves: 72 blocks exceed the 64 MiB a direct launch takes and go in two
    pack and two unpack launches (64 and 8 blocks); 16 blocks at an offset inside
    a larger pinned buffer, and a single block, in one each. The staging buffer
    keeps its sentinel bytes. Bytes equal the oracle's on the host and back in
    the pool."""
    from iekv import _native
    from iekv.engine.pools import KVPool

    bs, layers, heads, dim = 16, 4, 8, 128     # 1 MiB block images (8 arrays x 128 KiB)
    sk, sv = allocate(80, bs, layers, heads, dim, torch.bfloat16, gpu, seed=71)
    dk, dv = allocate(80, bs, layers, heads, dim, torch.bfloat16, gpu, seed=72)
    src, dst = KVPool(sk, sv, bs), KVPool(dk, dv, bs)
    rng = np.random.default_rng(73)
    src_ids, dst_ids = random_tables(rng, 80, 80, blocks)
    block = src.block_bytes
    buf = torch.empty(offset + blocks * block + 4096, dtype=torch.uint8, pin_memory=True)
    host = buf[offset:offset + blocks * block]
    staging = torch.full((4 * block,), 0xA5, dtype=torch.uint8, device=gpu)
    stream, side = torch.cuda.current_stream(), torch.cuda.Stream()
    _native.call("iekv_offload", src.native.handle, src.block_ids(src_ids).data_ptr(), blocks,
                 host.data_ptr(), host.numel(), staging.data_ptr(), staging.numel(),
                 stream.cuda_stream, side.cuda_stream)
    stream.synchronize()
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    payloads = pack(src_o, src_ids)
    assert np.array_equal(host.numpy(), packed_image(payloads).reshape(-1))
    _native.call("iekv_restore", dst.native.handle, dst.block_ids(dst_ids).data_ptr(), blocks,
                 host.data_ptr(), host.numel(), staging.data_ptr(), staging.numel(),
                 stream.cuda_stream, side.cuda_stream)
    side.synchronize()          # the copy stream is ordered after the last unpack
    for d, p in zip(dst_ids, payloads):
        dst_o.write_block(d, p)
    assert_pool_equals(dk, dv, dst_o)
    assert bool((staging == 0xA5).all())


@pytest.mark.parametrize("shape,blocks,pinned", [
    ("64k", 1, True), ("64k", 257, True), ("64k", 300, False), ("64k", 600, True),
    ("1m", 72, True), ("1m", 5, False)])
def test_host_tier_calls_with_host_ids(gpu, shape, blocks, pinned):
    """iekv_offload_ids, iekv_restore_ids and iekv_restore_blocks_ids take their
    ids from host memory (IEKV_INLINE_IDS per launch): bytes equal the oracle's on
    the direct paths (pinned images of at most 64 MiB, scattered images at most
    IEKV_INLINE_IMAGES) and on the staged pipelines (pageable memory, more than
    64 MiB or more images), for lists shorter and longer than one launch's ids."""
    from array import array

    from iekv import _native
    from iekv.engine.pools import KVPool

    bs, layers, heads, dim, dt, n_pool = ((16, 4, 4, 32, torch.float32, 640) if shape == "64k"
                                          else (16, 4, 8, 128, torch.bfloat16, 80))
    sk, sv = allocate(n_pool, bs, layers, heads, dim, dt, gpu, seed=91)
    dk, dv = allocate(n_pool, bs, layers, heads, dim, dt, gpu, seed=92)
    src, dst = KVPool(sk, sv, bs), KVPool(dk, dv, bs)
    rng = np.random.default_rng(93 + blocks)
    src_ids, dst_ids = random_tables(rng, n_pool, n_pool, blocks)
    s_host, d_host = array("i", src_ids), array("i", dst_ids)
    block = src.block_bytes
    host = torch.empty(blocks * block, dtype=torch.uint8, pin_memory=pinned)
    staging = torch.empty(4 * block, dtype=torch.uint8, device=gpu)
    stream, side = torch.cuda.current_stream(), torch.cuda.Stream()
    print(f"offload_ids {shape} x {blocks} pinned={pinned}", flush=True)
    _native.call("iekv_offload_ids", src.native.handle, s_host.buffer_info()[0], blocks,
                 host.data_ptr(), host.numel(), staging.data_ptr(), staging.numel(),
                 stream.cuda_stream, side.cuda_stream)
    stream.synchronize()
    src_o = oracle_of(sk, sv, bs)
    payloads = pack(src_o, src_ids)
    assert np.array_equal(host.numpy(), packed_image(payloads).reshape(-1))
    # The contiguous image back to dst_ids.
    dst_o = oracle_of(dk, dv, bs)
    _native.call("iekv_restore_ids", dst.native.handle, d_host.buffer_info()[0], blocks,
                 host.data_ptr(), host.numel(), staging.data_ptr(), staging.numel(),
                 stream.cuda_stream, side.cuda_stream)
    side.synchronize()
    for d, p in zip(dst_ids, payloads):
        dst_o.write_block(d, p)
    assert_pool_equals(dk, dv, dst_o)
    # The same images in reverse order, one address each, onto a fresh table.
    order = list(reversed(range(blocks)))
    again = [int(b) for b in rng.permutation(n_pool)[:blocks]]
    addresses = (ctypes.c_void_p * blocks)(*[host.data_ptr() + i * block for i in order])
    a_host = array("i", again)
    print(f"restore_blocks_ids {shape} x {blocks}", flush=True)
    _native.call("iekv_restore_blocks_ids", dst.native.handle, a_host.buffer_info()[0], blocks,
                 addresses, staging.data_ptr(), staging.numel(), stream.cuda_stream,
                 side.cuda_stream)
    side.synchronize()
    for d, i in zip(again, order):
        dst_o.write_block(d, payloads[i])
    assert_pool_equals(dk, dv, dst_o)


@pytest.mark.parametrize("blocks,memory,host_ids", [
    (1, "pinned", False), (7, "pinned", True), (128, "pinned", True), (130, "pinned", False),
    (9, "pageable", True), (300, "pinned", True)])
def test_offload_into_one_image_per_block(gpu, blocks, memory, host_ids):
    """iekv_offload_blocks(_ids) packs block ids[i] into its own host image: up to
    IEKV_INLINE_IMAGES pinned images with one launch, more images or pageable ones
    through the staged pipeline (one copy per run of images adjacent within one
    allocation). Every image equals the oracle's payload."""
    from array import array

    from iekv import _native
    from iekv.engine.pools import KVPool

    bs, layers, heads, dim = 16, 2, 4, 32            # 32 KiB block images (4 arrays x 8 KiB)
    sk, sv = allocate(400, bs, layers, heads, dim, torch.float32, gpu, seed=95)
    src = KVPool(sk, sv, bs)
    rng = np.random.default_rng(96 + blocks)
    src_ids = [int(b) for b in rng.permutation(400)[:blocks]]
    block = src.block_bytes
    # The first half of the images are allocations of their own; the second half lie
    # one after another in one shared buffer (copied as one run when staged).
    half = blocks // 2
    pinned = memory == "pinned"
    shared = torch.empty((blocks - half) * block, dtype=torch.uint8, pin_memory=pinned)
    own = [torch.empty(block, dtype=torch.uint8, pin_memory=pinned) for _ in range(half)]
    images = own + [shared[j * block:(j + 1) * block] for j in range(blocks - half)]
    addresses = (ctypes.c_void_p * blocks)(*[t.data_ptr() for t in images])
    staging = torch.empty(3 * block, dtype=torch.uint8, device=gpu)
    stream, side = torch.cuda.current_stream(), torch.cuda.Stream()
    ids = array("i", src_ids) if host_ids else src.block_ids(src_ids)
    id_ptr = ids.buffer_info()[0] if host_ids else ids.data_ptr()
    fn = "iekv_offload_blocks_ids" if host_ids else "iekv_offload_blocks"
    print(f"{fn} x {blocks} {memory}", flush=True)
    _native.call(fn, src.native.handle, id_ptr, blocks, addresses, staging.data_ptr(),
                 staging.numel(), stream.cuda_stream, side.cuda_stream)
    stream.synchronize()
    payloads = pack(oracle_of(sk, sv, bs), src_ids)
    for i, (img, want) in enumerate(zip(images, payloads)):
        assert np.array_equal(img.numpy(), packed_image([want]).reshape(-1)), i


def test_deferred_offloads_keep_one_buffer_per_block(gpu):
    """Deferred host reads flush into pinned buffers of one block each, so a payload the
    tier keeps holds only its own block; bytes equal the oracle's, and restoring a mix
    of them writes the oracle's blocks."""
    from iekv.engine.copier import HipSlotCopier

    bs = 8
    sk, sv = allocate(64, bs, 2, 2, 16, torch.bfloat16, gpu, seed=97)
    dk, dv = allocate(64, bs, 2, 2, 16, torch.bfloat16, gpu, seed=98)
    src = HipSlotCopier(sk, sv, bs, payload_location="host")
    dst = HipSlotCopier(dk, dv, bs)
    assert src.defer_reads
    reads = [src.read_block(b) for b in (5, 9, 2, 40, 33)]
    assert src.flush() == 5 and src.offload_launches == 1
    roots = {id(p.packed._root) for p in reads}
    assert len(roots) == 5 and all(len(p.packed._root) == 1 for p in reads)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    for p, b in zip(reads, (5, 9, 2, 40, 33)):
        want = packed_image(pack(src_o, [b])).reshape(-1)
        assert np.array_equal(p.packed.host_data()[p.index].reshape(-1).numpy(), want)
    dst.write_blocks([1, 2, 3], [reads[4], reads[0], reads[2]])
    torch.cuda.synchronize()
    for d, b in zip((1, 2, 3), (33, 5, 2)):
        dst_o.write_block(d, src_o.read_block(b))
    assert_pool_equals(dk, dv, dst_o)


def test_staged_host_calls_on_two_streams_share_one_staging_buffer(gpu):
    """A host copier has one device staging buffer for all its staged transfers
    (restores of pageable payloads; pinned ones are read by the kernel itself).
    Two restores of pageable payloads issued back to back on two streams must
    each write only their own bytes: the second call on a new stream is ordered
    after the first one's use of the buffer. A third, larger restore then
    replaces the buffer while the previous calls may still run. The pinned
    offloads that made the payloads used no staging. Bytes equal the oracle's."""
    from iekv.engine.copier import HipSlotCopier, PackedBlocks

    bs, layers, heads, dim = 16, 2, 8, 128               # 128 KiB block images
    sk, sv = allocate(2000, bs, layers, heads, dim, torch.bfloat16, gpu, seed=91)
    dk, dv = allocate(2000, bs, layers, heads, dim, torch.bfloat16, gpu, seed=92)
    src = HipSlotCopier(sk, sv, bs, payload_location="host", defer_reads=False)
    dst = HipSlotCopier(dk, dv, bs)
    n = 300                                  # 37.5 MiB: more than the first buffer holds
    rng = np.random.default_rng(93)
    order = [int(b) for b in rng.permutation(2000)]
    ids_a, ids_b, ids_c = order[:n], order[n:2 * n], order[2 * n:3 * n + 900]
    main = torch.cuda.current_stream()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(main)
    s2.wait_stream(main)
    pinned = [src.read_blocks(ids, stream=s) for ids, s in ((ids_a, s1), (ids_b, s2),
                                                            (ids_c, s1))]
    assert src._staging is None                          # pinned offloads: direct
    pageable = [PackedBlocks(p.synchronize().data.clone(), layers, (bs, heads, dim),
                             torch.bfloat16) for p in pinned]
    assert not any(p.pinned for p in pageable)
    targets = [int(t) for t in rng.permutation(2000)]
    da, db, dc = targets[:n], targets[n:2 * n], targets[2 * n:3 * n + 900]
    dst.write_blocks(da, pageable[0], stream=s2)
    dst.write_blocks(db, pageable[1], stream=s1)
    first = dst._staging
    dst.write_blocks(dc, pageable[2], stream=s2)         # a larger staging buffer
    assert first is not None and dst._staging.numel() > first.numel()
    main.wait_stream(s1)
    main.wait_stream(s2)
    torch.cuda.synchronize()
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    for payload, ids in zip(pinned, (ids_a, ids_b, ids_c)):
        got = payload.synchronize().data.view(torch.uint8).numpy()
        assert np.array_equal(got, packed_image(pack(src_o, ids)))
    handoff(src_o, dst_o, [ids_a, ids_b, ids_c], [da, db, dc])
    assert_pool_equals(dk, dv, dst_o)


def test_a_payload_dropped_during_its_restore_keeps_its_memory_until_done(gpu):
    """Host payloads restored and dropped at once, then new offloads made at once (which
    torch's pinned cache would serve from freed buffers): the dropped buffers are held
    until their restores finish, so every restored block is its source's bytes."""
    from iekv.engine import copier as copier_mod
    from iekv.engine.copier import HipSlotCopier

    bs, layers, heads, dim = 16, 4, 8, 128        # 1 MiB block images
    sk, sv = allocate(96, bs, layers, heads, dim, torch.bfloat16, gpu, seed=99)
    dk, dv = allocate(96, bs, layers, heads, dim, torch.bfloat16, gpu, seed=100)
    src = HipSlotCopier(sk, sv, bs, payload_location="host")
    dst = HipSlotCopier(dk, dv, bs)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    for rnd in range(4):
        ids = list(range(rnd * 16, rnd * 16 + 16))
        tier = [src.read_block(b) for b in ids]
        src.flush()
        dst.write_blocks([b + 1 for b in ids], tier)
        del tier                                   # dies while the restore may still read it
        again = [src.read_block(b) for b in range(64, 80)]
        src.flush()                                # new pinned buffers, right away
        del again
        for b in ids:
            dst_o.write_block(b + 1, src_o.read_block(b))
    torch.cuda.synchronize()
    assert_pool_equals(dk, dv, dst_o)
    copier_mod._release_finished()
    assert not copier_mod._UNFINISHED


def test_host_payload_views_wait_for_their_copy(gpu):
    """A host payload is read right after read_block / read_blocks returns, with no
    synchronisation by the caller: its tiles must already be the finished snapshot,
    for one block (written by the pack kernel), for 80 MiB (the staged pipeline)
    and for a deferred single-block read (flushed by its first access)."""
    from iekv.engine.copier import HipSlotCopier
    from iekv.serve.disaggregated import KVTransfer
    from iekv.serve.wire import to_wire

    bs, layers, heads, dim = 16, 4, 8, 128       # 1 MiB block images
    sk, sv = allocate(96, bs, layers, heads, dim, torch.bfloat16, gpu, seed=81)
    src_o = oracle_of(sk, sv, bs)
    eager = HipSlotCopier(sk, sv, bs, payload_location="host", defer_reads=False)
    deferred = HipSlotCopier(sk, sv, bs, payload_location="host", defer_reads=True)

    def as_bytes(tiles):
        return [t.contiguous().view(torch.uint8).reshape(bs, -1).numpy() for t in tiles]

    def expect(block_id, k_list, v_list):
        want_k, want_v = src_o.read_block(block_id)
        got = as_bytes(k_list) + as_bytes(v_list)
        for g, w in zip(got, list(want_k) + list(want_v)):
            assert np.array_equal(g, w)

    one = eager.read_block(17)
    k_list, v_list = one
    expect(17, k_list, v_list)
    ids = [int(b) for b in np.random.default_rng(82).permutation(96)[:80]]
    many = eager.read_blocks(ids)
    last = many[len(ids) - 1]
    expect(ids[-1], last.k, last.v)
    payload = deferred.read_block(5)
    expect(5, payload.k, payload.v)
    # The wire sender hands out the finished bytes of a host payload as well.
    again = eager.read_blocks(ids)
    _, data = to_wire(KVTransfer(token_ids=[1], num_computed=0, block_payloads=again))
    assert np.array_equal(data.numpy(), packed_image(pack(src_o, ids)))


def test_a_hip_failure_raises_and_leaves_no_error_behind(gpu):
    """A HIP call that fails inside the library (switching to a device that does not
    exist, to upload an address table) raises NativeError with IEKV_ERR_HIP and the
    runtime's message, and leaves HIP's last error clear: the next call's launch
    check must not report it again, and that call moves its blocks bit-exactly."""
    import ctypes

    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    _native.lib()
    runtime = [line.split()[-1] for line in open("/proc/self/maps")
               if line.rstrip().endswith("libamdhip64.so")][0]
    hip = ctypes.CDLL(runtime)      # the runtime instance torch and libiekv share
    missing = torch.cuda.device_count() + 7
    with pytest.raises(_native.NativeError) as err:
        _native.Pool([1 << 30, (1 << 30) + 4096, (1 << 30) + 3 * 4096], tile_bytes=64,
                     num_blocks=16, device=missing)
    assert err.value.code == _native.IEKV_ERR_HIP
    assert f"cannot make device {missing} current: " in str(err.value)
    assert hip.hipGetLastError() == 0
    bs = 16
    sk, sv = allocate(16, bs, 2, 2, 32, torch.float16, gpu, seed=85)
    dk, dv = allocate(16, bs, 2, 2, 32, torch.float16, gpu, seed=86)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    HipSlotCopier(dk, dv, bs).copy_blocks(HipSlotCopier(sk, sv, bs), [3, 9], [0, 15])
    torch.cuda.synchronize()
    handoff(src_o, dst_o, [[3, 9]], [[0, 15]])
    assert_pool_equals(dk, dv, dst_o)


def test_requests_issued_on_alternating_streams_are_bit_exact(gpu):
    """Independent requests on two side streams (copy_blocks / read_blocks /
    write_blocks with stream=), forked from and joined back into the current
    stream: every destination tile equals the oracle's, source untouched. One
    request in three mixes a host source table with device destination ids, whose
    host side is uploaded on the request's stream."""
    from iekv.engine.copier import HipSlotCopier

    bs = 16
    sk, sv = allocate(200, bs, 3, 4, 32, torch.bfloat16, gpu, seed=87)
    dk, dv = allocate(200, bs, 3, 4, 32, torch.bfloat16, gpu, seed=88)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    rng = np.random.default_rng(89)
    src_perm, dst_perm = rng.permutation(200), rng.permutation(200)
    sizes = [int(n) for n in rng.integers(1, 12, size=16)]
    at, src_tables, dst_tables = 0, [], []
    for n in sizes:
        src_tables.append([int(b) for b in src_perm[at:at + n]])
        dst_tables.append([int(b) for b in dst_perm[at:at + n]])
        at += n
    # device ids made (and complete) before the fork; held until after the join
    dst_on_device = [torch.tensor(d, dtype=torch.int32, device=gpu) for d in dst_tables]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    main = torch.cuda.current_stream()
    start = torch.cuda.Event()
    start.record(main)
    for st in streams:
        st.wait_event(start)
    for k, (s_ids, d_ids) in enumerate(zip(src_tables, dst_tables)):
        st = streams[k % 2]
        if k % 3 == 1:
            dst.copy_blocks(src, s_ids, dst_on_device[k], stream=st)
        elif k % 3:
            dst.copy_blocks(src, s_ids, d_ids, stream=st)
        else:
            dst.write_blocks(d_ids, src.read_blocks(s_ids, stream=st), stream=st)
    for st in streams:
        done = torch.cuda.Event()
        done.record(st)
        main.wait_event(done)
    torch.cuda.synchronize()
    handoff(src_o, dst_o, src_tables, dst_tables)
    assert_pool_equals(dk, dv, dst_o)
    assert_pool_equals(sk, sv, src_o)
    del dst_on_device


def test_a_request_list_moves_each_request_on_its_stream_with_its_event(gpu):
    """copy_requests (iekv_copy_direct_requests): one launch per request on streams
    in turn, an event per request; once request k's event completes, its tiles are
    in place. Empty requests, requests of one block and of hundreds, three streams;
    the whole pool equals the oracle's at the end, and bad tables are refused
    before anything is enqueued."""
    from iekv.engine.copier import HipSlotCopier

    bs = 16
    sk, sv = allocate(900, bs, 2, 2, 32, torch.float16, gpu, seed=101)
    dk, dv = allocate(900, bs, 2, 2, 32, torch.float16, gpu, seed=102)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    rng = np.random.default_rng(103)
    sizes = [3, 0, 1, 300, 17, 0, 2, 260, 40, 5]
    src_perm, dst_perm = rng.permutation(900), rng.permutation(900)
    tables, at = [], 0
    for n in sizes:
        tables.append(([int(b) for b in src_perm[at:at + n]],
                       [int(b) for b in dst_perm[at:at + n]]))
        at += n
    streams = [torch.cuda.current_stream(), torch.cuda.Stream(), torch.cuda.Stream()]
    events = [torch.cuda.Event() for _ in tables]
    dst.copy_requests(src, tables, streams=streams, done_events=events)
    src_bytes = host_bytes(sk + sv)
    for (s_ids, d_ids), ev in zip(tables, events):
        ev.synchronize()
        if not d_ids:
            continue
        d_t = torch.tensor(d_ids, device=gpu)
        for a, cache in enumerate(dk + dv):
            rows = torch.stack([d_t * bs + r for r in range(bs)], 1).reshape(-1)
            got = cache.view(torch.uint8).reshape(cache.shape[0], -1)[rows].cpu().numpy()
            want = np.concatenate([src_bytes[a][b * bs:(b + 1) * bs] for b in s_ids])
            assert np.array_equal(got, want), (a, len(d_ids))
    for st in streams:
        st.synchronize()
    handoff(src_o, dst_o, [t[0] for t in tables], [t[1] for t in tables])
    assert_pool_equals(dk, dv, dst_o)
    assert src.blocks_read == dst.blocks_written == sum(sizes)
    with pytest.raises(ValueError, match="must be distinct"):       # shared destination
        dst.copy_requests(src, [([1], [5]), ([2], [5])])
    with pytest.raises(IndexError, match="out of range"):
        dst.copy_requests(src, [([1], [900])])
    with pytest.raises(ValueError, match="2 events for 1 requests"):
        dst.copy_requests(src, [([1], [5])], done_events=[torch.cuda.Event()] * 2)
    assert dst.blocks_written == sum(sizes)


def test_short_python_tables_and_numpy_tables_move_the_same_bytes(gpu):
    """Short Python tables go to the library unconverted (it checks and orders the
    ids), NumPy arrays and long lists through the NumPy checks; both must move the
    same tiles and refuse the same ids.
    Table lengths sit on either side of INLINE_IDS (the most ids one launch's
    arguments carry; longer tables take several launches), and one direct copy
    stays within one pool."""
    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    bs = 16
    n_blocks = 700
    sk, sv = allocate(n_blocks, bs, 2, 2, 32, torch.float16, gpu, seed=91)
    src = HipSlotCopier(sk, sv, bs)
    sizes = [1, 2, 7, 100, _native.INLINE_IDS, _native.INLINE_IDS + 1, 600]
    results = []
    for as_numpy in (False, True):
        dk, dv = allocate(n_blocks, bs, 2, 2, 32, torch.float16, gpu, seed=93)
        dst = HipSlotCopier(dk, dv, bs)
        r = np.random.default_rng(94)
        for n in sizes:
            s_ids = r.permutation(n_blocks)[:n]
            d_ids = r.permutation(n_blocks)[:n]
            if as_numpy:
                dst.copy_blocks(src, s_ids, d_ids)
            else:
                dst.copy_blocks(src, [int(b) for b in s_ids], [int(b) for b in d_ids])
            s2 = r.permutation(n_blocks)[:n]
            d2 = r.permutation(n_blocks)[:n]
            payload = src.read_blocks(s2 if as_numpy else [int(b) for b in s2])
            dst.write_blocks(d2 if as_numpy else [int(b) for b in d2], payload)
        # within one pool: disjoint source and destination halves
        within = r.permutation(n_blocks)[:20]
        a, b = within[:10], within[10:]
        dst.copy_blocks(dst, a if as_numpy else [int(x) for x in a],
                        b if as_numpy else [int(x) for x in b])
        torch.cuda.synchronize()
        results.append(host_bytes(dk + dv))
        for bad in ([0, n_blocks], [-1, 3]):
            with pytest.raises(IndexError, match="out of range"):
                dst.copy_blocks(src, [1, 2], np.array(bad) if as_numpy else bad)
        with pytest.raises(ValueError, match="must be distinct"):
            dst.copy_blocks(src, [1, 2], np.array([5, 5]) if as_numpy else [5, 5])
        with pytest.raises(ValueError, match="disjoint"):
            dst.copy_blocks(dst, np.array([1, 2]) if as_numpy else [1, 2],
                            np.array([2, 3]) if as_numpy else [2, 3])
        with pytest.raises(ValueError, match="2 source blocks for 3 destinations"):
            dst.copy_blocks(src, [1, 2], np.array([4, 5, 6]) if as_numpy else [4, 5, 6])
    assert all(np.array_equal(x, y) for x, y in zip(*results))


def test_host_payloads_through_the_copier(gpu):
    from iekv.engine.copier import HipSlotCopier

    bs = 16
    sk, sv = allocate(30, bs, 2, 2, 64, torch.float16, gpu, seed=23)
    dk, dv = allocate(30, bs, 2, 2, 64, torch.float16, gpu, seed=24)
    src = HipSlotCopier(sk, sv, bs, payload_location="host")
    dst = HipSlotCopier(dk, dv, bs)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    packed = src.read_blocks([3, 14, 29, 0])
    assert packed.on_host
    one = src.read_block(11)
    dst.write_blocks([7, 8, 9, 10], packed)
    dst.write_block(12, one)
    torch.cuda.synchronize()
    handoff(src_o, dst_o, [[3, 14, 29, 0, 11]], [[7, 8, 9, 10, 12]])
    assert_pool_equals(dk, dv, dst_o)
    assert np.array_equal(packed.synchronize().data.numpy(),
                          packed_image(pack(oracle_of(sk, sv, bs), [3, 14, 29, 0])))


@pytest.mark.parametrize("memory", ["pinned", "pageable", "mixed"])
@pytest.mark.parametrize("staging_blocks", [1, 2, 3, 64])
def test_host_payloads_from_unrelated_buffers_restore_in_one_call(gpu, staging_blocks, memory):
    """Tier entries come from different offload batches: write_blocks gathers
    their host images (scattered, some adjacent) with one iekv_restore_blocks.
    Pinned images are read by one unpack launch directly; pageable copies of the
    same buffers, or a mix of pinned and pageable ones, go through a staging
    buffer of 1 to 64 blocks (1 to 7 pipeline chunks)."""
    from iekv.engine import copier as copier_mod
    from iekv.engine.copier import HipSlotCopier, PackedBlocks

    bs = 16
    sk, sv = allocate(40, bs, 3, 2, 32, torch.bfloat16, gpu, seed=26)
    dk, dv = allocate(40, bs, 3, 2, 32, torch.bfloat16, gpu, seed=27)
    src = HipSlotCopier(sk, sv, bs, payload_location="host")
    dst = HipSlotCopier(dk, dv, bs)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    first = src.read_blocks([5, 6, 7, 30])        # one offload batch
    second = src.read_blocks([12, 0, 39])         # another
    single = src.read_block(21)
    def pageable(packed):
        packed.synchronize()
        data = torch.empty(packed.data.shape, dtype=torch.uint8).copy_(packed.data)
        assert not data.is_pinned()
        return PackedBlocks(data, packed.num_layers, packed.tile_shape, packed.dtype)

    if memory != "pinned":
        first = pageable(first)
    if memory == "pageable":
        second = pageable(second)
        single = pageable(single.packed[single.index:single.index + 1])[0]
    payloads = [second[2], first[0], first[1], single, second[0], first[3], second[1]]
    src_ids = [39, 5, 6, 21, 12, 30, 0]
    dst_ids = [3, 17, 9, 33, 2, 25, 11]
    old = copier_mod.HOST_STAGING_BYTES
    copier_mod.HOST_STAGING_BYTES = staging_blocks * dst.pool.block_bytes
    try:
        dst.write_blocks(dst_ids, payloads)
    finally:
        copier_mod.HOST_STAGING_BYTES = old
    assert dst.restore_launches == 1
    torch.cuda.synchronize()
    handoff(src_o, dst_o, [src_ids], [dst_ids])
    assert_pool_equals(dk, dv, dst_o)
    assert dst.blocks_written == 7


def test_scattered_host_images_are_copied_together_only_within_one_allocation(gpu):
    """The staged path of the scattered-image calls copies each run of host images
    that are adjacent inside one pinned allocation with one hipMemcpyAsync, and
    starts a new copy at every allocation's end (a copy spanning two allocations
    would run past the end of the one its host pointer belongs to).

    Three pinned buffers of 50 block images each, and one pageable image: a list
    with any image outside pinned memory takes the staged pipeline (an all-pinned
    list is moved by the kernels directly). One iekv_offload_blocks call of 151
    blocks lists the pinned images buffer after buffer, then the pageable one: runs
    to merge and, at two places, a step from one allocation's last image to
    another's first. Where the allocator placed two buffers back to back (on MI355X
    boxes so far it has left a gap of at least one buffer's size after each pinned
    allocation), that step is adjacent in memory too, and the run must still end
    there. A second offload interleaves the buffers image by image (no merges).
    Every image equals the oracle's, and one iekv_restore_blocks of all 151 (staged
    as well) writes the oracle's blocks."""
    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    bs = 16
    sk, sv = allocate(160, bs, 2, 2, 64, torch.bfloat16, gpu, seed=61)   # 16 KiB images
    dk, dv = allocate(160, bs, 2, 2, 64, torch.bfloat16, gpu, seed=62)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    rng = np.random.default_rng(63)
    shape = (50, src.pool.n_arrays, src.pool.tile_bytes)
    bufs = [torch.empty(shape, dtype=torch.uint8, pin_memory=True) for _ in range(3)]
    bufs.append(torch.empty((1,) + shape[1:], dtype=torch.uint8))     # pageable
    ends = {b.data_ptr() + b.numel() for b in bufs[:3]}
    print(f"{len(ends & {b.data_ptr() for b in bufs[:3]})} pinned buffers start where another "
          f"ends", flush=True)
    image = src.pool.block_bytes
    # Two slots of 32 images: both steps between buffers (entries 50 and 100) fall
    # inside a chunk, where the copies of one chunk are planned together.
    staging = torch.empty(64 * image, dtype=torch.uint8, device=gpu)
    stream, side = torch.cuda.current_stream(), torch.cuda.Stream()
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    n = 151
    for layout in ("buffer after buffer", "interleaved"):
        picks = [(b, i) for i in range(50) for b in range(3)] if layout == "interleaved" \
            else [(b, i) for b in range(3) for i in range(50)]
        picks.append((3, 0))
        sources = [int(x) for x in rng.permutation(160)[:n]]
        addresses = (ctypes.c_void_p * n)(*[bufs[b].data_ptr() + i * image for b, i in picks])
        _native.call("iekv_offload_blocks", src.pool.native.handle,
                     src.pool.block_ids(sources).data_ptr(), n, addresses, staging.data_ptr(),
                     staging.numel(), stream.cuda_stream, side.cuda_stream)
        torch.cuda.synchronize()
        want = packed_image(pack(src_o, sources))
        for k, (b, i) in enumerate(picks):
            assert np.array_equal(bufs[b][i].numpy(), want[k]), (layout, k)
        targets = [int(t) for t in rng.permutation(160)[:n]]
        _native.call("iekv_restore_blocks", dst.pool.native.handle,
                     dst.pool.block_ids(targets).data_ptr(), n, addresses, staging.data_ptr(),
                     staging.numel(), stream.cuda_stream, side.cuda_stream)
        side.synchronize()
        torch.cuda.synchronize()
        handoff(src_o, dst_o, [sources], [targets])
        assert_pool_equals(dk, dv, dst_o)


def test_more_scattered_images_than_one_direct_launch_takes(gpu):
    """130 one-block tier payloads (more than IEKV_INLINE_IMAGES) restore through the
    copier in two direct calls (128 images, then 2), and in one library call, which
    makes the two launches itself; bytes equal to the oracle's either way."""
    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    bs = 4
    sk, sv = allocate(140, bs, 1, 1, 32, torch.float32, gpu, seed=81)   # 512 B tiles
    dk, dv = allocate(140, bs, 1, 1, 32, torch.float32, gpu, seed=82)
    src = HipSlotCopier(sk, sv, bs, payload_location="host", defer_reads=False)
    dst = HipSlotCopier(dk, dv, bs)
    n = _native.INLINE_IMAGES + 2
    rng = np.random.default_rng(83)
    src_ids, dst_ids = random_tables(rng, 140, 140, n)
    payloads = [src.read_blocks([b])[0] for b in src_ids]
    dst.write_blocks(dst_ids, payloads)
    assert dst.restore_launches == 2
    torch.cuda.synchronize()
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    handoff(src_o, dst_o, [src_ids], [dst_ids])
    assert_pool_equals(dk, dv, dst_o)
    # All 130 in one library call: two direct unpack launches inside the library.
    again = [int(b) for b in rng.permutation(140)[:n]]
    addresses = (ctypes.c_void_p * n)(*[p.packed.data[p.index].data_ptr() for p in payloads])
    staging = torch.empty(8 * src.pool.block_bytes, dtype=torch.uint8, device=gpu)
    stream, side = torch.cuda.current_stream(), torch.cuda.Stream()
    _native.call("iekv_restore_blocks", dst.pool.native.handle,
                 dst.pool.block_ids(again).data_ptr(), n, addresses, staging.data_ptr(),
                 staging.numel(), stream.cuda_stream, side.cuda_stream)
    side.synchronize()
    handoff(src_o, dst_o, [src_ids], [again])
    assert_pool_equals(dk, dv, dst_o)


def test_a_victim_read_sees_the_bytes_before_a_restore_overwrites_them(gpu):
    """Restore into block X right after offloading X's victim (ie/core/block_manager.py:161-162)."""
    from iekv.engine.copier import HipSlotCopier

    bs = 16
    k, v = allocate(6, bs, 2, 2, 16, torch.float32, gpu, seed=25)
    tier_copier = HipSlotCopier(k, v, bs, payload_location="host")
    before = host_bytes(k) + host_bytes(v)
    saved = tier_copier.read_block(1)           # the returning prefix, offloaded earlier
    victim = tier_copier.read_block(4)          # eviction of block 4's old contents
    tier_copier.write_block(4, saved)           # restore lands in the same block
    torch.cuda.synchronize()
    got = victim.packed.synchronize().tiles(victim.index).view(torch.uint8).reshape(4, bs, -1).numpy()
    for a in range(4):
        assert np.array_equal(got[a], before[a][4 * bs:5 * bs])
    after = host_bytes(k) + host_bytes(v)
    for a in range(4):
        assert np.array_equal(after[a][4 * bs:5 * bs], before[a][1 * bs:2 * bs])


def test_cfg1_handoff_reproduces_the_reference_digests(gpu):
    """The CPU-runnable benchmark case on the GPU, checked against the reference's own output."""
    from iekv.engine.copier import HipSlotCopier
    from iekv.engine.pools import allocate_pool

    g = golden("cfg1_handoff")
    _, src_tables, k_np, v_np = cfg1_inputs()
    sk, sv = allocate_pool(4096, 16, 4, 4, 32, dtype=torch.float32, device=gpu)
    for t, a in zip(sk + sv, k_np + v_np):
        t.copy_(torch.from_numpy(a))
    src = HipSlotCopier(sk, sv, 16)

    def digests(k, v):
        return ([hashlib.sha256(t.cpu().numpy().tobytes()).hexdigest() for t in k],
                [hashlib.sha256(t.cpu().numpy().tobytes()).hexdigest() for t in v])

    # pack -> unpack, request by request
    dk, dv = allocate_pool(4096, 16, 4, 4, 32, dtype=torch.float32, device=gpu)
    dst = HipSlotCopier(dk, dv, 16)
    image = hashlib.sha256()
    for s_tab, d_tab in zip(src_tables, g["dst_tables"]):
        packed = src.read_blocks(s_tab)
        image.update(packed.data.cpu().numpy().tobytes())
        dst.write_blocks(d_tab, packed)
    torch.cuda.synchronize()
    assert image.hexdigest() == g["packed_sha256"]
    assert digests(dk, dv) == (g["dst_sha256"]["k"], g["dst_sha256"]["v"])
    assert src.blocks_read == g["src_counters"]["blocks_read"]
    assert src.bytes_moved == g["src_counters"]["bytes_moved"]
    assert dst.bytes_moved == g["dst_counters"]["bytes_moved"]

    # direct, all requests in one launch
    dk2, dv2 = allocate_pool(4096, 16, 4, 4, 32, dtype=torch.float32, device=gpu)
    dst2 = HipSlotCopier(dk2, dv2, 16)
    dst2.copy_blocks(src, sum(src_tables, []), sum(g["dst_tables"], []))
    torch.cuda.synchronize()
    assert digests(dk2, dv2) == (g["dst_sha256"]["k"], g["dst_sha256"]["v"])
    assert digests(sk, sv) == (g["src_sha256"]["k"], g["src_sha256"]["v"])


def test_deferred_host_reads_batch_and_keep_snapshot_semantics(gpu):
    from iekv.engine.copier import DeferredBlockPayload, HipSlotCopier

    bs = 16
    k, v = allocate(12, bs, 2, 2, 16, torch.float16, gpu, seed=26)
    before = host_bytes(k) + host_bytes(v)
    copier = HipSlotCopier(k, v, bs, payload_location="host")
    kept = [copier.read_block(b) for b in (3, 7, 9)]
    dropped = copier.read_block(5)
    assert all(isinstance(p, DeferredBlockPayload) for p in kept)
    assert copier.pending_reads == 4 and copier.blocks_read == 4
    del dropped                                   # nobody holds it: never copied
    copier.write_block(7, kept[0])                # a write flushes the queued reads first
    torch.cuda.synchronize()
    assert copier.offload_launches == 1 and copier.blocks_offloaded == 3
    for payload, block in zip(kept, (3, 7, 9)):
        got = payload.packed.synchronize().tiles(payload.index).view(torch.uint8).reshape(4, bs, -1)
        for a in range(4):
            assert np.array_equal(got[a].numpy(), before[a][block * bs:(block + 1) * bs])
    after = host_bytes(k) + host_bytes(v)
    for a in range(4):
        assert np.array_equal(after[a][7 * bs:8 * bs], before[a][3 * bs:4 * bs])


def test_launch_timer_times_each_library_launch(gpu):
    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    sk, sv = allocate(40, 16, 2, 8, 128, torch.bfloat16, gpu, seed=27)
    dk, dv = allocate(40, 16, 2, 8, 128, torch.bfloat16, gpu, seed=28)
    src, dst = HipSlotCopier(sk, sv, 16), HipSlotCopier(dk, dv, 16)
    with _native.LaunchTimer(8) as timer:
        dst.copy_blocks(src, [1, 2, 3], [4, 5, 6])
        packed = src.read_blocks([7, 8])
        dst.write_blocks([9, 10], packed)
    assert len(timer.durations_ms) == 3 and all(ms > 0 for ms in timer.durations_ms)
    dst.copy_blocks(src, [11], [12])          # outside a session: launched, not timed
    with _native.LaunchTimer(2) as timer:     # a session with no launches
        pass
    assert timer.durations_ms == []


@pytest.mark.parametrize("pad", [1, 3])
def test_padded_pools_move_bit_exactly(gpu, pad):
    """Pools whose arrays are padded by unused blocks (pad_blocks) are still one slab
    of equally spaced arrays: direct copies, pack -> unpack and a host round trip
    between a padded and an unpadded pool equal the oracle's, and the padding
    bytes are never written."""
    from iekv.engine.copier import HipSlotCopier
    from iekv.engine.pools import allocate_pool

    bs, layers, heads, dim = 16, 3, 2, 64
    sk, sv = allocate_pool(40, bs, layers, heads, dim, dtype=torch.bfloat16, device=gpu,
                           zero=False, pad_blocks=pad)
    slab = sk[0]._base
    raw = slab.view(torch.uint8)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(61 + pad)
    raw.copy_(torch.randint(0, 256, raw.shape, dtype=torch.uint8, device=gpu, generator=gen))
    dk, dv = allocate_pool(50, bs, layers, heads, dim, dtype=torch.bfloat16, device=gpu,
                           zero=True, pad_blocks=pad)
    dslab = dk[0]._base
    dslab.view(torch.uint8).fill_(0x5A)
    for t in dk + dv:
        t.zero_()                                     # the arrays; padding keeps 0x5A
    src = HipSlotCopier(sk, sv, bs, payload_location="host")
    dst = HipSlotCopier(dk, dv, bs)
    assert src.pool.native.handle.value and len(sk[0].shape) == 3
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(62)
    a_src, a_dst = random_tables(rng, 40, 50, 12)
    dst.copy_blocks(src, a_src, a_dst)
    b_src = [int(b) for b in rng.permutation(40)[:9]]
    b_dst = [int(b) for b in rng.permutation([b for b in range(50) if b not in a_dst])[:9]]
    dst.write_blocks(b_dst, src.read_blocks(b_src))            # host round trip
    torch.cuda.synchronize()
    handoff(src_o, dst_o, [a_src, b_src], [a_dst, b_dst])
    assert_pool_equals(dk, dv, dst_o)
    rows = 50 * bs
    padding = dslab.view(2, layers, -1, heads, dim)[:, :, rows:]
    assert bool((padding.contiguous().view(torch.uint8) == 0x5A).all())


@pytest.mark.parametrize("chunks", [(4096, 8192), (1024, 16384), (8192, 2048)],
                         ids=["staging4K-pool8K", "staging1K-pool16K", "staging8K-pool2K"])
def test_unpack_chunk_follows_the_tile_size(gpu, chunks):
    """An unpack takes the pool-writing chunk (iekv_set_direct_chunk) when its tiles
    are at least that large and the staging chunk otherwise, so with the two settings
    apart every tile size takes another launch shape on each side of the pair: tiles
    of 1 to 32 KiB, split or grouped, through pack -> unpack and the direct copy,
    against the oracle byte for byte."""
    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    staging_chunk, pool_chunk = chunks
    before = _native.get_launch()
    try:
        _native.set_launch(chunk_bytes=staging_chunk, direct_chunk_bytes=pool_chunk)
        for heads, dim in ((1, 32), (2, 64), (4, 64), (8, 64), (8, 128)):   # 1 .. 32 KiB tiles
            bs, layers = 16, 3
            sk, sv = allocate(48, bs, layers, heads, dim, torch.bfloat16, gpu, seed=70 + heads)
            dk, dv = allocate(40, bs, layers, heads, dim, torch.bfloat16, gpu, seed=80 + heads)
            src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
            rng = np.random.default_rng(90 + heads)
            src_ids, dst_ids = random_tables(rng, 48, 40, 30)
            src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
            tile = src.pool.tile_bytes
            print(f"[unpack chunk] {chunks} tile {tile} B", flush=True)
            dev = lambda ids: torch.tensor(ids, dtype=torch.int32, device=gpu)  # noqa: E731
            packed = src.read_blocks(dev(src_ids[:18]))
            dst.write_blocks(dev(dst_ids[:18]), packed)
            dst.copy_blocks(src, dev(src_ids[18:]), dev(dst_ids[18:]))
            torch.cuda.synchronize()
            assert np.array_equal(packed.data.cpu().numpy(),
                                  packed_image(pack(src_o, src_ids[:18]))), (chunks, tile)
            handoff(src_o, dst_o, [src_ids], [dst_ids])
            assert_pool_equals(dk, dv, dst_o)
    finally:
        _native.set_launch(**before)
