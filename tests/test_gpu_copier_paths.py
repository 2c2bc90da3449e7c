"""Less-trodden paths of the drop-in copier (GPU), byte for byte against the NumPy oracle.

The reference's payload shape and indexing, deferred reads into device payloads
that a later write must not overtake, payloads gathered from several reads into
one buffer or taken from a strided slice, and host buffers dropped while their
copies still run.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.copier import handoff, pack, packed_image
from test_gpu_kernels import allocate, assert_pool_equals, oracle_of, random_tables

pytestmark = pytest.mark.gpu


def image_of(payload) -> np.ndarray:
    """A payload's bytes as its [2L, T] image (K tiles of every layer, then V)."""
    k, v = payload
    return np.stack([t.contiguous().view(torch.uint8).reshape(-1).cpu().numpy()
                     for t in (*k, *v)])


def test_payloads_keep_the_reference_shape_and_index_like_a_list(gpu):
    """A payload unpacks, indexes and measures as the reference's (k_list, v_list)
    (ie/engine/copier.py:18-22): len 2, [0] the K tiles and [1] the V tiles of every
    layer, as many bytes as a block; the packed list indexes from either end like
    the reference's block_payloads list and refuses indexes past either end."""
    from iekv.engine.copier import HipSlotCopier

    bs, layers, heads, dim = 4, 3, 2, 8
    sk, sv = allocate(40, bs, layers, heads, dim, torch.bfloat16, gpu, seed=81)
    copier = HipSlotCopier(sk, sv, bs)
    ids = [7, 3, 30, 11]
    packed = copier.read_blocks(ids)
    torch.cuda.synchronize()
    want = packed_image(pack(oracle_of(sk, sv, bs), ids))
    assert len(packed) == 4
    for i in range(-4, 4):
        p = packed[i]
        assert len(p) == 2 and len(p[0]) == layers and len(p[1]) == layers
        assert tuple(p[0][0].shape) == (bs, heads, dim) and p[1][-1].dtype == torch.bfloat16
        assert p.nbytes == 2 * layers * bs * heads * dim * 2
        assert np.array_equal(image_of(p), want[i % 4]), i
        k, v = p
        assert all(torch.equal(a.view(torch.uint8), b.view(torch.uint8))
                   for a, b in zip(k + v, p[0] + p[1]))
    for bad in (4, -5):
        with pytest.raises(IndexError):
            packed[bad]


def test_a_deferred_device_read_is_gathered_before_a_write_overtakes_it(gpu):
    """With deferred reads (defer_reads=True) a device payload is a promise until the
    copier flushes. A direct copy onto the read block flushes first, so the payload
    still holds the block as it was at read_block time; a payload read before any
    flush gathers itself on first use; a payload dropped before the flush is
    skipped."""
    from iekv.engine.copier import DeferredBlockPayload, HipSlotCopier

    bs, layers, heads, dim = 2, 2, 4, 16
    sk, sv = allocate(24, bs, layers, heads, dim, torch.float16, gpu, seed=82)
    dk, dv = allocate(24, bs, layers, heads, dim, torch.float16, gpu, seed=83)
    src = HipSlotCopier(sk, sv, bs)
    dst = HipSlotCopier(dk, dv, bs, payload_location="device", defer_reads=True)
    before = oracle_of(dk, dv, bs)
    p = dst.read_block(5)
    assert isinstance(p, DeferredBlockPayload) and dst.pending_reads == 1
    dst.copy_blocks(src, [2], [5])            # overwrites block 5: the read goes first
    assert dst.pending_reads == 0
    torch.cuda.synchronize()
    assert np.array_equal(image_of(p), packed_image([before.read_block(5)])[0])
    after = oracle_of(dk, dv, bs)
    assert np.array_equal(packed_image([after.read_block(5)])[0],
                          packed_image([oracle_of(sk, sv, bs).read_block(2)])[0])
    q = dst.read_block(9)
    assert dst.pending_reads == 1
    assert q.index == 0 and dst.pending_reads == 0   # first use gathers it
    torch.cuda.synchronize()
    assert np.array_equal(image_of(q), packed_image([after.read_block(9)])[0])
    r = dst.read_block(12)
    del r
    assert dst.flush() == 0                   # nobody holds it: nothing is moved
    assert_pool_equals(dk, dv, after)


def test_payloads_from_several_reads_and_strided_slices_restore_the_same_bytes(gpu):
    """stack_payloads gathers payloads of different reads into one contiguous
    buffer that one unpack restores. A strided slice of a payload list
    (payloads[::2], which the reference's list allows) is not one run of rows: its
    device rows are written one by one, its host rows through the scattered-image
    restore, and a single payload taken from it is written as its own row. Every
    destination block equals the source block read, as the reference's write_block
    loop leaves it."""
    from iekv.engine.copier import HipSlotCopier, stack_payloads

    bs, layers, heads, dim = 4, 2, 2, 32
    sk, sv = allocate(32, bs, layers, heads, dim, torch.float32, gpu, seed=84)
    dk, dv = allocate(40, bs, layers, heads, dim, torch.float32, gpu, seed=85)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    first, second = src.read_blocks([1, 2, 3]), src.read_blocks([10, 11])
    stacked = stack_payloads([first[2], second[0], first[0]])
    assert len(stacked) == 3 and stacked.data.is_contiguous()
    dst.write_blocks([20, 21, 22], stacked)
    strided = first[::2]                      # blocks 1 and 3: rows 0 and 2
    assert len(strided) == 2 and not strided.data.is_contiguous()
    dst.write_blocks([30, 31], strided)
    dst.write_block(34, strided[1])           # one row of a strided slice: block 3
    host = src.read_blocks([4, 5, 6, 7, 8], location="host")
    dst.write_blocks([35, 36, 37], host[::2])             # blocks 4, 6 and 8, from the host
    dst.write_blocks([38, 39], [host[::2][1], host[1]])   # rows of two views: 6, 5
    torch.cuda.synchronize()
    for d, s in ((20, 3), (21, 10), (22, 1), (30, 1), (31, 3), (34, 3), (35, 4), (36, 6),
                 (37, 8), (38, 6), (39, 5)):
        dst_o.write_block(d, src_o.read_block(s))
    assert_pool_equals(dk, dv, dst_o)
    with pytest.raises(ValueError):
        stack_payloads([])


def test_host_buffers_dropped_while_their_copies_run_are_held_then_released(gpu):
    """A host payload dropped while its device-to-host copy still runs keeps its
    pinned buffer alive until that copy ends, so the memory is not handed out
    again early. Forty payloads dropped behind a long copy on the same stream are
    held, pass the 32-buffer mark at which finished ones are let go, and are all
    released once the stream is idle; the payloads that were kept hold their
    blocks' bytes."""
    from iekv.engine import copier as copier_module
    from iekv.engine.copier import HipSlotCopier

    bs, layers, heads, dim = 16, 4, 8, 128        # 32 KiB bf16 tiles, 256 KiB blocks
    n = 4096                                      # 1 GiB pools: a copy of every block
    sk, sv = allocate(n, bs, layers, heads, dim, torch.bfloat16, gpu, seed=86)
    dk, dv = allocate(n, bs, layers, heads, dim, torch.bfloat16, gpu, seed=87)
    src = HipSlotCopier(sk, sv, bs, payload_location="host", defer_reads=False)
    dst = HipSlotCopier(dk, dv, bs)
    ids = torch.arange(n, dtype=torch.int32, device=gpu)
    copier_module._release_finished()
    held_before = len(copier_module._UNFINISHED)
    kept = []
    for _ in range(6):                            # about 2 ms of copies ahead of the reads,
        dst.copy_blocks(src, ids, ids)            # which Python issues in well under that
    for i in range(40):
        p = src.read_block(i)
        if i % 10 == 0:
            kept.append((i, p))
        del p                                     # the rest die while queued
    held_peak = len(copier_module._UNFINISHED)
    torch.cuda.synchronize()
    copier_module._release_finished()
    assert held_peak > held_before                # buffers were held while copies ran
    assert len(copier_module._UNFINISHED) == 0    # and all let go once they finished
    src_o = oracle_of(sk, sv, bs)
    for i, p in kept:
        assert np.array_equal(image_of(p), packed_image([src_o.read_block(i)])[0]), i


def test_the_copier_without_torchs_raw_stream_accessors(gpu, monkeypatch):
    """Where torch lacks its raw stream accessors the copier uses the public ones:
    torch.cuda.current_stream for the launch stream and torch.cuda.stream for a
    stream= call. The same calls then run on the same streams and move the same
    bytes, and each call leaves the current stream as it found it."""
    from iekv.engine import pools
    from iekv.engine.copier import HipSlotCopier

    monkeypatch.setattr(pools, "_raw_current_stream", None)
    monkeypatch.setattr(pools, "_LIGHT_SCOPE", False)
    bs, layers, heads, dim = 4, 2, 2, 16
    sk, sv = allocate(24, bs, layers, heads, dim, torch.float16, gpu, seed=92)
    dk, dv = allocate(24, bs, layers, heads, dim, torch.float16, gpu, seed=93)
    src, dst = HipSlotCopier(sk, sv, bs), HipSlotCopier(dk, dv, bs)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    assert pools.current_stream_handle(gpu) == torch.cuda.current_stream(gpu).cuda_stream
    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    before = torch.cuda.current_stream(gpu)
    packed = src.read_blocks([3, 9, 14], stream=side)
    assert torch.cuda.current_stream(gpu) == before
    dst.write_blocks([1, 2, 3], packed, stream=side)
    dst.copy_blocks(src, [20, 21], [10, 11], stream=side)
    assert torch.cuda.current_stream(gpu) == before
    side.synchronize()
    for d, s in ((1, 3), (2, 9), (3, 14), (10, 20), (11, 21)):
        dst_o.write_block(d, src_o.read_block(s))
    assert_pool_equals(dk, dv, dst_o)


def test_pools_whose_arrays_interleave_in_memory_are_told_apart(gpu):
    """Two pools may take turns along one allocation (pool A's arrays at even
    positions, pool B's at odd ones). Their spans overlap, so only the sorted walk
    over every array decides: they share no byte and copy into each other like two
    allocations. A pool over part of another's arrays is refused."""
    from iekv.engine.copier import HipSlotCopier
    from iekv.engine.pools import KVPool

    bs, heads, dim, n = 2, 2, 8, 16
    slab = torch.randint(0, 256, (8, n * bs, heads, dim * 2), dtype=torch.uint8,
                         device=gpu).view(torch.float16)
    arrays = [slab[i] for i in range(8)]
    a_k, a_v = arrays[0:4:2], arrays[4:8:2]       # arrays 0, 2 | 4, 6
    b_k, b_v = arrays[1:4:2], arrays[5:8:2]       # arrays 1, 3 | 5, 7
    a, b = HipSlotCopier(a_k, a_v, bs), HipSlotCopier(b_k, b_v, bs)
    assert a.pool.memory_relation(b.pool) == "separate"
    a_o, b_o = oracle_of(a_k, a_v, bs), oracle_of(b_k, b_v, bs)
    b.copy_blocks(a, [0, 5, 9], [9, 5, 0])         # the same ids: separate pools
    torch.cuda.synchronize()
    for d, s in ((9, 0), (5, 5), (0, 9)):
        b_o.write_block(d, a_o.read_block(s))
    assert_pool_equals(b_k, b_v, b_o)
    assert_pool_equals(a_k, a_v, a_o)              # the source is untouched
    half = [t[: n * bs // 2] for t in a_k], [t[: n * bs // 2] for t in a_v]
    with pytest.raises(ValueError, match="overlap"):
        KVPool(*half, bs).same_pool_as(a.pool)


def test_copiers_used_from_several_host_threads_at_once(gpu):
    """The library keeps no shared mutable state on its launch path (error text is
    per thread, launch settings are atomics, pool handles never change), so four
    host threads, each moving requests between pools of its own on a stream of its
    own by direct copy, pack -> unpack and with host and device ids, interleave
    freely; every pool ends byte for byte as the oracle's sequential handoffs leave
    it, and an error raised in one thread carries that thread's message."""
    import threading

    from iekv import _native
    from iekv.engine.copier import HipSlotCopier

    bs, layers, heads, dim, n = 4, 2, 2, 32, 64
    jobs = []
    for t in range(4):
        sk, sv = allocate(n, bs, layers, heads, dim, torch.bfloat16, gpu, seed=300 + t)
        dk, dv = allocate(n, bs, layers, heads, dim, torch.bfloat16, gpu, seed=400 + t)
        rng = np.random.default_rng(500 + t)
        tables = [random_tables(rng, n, n, int(rng.integers(1, 12))) for _ in range(25)]
        jobs.append(dict(src=HipSlotCopier(sk, sv, bs), dst=HipSlotCopier(dk, dv, bs),
                         src_o=oracle_of(sk, sv, bs), dst_o=oracle_of(dk, dv, bs),
                         pools=(dk, dv), tables=tables, stream=torch.cuda.Stream(gpu),
                         error=None, message=None))
    torch.cuda.synchronize()
    start = threading.Barrier(len(jobs))

    def work(job):
        try:
            start.wait()
            with torch.cuda.stream(job["stream"]):
                for i, (s, d) in enumerate(job["tables"]):
                    if i % 3 == 0:
                        job["dst"].copy_blocks(job["src"], s, d)
                    elif i % 3 == 1:
                        job["dst"].write_blocks(d, job["src"].read_blocks(s))
                    else:
                        ids = lambda x: torch.tensor(x, dtype=torch.int32, device=gpu)
                        job["dst"].copy_blocks(job["src"], ids(s), ids(d))
                try:
                    job["dst"].copy_blocks(job["src"], [0], [n + 7])
                except IndexError as e:
                    job["message"] = str(e)
            job["stream"].synchronize()
        except BaseException as e:        # reported by the main thread
            job["error"] = e

    threads = [threading.Thread(target=work, args=(job,)) for job in jobs]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads)
    for job in jobs:
        assert job["error"] is None, job["error"]
        assert job["message"] is not None and str(n + 7) in job["message"]
        for s, d in job["tables"]:
            handoff(job["src_o"], job["dst_o"], [s], [d])
        assert_pool_equals(*job["pools"], job["dst_o"])
    assert _native.lib().iekv_abi_version() == _native.ABI_VERSION
