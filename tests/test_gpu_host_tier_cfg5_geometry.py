"""The host tier at the 70B-share workload's block geometry, against the oracle (GPU).

cfg5's blocks are 80 layers x K/V of 16 KiB fp8 tiles: 160 arrays, 2.5 MiB block
images, a size that is not a power of two. On bounded pools (400 blocks, 1 GB
each) every host path moves such blocks and is compared byte for byte with the
NumPy restatement of the reference copier (ie/engine/copier.py:18-31):

* iekv_offload of a whole list (300 images, 750 MB) into a host image pinned at
  exactly its size (the pack kernel writes it, 25 images per launch), then
  iekv_restore of that image onto other ids (the unpack kernel reads it); the same
  list through pageable memory (the staged pipelines: 102 images per staging slot,
  runtime copies);
* the same calls once per block on interior addresses of that image (direct);
* the drop-in tier path: deferred evictions flushed 64 at a time into one-block
  buffers of exactly 2.5 MiB (iekv_offload_blocks_ids, 25 images per launch),
  restored as scattered tier entries (iekv_restore_blocks_ids), and the same
  payloads restored from pageable copies through the staged pipeline;
* a copier whose transfers are all direct holds no device staging;
* the one-block buffers go back to the free list when the payloads die, and
  release_pinned frees them.

Reference: ie/core/block_manager.py:79-85 (offload hook), :159-167 (restore),
ie/engine/engine.py:57-63 (the offload copier).
"""
from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

from oracle.copier import LayeredSlotCopier, pack, packed_image

pytestmark = pytest.mark.gpu

BS, LAYERS, HEADS, DIM = 16, 80, 8, 128      # cfg5: 16 KiB fp8 tiles, 2.5 MiB blocks
BLOCKS = 400


def pool(device, seed):
    from iekv.engine.pools import allocate_pool

    k, v = allocate_pool(BLOCKS, BS, LAYERS, HEADS, DIM, dtype=torch.float8_e4m3fn,
                         device=device, zero=False)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    raw = (k[0]._base if k[0]._base is not None else k[0]).view(torch.uint8)
    raw.copy_(torch.randint(0, 256, raw.shape, dtype=torch.uint8, device=device, generator=gen))
    return k, v


def host_bytes(arrays):
    return [t.view(torch.uint8).reshape(t.shape[0], -1).cpu().numpy() for t in arrays]


def oracle(k, v):
    return LayeredSlotCopier(host_bytes(k), host_bytes(v), BS)


def assert_equal_pools(k, v, want):
    for a, (got, exp) in enumerate(zip(host_bytes(k) + host_bytes(v),
                                        list(want.k_caches) + list(want.v_caches))):
        if not np.array_equal(got, exp):
            rows = np.nonzero((got != exp).any(axis=1))[0]
            raise AssertionError(f"array {a}: {rows.size} rows differ, first {rows[0]}")


def test_whole_list_and_per_block_host_calls_at_the_70b_share_geometry(gpu):
    from iekv import _native
    from iekv.engine.copier import HOST_STAGING_BYTES
    from iekv.engine.pools import KVPool, pinned_empty, release_pinned

    sk, sv = pool(gpu, 501)
    dk, dv = pool(gpu, 502)
    src, dst = KVPool(sk, sv, BS), KVPool(dk, dv, BS)
    bb = src.block_bytes
    assert (src.n_arrays, src.tile_bytes, bb) == (160, 16384, 2621440)
    src_o, dst_o = oracle(sk, sv), oracle(dk, dv)
    rng = np.random.default_rng(503)
    n = 300
    src_ids = [int(b) for b in rng.permutation(BLOCKS)[:n]]
    dst_ids = [int(b) for b in rng.permutation(BLOCKS)[:n]]
    staging = torch.empty(2 * HOST_STAGING_BYTES, dtype=torch.uint8, device=gpu)
    stream, side = torch.cuda.current_stream(), torch.cuda.Stream()
    host = pinned_empty(n * bb)
    print(f"[cfg5-geometry] whole list: {n} blocks, {n * bb} bytes pinned exactly", flush=True)
    s_ids, d_ids = src.block_ids(src_ids), dst.block_ids(dst_ids, unique=True)
    _native.call("iekv_offload", src.native.handle, s_ids.data_ptr(), n, host.data_ptr(),
                 host.numel(), staging.data_ptr(), staging.numel(), stream.cuda_stream,
                 side.cuda_stream)
    stream.synchronize()
    payloads = pack(src_o, src_ids)
    assert np.array_equal(host.numpy().reshape(n, 160, 16384), packed_image(payloads))
    _native.call("iekv_restore", dst.native.handle, d_ids.data_ptr(), n, host.data_ptr(),
                 host.numel(), None, 0, stream.cuda_stream, stream.cuda_stream)
    stream.synchronize()
    for d, p in zip(dst_ids, payloads):
        dst_o.write_block(d, p)
    assert_equal_pools(dk, dv, dst_o)

    print("[cfg5-geometry] the same list through pageable memory (staged)", flush=True)
    pageable = torch.empty(n * bb, dtype=torch.uint8)
    again = [int(b) for b in rng.permutation(BLOCKS)[:n]]
    _native.call("iekv_offload", src.native.handle, s_ids.data_ptr(), n, pageable.data_ptr(),
                 pageable.numel(), staging.data_ptr(), staging.numel(), stream.cuda_stream,
                 side.cuda_stream)
    stream.synchronize()
    assert np.array_equal(pageable.numpy().reshape(n, 160, 16384), packed_image(payloads))
    a_ids = dst.block_ids(again, unique=True)
    _native.call("iekv_restore", dst.native.handle, a_ids.data_ptr(), n, pageable.data_ptr(),
                 pageable.numel(), staging.data_ptr(), staging.numel(), stream.cuda_stream,
                 side.cuda_stream)
    side.synchronize()
    stream.synchronize()
    for d, p in zip(again, payloads):
        dst_o.write_block(d, p)
    assert_equal_pools(dk, dv, dst_o)
    del pageable

    print("[cfg5-geometry] one call per block on 64 blocks", flush=True)
    each_src = [int(b) for b in rng.permutation(BLOCKS)[:64]]
    each_dst = [int(b) for b in rng.permutation(BLOCKS)[:64]]
    host.fill_(0)
    for i, b in enumerate(each_src):
        one = src.block_ids([b])
        _native.call("iekv_offload", src.native.handle, one.data_ptr(), 1,
                     host.data_ptr() + i * bb, bb, None, 0, stream.cuda_stream,
                     side.cuda_stream)
    stream.synchronize()
    want = packed_image(pack(src_o, each_src))
    assert np.array_equal(host.numpy()[:64 * bb].reshape(64, 160, 16384), want)
    for i, b in enumerate(each_dst):
        one = dst.block_ids([b])
        _native.call("iekv_restore", dst.native.handle, one.data_ptr(), 1,
                     host.data_ptr() + i * bb, bb, None, 0, stream.cuda_stream,
                     stream.cuda_stream)
    stream.synchronize()
    for d, s in zip(each_dst, each_src):
        dst_o.write_block(d, src_o.read_block(s))
    assert_equal_pools(dk, dv, dst_o)
    del host
    gc.collect()
    assert release_pinned() >= n * bb


def test_the_drop_in_tier_path_at_the_70b_share_geometry(gpu):
    from iekv.engine.copier import HipSlotCopier
    from iekv.engine.pools import host_buffer, pinned_bytes_cached, release_pinned

    sk, sv = pool(gpu, 511)
    dk, dv = pool(gpu, 512)
    src = HipSlotCopier(sk, sv, BS, payload_location="host")
    dst = HipSlotCopier(dk, dv, BS)
    src_o, dst_o = oracle(sk, sv), oracle(dk, dv)
    rng = np.random.default_rng(513)
    k = 130
    src_ids = [int(b) for b in rng.permutation(BLOCKS)[:k]]
    dst_ids = [int(b) for b in rng.permutation(BLOCKS)[:k]]
    release_pinned()
    print(f"[cfg5-geometry] tier: {k} evictions, flushed every 64", flush=True)
    payloads = []
    for g in range(0, k, 64):
        payloads += [src.read_block(b) for b in src_ids[g:g + 64]]
        src.flush()
    # each payload lives in a buffer of its own, of exactly one block image
    roots = {id(p.packed._root): p.packed._root for p in payloads}
    assert len(roots) == k
    assert all(r.data.numel() == 2621440 for r in roots.values())
    assert src.offload_launches == 7          # 64 = 25 + 25 + 14, again, then 2
    for p, b in zip(payloads, src_ids):
        want = packed_image(pack(src_o, [b]))[0]
        assert np.array_equal(p.packed.host_data()[p.index].numpy(), want), b
    print("[cfg5-geometry] tier restore: scattered pinned payloads, 64 per call", flush=True)
    for g in range(0, k, 64):
        dst.write_blocks(dst_ids[g:g + 64], payloads[g:g + 64])
    torch.cuda.synchronize()
    for d, s in zip(dst_ids, src_ids):
        dst_o.write_block(d, src_o.read_block(s))
    assert_equal_pools(dk, dv, dst_o)
    # every transfer so far was direct: neither copier holds device staging
    assert src._staging is None and dst._staging is None

    print("[cfg5-geometry] the same payloads from pageable copies (staged)", flush=True)
    pageable = []
    for p in payloads:
        buf = host_buffer((1, 160, 16384), pinned=False)
        buf.copy_(p.packed.host_data())
        pageable.append(buf)
    again = [int(b) for b in rng.permutation(BLOCKS)[:k]]
    from iekv.engine.copier import PackedBlocks

    staged = [PackedBlocks(b, LAYERS, (BS, HEADS, DIM), torch.float8_e4m3fn)[0] for b in pageable]
    dst.write_blocks(again, staged)
    torch.cuda.synchronize()
    assert dst._staging is not None           # pageable images go through staging
    for d, s in zip(again, src_ids):
        dst_o.write_block(d, src_o.read_block(s))
    assert_equal_pools(dk, dv, dst_o)
    del payloads, roots, staged, pageable, p, buf     # the loops' last items hold buffers too
    gc.collect()
    torch.cuda.synchronize()
    from iekv.engine import copier as copier_module

    copier_module._release_finished()
    gc.collect()
    assert pinned_bytes_cached() == k * 2621440
    assert release_pinned() == k * 2621440
