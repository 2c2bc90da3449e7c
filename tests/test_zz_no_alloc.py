"""The allocation-free offload (iekv_offload_static) against iekv_offload (GPU).

iekv_offload_static runs the offload kernels with the library's own static
device staging buffer instead of a caller-allocated one. Called through the
C-ABI twice in a row, the second time with fewer blocks, it must write the
same host image, byte for byte, as iekv_offload with a staging buffer from
torch, and both must equal the pool's tiles gathered by torch indexing.
Calls on unrelated stream pairs, with no host synchronisation between them,
and calls from two host threads at once share the one buffer without
overwriting a slot another call still copies from.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SENTINEL = 0xA5


def random_pool(num_blocks, bs, layers, heads, dim, device, seed):
    from iekv.engine.pools import allocate_pool

    k, v = allocate_pool(num_blocks, bs, layers, heads, dim, dtype=torch.bfloat16,
                         device=device, zero=False)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    slab = k[0]._base if k[0]._base is not None else k[0]
    raw = slab.view(torch.uint8)
    raw.copy_(torch.randint(0, 256, raw.shape, dtype=torch.uint8, device=device, generator=gen))
    return k, v


def expected_image(k, v, ids, tile_bytes):
    """Block-major [n, 2L, T] image of blocks ``ids``, gathered by torch indexing."""
    index = torch.as_tensor(ids, dtype=torch.long, device=k[0].device)
    tiles = [a.view(torch.uint8).reshape(-1, tile_bytes).index_select(0, index)
             for a in list(k) + list(v)]
    return torch.stack(tiles, dim=1).cpu().numpy()


def host_buffer(n, n_arrays, tile_bytes, pinned):
    buf = torch.empty((n, n_arrays, tile_bytes), dtype=torch.uint8, pin_memory=pinned)
    buf.fill_(SENTINEL)
    return buf


# (block_size, layers, heads, head_dim): 1 MiB block images (16 per staging slot),
# and 20 MiB images (one staging slot of the 32 MiB buffer).
SHAPES = {"1MiB-images": (16, 4, 8, 128), "20MiB-images": (256, 20, 8, 128)}
# Blocks per call: the second call of each pair moves fewer blocks than the first.
CALLS = {"1MiB-images": (90, 7), "20MiB-images": (5, 2)}


@pytest.mark.parametrize("pinned", [True, False], ids=["pinned", "pageable"])
@pytest.mark.parametrize("shape", list(SHAPES))
def test_static_offload_writes_what_the_staged_offload_writes(gpu, shape, pinned):
    from iekv import _native
    from iekv.engine.pools import KVPool

    bs, layers, heads, dim = SHAPES[shape]
    num_blocks = 120 if shape == "1MiB-images" else 12
    k, v = random_pool(num_blocks, bs, layers, heads, dim, gpu, seed=91)
    pool = KVPool(k, v, bs)
    block = pool.block_bytes
    assert block <= _native.STATIC_STAGING
    staging = torch.empty(4 * block, dtype=torch.uint8, device=gpu)
    stream, side = torch.cuda.current_stream(), torch.cuda.Stream()
    rng = np.random.default_rng(92)
    for n in CALLS[shape]:
        ids = [int(b) for b in rng.permutation(num_blocks)[:n]]
        dev_ids = pool.block_ids(ids)
        print(f"[no-alloc] {shape} pinned={pinned} blocks={n}", flush=True)
        ref = host_buffer(n, pool.n_arrays, pool.tile_bytes, pinned)
        got = host_buffer(n, pool.n_arrays, pool.tile_bytes, pinned)
        _native.call("iekv_offload", pool.native.handle, dev_ids.data_ptr(), n, ref.data_ptr(),
                     ref.numel(), staging.data_ptr(), staging.numel(), stream.cuda_stream,
                     side.cuda_stream)
        _native.call("iekv_offload_static", pool.native.handle, dev_ids.data_ptr(), n,
                     got.data_ptr(), got.numel(), stream.cuda_stream, side.cuda_stream)
        stream.synchronize()       # `compute` is ordered after every device-to-host copy
        want = expected_image(k, v, ids, pool.tile_bytes)
        assert np.array_equal(ref.numpy(), want)
        assert np.array_equal(got.numpy(), ref.numpy())


def test_static_offload_of_nothing_enqueues_nothing(gpu):
    from iekv import _native
    from iekv.engine.pools import KVPool

    k, v = random_pool(8, 16, 2, 2, 64, gpu, seed=93)
    pool = KVPool(k, v, 16)
    host = torch.empty(1, dtype=torch.uint8)
    stream = torch.cuda.current_stream()
    _native.call("iekv_offload_static", pool.native.handle, None, 0, host.data_ptr(), 0,
                 stream.cuda_stream, stream.cuda_stream)


def staged_case(gpu, seed):
    """A pool of 1 MiB block images (32 arrays of 32 KiB tiles). Offloads into
    pageable memory go through the static buffer's two 16 MiB slots (pinned images
    are written by the pack kernel itself and use no staging)."""
    from iekv.engine.pools import KVPool

    k, v = random_pool(400, 16, 16, 8, 128, gpu, seed=seed)
    pool = KVPool(k, v, 16)
    assert pool.block_bytes == 1 << 20
    return k, v, pool


def test_static_offloads_on_unrelated_streams_wait_for_each_other(gpu):
    from iekv import _native

    k, v, pool = staged_case(gpu, 94)
    rng = np.random.default_rng(95)
    pairs = [(torch.cuda.Stream(), torch.cuda.Stream()) for _ in range(3)]
    calls = []
    for n, (compute, copy) in zip((150, 100, 70), pairs):
        ids = [int(b) for b in rng.permutation(400)[:n]]
        dev_ids = pool.block_ids(ids)
        torch.cuda.current_stream().synchronize()      # the ids are on the device
        host = host_buffer(n, pool.n_arrays, pool.tile_bytes, False)
        calls.append((ids, dev_ids, host, compute))
    print("[no-alloc] three staged calls on three stream pairs, no host sync", flush=True)
    for (ids, dev_ids, host, compute), (_, copy) in zip(calls, pairs):
        _native.call("iekv_offload_static", pool.native.handle, dev_ids.data_ptr(), len(ids),
                     host.data_ptr(), host.numel(), compute.cuda_stream, copy.cuda_stream)
    for ids, _, host, compute in calls:
        compute.synchronize()
        assert np.array_equal(host.numpy(), expected_image(k, v, ids, pool.tile_bytes))


def test_static_offloads_from_two_threads_share_the_buffer(gpu):
    from iekv import _native

    k, v, pool = staged_case(gpu, 96)
    rng = np.random.default_rng(97)
    plans = []
    for t in range(2):
        compute, copy = torch.cuda.Stream(), torch.cuda.Stream()
        jobs = []
        for n in (90, 120, 66):
            ids = [int(b) for b in rng.permutation(400)[:n]]
            jobs.append((ids, pool.block_ids(ids),
                         host_buffer(n, pool.n_arrays, pool.tile_bytes, False)))
        plans.append((compute, copy, jobs))
    torch.cuda.synchronize()
    errors = []

    def run(compute, copy, jobs):
        try:
            for ids, dev_ids, host in jobs:
                _native.call("iekv_offload_static", pool.native.handle, dev_ids.data_ptr(),
                             len(ids), host.data_ptr(), host.numel(), compute.cuda_stream,
                             copy.cuda_stream)
        except Exception as e:          # reported below, in the test's thread
            errors.append(e)

    print("[no-alloc] two threads, three staged calls each", flush=True)
    threads = [threading.Thread(target=run, args=plan) for plan in plans]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors and not any(t.is_alive() for t in threads)
    torch.cuda.synchronize()
    for _, _, jobs in plans:
        for ids, _, host in jobs:
            assert np.array_equal(host.numpy(), expected_image(k, v, ids, pool.tile_bytes))
