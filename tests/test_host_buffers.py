"""Pinned host buffers pin exactly what they hold (CPU; the allocator is simulated).

torch's caching host allocator rounds every pinned request up to a power of two
and keeps the block after its tensor dies. A 2.5 MiB block image (the 70B-share
workload's) then pins 4 MiB, and the host round trip's 42.95 GB image 64 GiB.
The host tier's one-block buffers (iekv.engine.pools.host_buffer) and the
benchmark's round-trip image are instead taken at exactly their size from
iekv_host_alloc, and a buffer whose tensors are all gone is reused for the next
request of its size. Here iekv_host_alloc / iekv_host_free are replaced by
ctypes buffers, so the sizes requested and the reuse are observable without a
GPU.
"""
from __future__ import annotations

import ctypes
import gc

import pytest
import torch


@pytest.fixture
def fake_pinning(monkeypatch):
    """Record iekv_host_alloc / iekv_host_free calls and torch's pinned requests."""
    from iekv import _native
    from iekv.engine import pools

    log = {"alloc": [], "free": [], "torch_pinned": [], "buffers": {}}
    real_call = _native.call
    real_empty = torch.empty

    def call(name, *args):
        if name == "iekv_host_alloc":
            nbytes, out = args
            buf = ctypes.create_string_buffer(nbytes)
            log["buffers"][ctypes.addressof(buf)] = buf
            log["alloc"].append(nbytes)
            out._obj.value = ctypes.addressof(buf)
            return
        if name == "iekv_host_free":
            log["free"].append(args[0])
            return
        real_call(name, *args)

    def empty(*shape, **kw):
        if kw.pop("pin_memory", False):
            log["torch_pinned"].append(tuple(shape[0]) if len(shape) == 1 else shape)
        return real_empty(*shape, **kw)

    monkeypatch.setattr(_native, "call", call)
    monkeypatch.setattr(torch, "empty", empty)
    pools.release_pinned()
    yield log
    gc.collect()
    pools.release_pinned()


def test_a_block_image_that_is_not_a_power_of_two_pins_exactly_its_size(fake_pinning):
    from iekv.engine.pools import host_buffer

    cfg5_block = (1, 160, 16384)                 # 80 layers x K/V x 16 KiB = 2.5 MiB
    t = host_buffer(cfg5_block)
    assert tuple(t.shape) == cfg5_block and t.dtype == torch.uint8
    assert fake_pinning["alloc"] == [2621440]
    assert fake_pinning["torch_pinned"] == []    # not rounded up to 4 MiB by torch
    cfg3_block = (1, 64, 32768)                  # 2 MiB: torch's class is exact
    u = host_buffer(cfg3_block)
    assert tuple(u.shape) == cfg3_block
    assert fake_pinning["torch_pinned"] == [cfg3_block] and fake_pinning["alloc"] == [2621440]
    pageable = host_buffer(cfg5_block, pinned=False)
    assert tuple(pageable.shape) == cfg5_block and fake_pinning["alloc"] == [2621440]


def test_a_dead_buffer_is_reused_then_released(fake_pinning):
    from iekv.engine.pools import pinned_bytes_cached, pinned_empty, release_pinned

    a = pinned_empty(3 << 20 | 4096)
    ptr = a.data_ptr()
    view = a[4096:].view(torch.int32)      # a view keeps the memory from reuse
    del a
    gc.collect()
    assert pinned_bytes_cached() == 0
    b = pinned_empty(3 << 20 | 4096)
    assert b.data_ptr() != ptr             # the live view's memory was not handed out
    del view
    gc.collect()
    assert pinned_bytes_cached() == (3 << 20 | 4096)
    c = pinned_empty(3 << 20 | 4096)
    assert c.data_ptr() == ptr             # now it is reused, with no new allocation
    assert fake_pinning["alloc"] == [3 << 20 | 4096] * 2
    d = pinned_empty(4 << 20 | 4096)      # another size takes its own buffer
    assert d.data_ptr() not in (ptr, b.data_ptr())
    del b, c, d
    gc.collect()
    assert release_pinned() == 2 * (3 << 20 | 4096) + (4 << 20 | 4096)
    assert sorted(fake_pinning["free"]) == sorted(fake_pinning["buffers"])
    assert pinned_bytes_cached() == 0
    with pytest.raises(ValueError):
        pinned_empty(0)


def test_the_round_trip_leg_pins_exactly_its_image_and_checks_the_host():
    """The host round trip of the 70B-share workload pins its 42.95 GB image at
    exactly that size (torch would pin 64 GiB) and refuses to start, with a clear
    error, on a host that cannot hold it."""
    import bench
    from iekv import workloads

    w = workloads.make("cfg5", 0, None)
    plan = bench.host_roundtrip_plan(w, 1024)
    assert plan["image_bytes"] == w.payload_bytes == 16384 * 2621440
    assert plan["tier_bytes"] == (1024 + 128) * 2621440
    assert plan["peak_pinned_bytes"] == w.payload_bytes < 1 << 36
    bench.check_host_budget(plan, None)
    bench.check_host_budget(plan, 270 << 30)
    with pytest.raises(RuntimeError, match="host_roundtrip needs 51.5 GB of host memory"):
        bench.check_host_budget(plan, 40 << 30)
    budget = bench.host_memory_budget()
    assert budget is None or budget > 0


def test_held_pinned_buffers_survive_pruning_reentry_and_threads():
    """Buffers whose copy still runs are held until their event completes. Pruning
    must lose none of them: not one added from inside the pruning itself (a payload
    dying in a garbage collection there, in the same thread, which must not
    deadlock either), nor ones added by other threads while it runs. Stand-in events
    whose query() answers from a flag play the copies."""
    import threading

    import torch

    from iekv.engine import copier

    class Copy:
        def __init__(self, done=False, on_query=None):
            self.done, self.on_query = done, on_query

        def query(self):
            if self.on_query is not None:
                hook, self.on_query = self.on_query, None
                hook()
            return self.done

    data = torch.zeros(1)
    copier._release_finished()
    saved = list(copier._UNFINISHED)
    copier._UNFINISHED.clear()
    try:
        late = Copy()
        copier._hold_until_done(data, Copy(done=True))
        copier._hold_until_done(data, Copy(on_query=lambda: copier._hold_until_done(data, late)))
        copier._release_finished()
        events = [e for _, e in copier._UNFINISHED]
        assert late in events and len(events) == 2       # the finished one went, none lost
        running = [Copy() for _ in range(400)]
        start = threading.Barrier(5)

        def add(chunk):
            start.wait()
            for ev in chunk:
                copier._hold_until_done(data, ev)

        def prune():
            start.wait()
            for _ in range(200):
                copier._release_finished()

        threads = [threading.Thread(target=add, args=(running[i::4],)) for i in range(4)]
        threads.append(threading.Thread(target=prune))
        for th in threads:
            th.start()
        for th in threads:
            th.join(timeout=60)
        assert not any(th.is_alive() for th in threads)
        held = {id(e) for _, e in copier._UNFINISHED}
        assert all(id(ev) in held for ev in running)
        for _, ev in copier._UNFINISHED:
            ev.done = True
        copier._release_finished()
        assert copier._UNFINISHED == []
    finally:
        copier._UNFINISHED[:] = saved
