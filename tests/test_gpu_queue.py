"""The resident request queue (iekv_queue_*, iekv.engine.queue) on the GPU, byte for byte
against the NumPy oracle.

A queue serves the reference's one-request-at-a-time handoffs
(ie/serve/disaggregated.py:106-116, each request a disaggregated.py:50 read and a
:81-82 write) without a kernel launch per request. Each test ends its queue
(stop or close) before reading pools with torch, and waits on streams, never on
the whole device: a device synchronize would wait for the resident kernel.
"""
from __future__ import annotations

import threading
import time

import numpy as np
import pytest
import torch

from oracle.copier import handoff
from test_gpu_kernels import allocate, assert_pool_equals, oracle_of

pytestmark = pytest.mark.gpu


def pools(gpu, n_src, n_dst, bs, layers, heads, dim, dtype, seed):
    from iekv.engine.pools import KVPool

    sk, sv = allocate(n_src, bs, layers, heads, dim, dtype, gpu, seed=seed)
    dk, dv = allocate(n_dst, bs, layers, heads, dim, dtype, gpu, seed=seed + 1)
    torch.cuda.current_stream().synchronize()
    return (sk, sv, KVPool(sk, sv, bs)), (dk, dv, KVPool(dk, dv, bs))


def requests(rng, n_src, n_dst, n_requests, longest):
    """Random requests whose destinations are distinct across all of them."""
    dst_order = rng.permutation(n_dst)
    src, dst, at = [], [], 0
    for _ in range(n_requests):
        n = int(rng.integers(1, longest + 1))
        if at + n > n_dst:
            break
        src.append([int(b) for b in rng.integers(0, n_src, n)])
        dst.append([int(b) for b in dst_order[at:at + n]])
        at += n
    return src, dst


# (block_size, layers, kv_heads, head_dim, dtype): 4 KiB tiles (16-byte vectors, one
# per lane), 64 KiB tiles (several steps per lane), 64-byte tiles grouped per unit,
# 24-byte tiles (8-byte vectors, ungrouped), 3-byte tiles (single bytes).
SHAPES = [(16, 2, 2, 64, torch.bfloat16), (256, 2, 2, 32, torch.float32),
          (4, 3, 1, 8, torch.float16), (3, 2, 1, 4, torch.float16),
          (3, 2, 1, 1, torch.uint8)]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"bs{s[0]}L{s[1]}H{s[2]}D{s[3]}{s[4]}")
def test_queued_requests_match_the_oracle(gpu, shape):
    from iekv.engine.queue import HandoffQueue

    bs, layers, heads, dim, dtype = shape
    (sk, sv, src), (dk, dv, dst) = pools(gpu, 96, 160, bs, layers, heads, dim, dtype, seed=11)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(12)
    src_tables, dst_tables = requests(rng, 96, 160, 40, 9)
    with HandoffQueue(src, dst) as q:
        tickets = [q.submit(s, d) for s, d in zip(src_tables, dst_tables)]
        assert tickets == sorted(tickets) and len(set(tickets)) == len(tickets)
        q.wait(tickets[-1])
        assert all(q.done(t) for t in tickets)
        q.stop()
    handoff(src_o, dst_o, src_tables, dst_tables)
    assert_pool_equals(dk, dv, dst_o)
    assert_pool_equals(sk, sv, src_o)


def test_slots_are_reused_and_long_requests_split(gpu):
    """More requests than ring slots (a submission then waits for a slot), and one
    request longer than a descriptor holds (split into three)."""
    from iekv import _native
    from iekv.engine.queue import HandoffQueue

    bs, layers, heads, dim = 2, 2, 1, 8
    (sk, sv, src), (dk, dv, dst) = pools(gpu, 512, 4096, bs, layers, heads, dim,
                                         torch.float16, seed=21)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(22)
    order = rng.permutation(4096)
    n_small = _native.QUEUE_SLOTS + 300
    src_tables = [[int(rng.integers(0, 512))] for _ in range(n_small)]
    dst_tables = [[int(order[i])] for i in range(n_small)]
    long_n = 2 * _native.QUEUE_MAX_BLOCKS + 100
    src_tables.append([int(b) for b in rng.integers(0, 512, long_n)])
    dst_tables.append([int(b) for b in order[n_small:n_small + long_n]])
    with HandoffQueue(src, dst) as q:
        first = q.stats()["descriptors"]
        tickets = [q.submit(s, d) for s, d in zip(src_tables, dst_tables)]
        q.wait()
        assert tickets[-1] - tickets[-2] == 3      # the long request took three descriptors
        assert q.stats()["descriptors"] - first == n_small + 3
        q.stop()
    handoff(src_o, dst_o, src_tables, dst_tables)
    assert_pool_equals(dk, dv, dst_o)


def test_requests_submitted_together_match_the_oracle(gpu):
    """iekv_queue_submit_requests: one call, one ticket per request, an empty request
    among them (its ticket is DONE)."""
    from iekv.engine.queue import DONE, HandoffQueue

    bs, layers, heads, dim = 16, 2, 2, 32
    (sk, sv, src), (dk, dv, dst) = pools(gpu, 64, 200, bs, layers, heads, dim,
                                         torch.bfloat16, seed=31)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(32)
    src_tables, dst_tables = requests(rng, 64, 200, 30, 12)
    src_tables.insert(5, [])
    dst_tables.insert(5, [])
    counts = [len(s) for s in src_tables]
    with HandoffQueue(src, dst) as q:
        tickets = q.submit_requests(counts, np.array(sum(src_tables, []), np.int32),
                                    np.array(sum(dst_tables, []), np.int32))
        assert tickets[5] == DONE
        issued = [t for t in tickets if t != DONE]
        assert issued == sorted(issued) and len(issued) == len(tickets) - 1
        q.wait()
        q.stop()
    handoff(src_o, dst_o, src_tables, dst_tables)
    assert_pool_equals(dk, dv, dst_o)


def test_a_source_rewritten_between_requests_is_read_anew(gpu):
    """The kernel stays resident across requests, so a request must read what the
    source blocks hold when it is submitted, not what an earlier request of the same
    kernel read; and a destination rewritten by a request is read back by torch."""
    from iekv.engine.queue import HandoffQueue

    bs, layers, heads, dim = 16, 2, 2, 64
    (sk, sv, src), (dk, dv, dst) = pools(gpu, 16, 16, bs, layers, heads, dim,
                                         torch.bfloat16, seed=41)
    arrays_s, arrays_d = sk + sv, dk + dv

    def tile(a, block):
        return a.view(-1, bs * heads * dim)[block]

    gen = torch.Generator(device=gpu)
    gen.manual_seed(42)
    with HandoffQueue(src, dst) as q:
        for round_ in range(6):
            q.wait(q.submit([3, 5], [round_, 8 + round_]))
            want = [tile(a, 3).clone() for a in arrays_s]
            got = [tile(a, round_) for a in arrays_d]
            assert all(torch.equal(g.view(torch.uint8), w.view(torch.uint8))
                       for g, w in zip(got, want)), round_
            for a in arrays_s:   # new bytes in block 3 before the next request
                t = tile(a, 3)
                t.copy_(torch.randn(t.shape, generator=gen, device=gpu).to(a.dtype))
            torch.cuda.current_stream().synchronize()
        q.stop()


def test_the_kernel_is_restarted_near_its_limits_and_after_stop(gpu):
    """A submission more than half the idle limit after the previous one, or after a
    stop, or after the kernel ended by itself, starts a new kernel; every request
    is served."""
    from iekv.engine.queue import HandoffQueue

    bs, layers, heads, dim = 16, 2, 1, 32
    (sk, sv, src), (dk, dv, dst) = pools(gpu, 32, 64, bs, layers, heads, dim,
                                         torch.float16, seed=51)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(52)
    src_tables, dst_tables = requests(rng, 32, 64, 12, 4)
    with HandoffQueue(src, dst, idle_ms=100) as q:
        assert q.stats()["launches"] == 0
        for i, (s, d) in enumerate(zip(src_tables, dst_tables)):
            q.wait(q.submit(s, d))
            if i == 3:
                time.sleep(0.06)    # past half the idle limit: restarted
            elif i == 6:
                q.stop()            # stopped: restarted
            elif i == 9:
                time.sleep(0.25)    # past the idle limit: the kernel has ended
        # (a host pause of over 50 ms elsewhere would add a restart, never lose one)
        assert q.stats()["launches"] >= 4
        q.stop()
    handoff(src_o, dst_o, src_tables, dst_tables)
    assert_pool_equals(dk, dv, dst_o)


def test_bad_requests_are_refused_before_anything_is_submitted(gpu):
    from iekv import _native
    from iekv.engine.queue import DONE, HandoffQueue

    (sk, sv, src), (dk, dv, dst) = pools(gpu, 16, 16, 4, 1, 1, 8, torch.float16, seed=61)
    before = [t.clone() for t in dk + dv]
    with HandoffQueue(src, dst) as q:
        with pytest.raises(IndexError):
            q.submit([0, 16], [1, 2])              # source id out of range
        with pytest.raises(IndexError):
            q.submit([0, 1], [-1, 2])              # destination id out of range
        with pytest.raises(ValueError):
            q.submit([0, 1], [3, 3])               # a destination twice
        with pytest.raises(ValueError):
            q.submit([0, 1], [3])                  # lengths differ
        with pytest.raises(TypeError):
            q.submit([0.5], [1])                   # not integers
        with pytest.raises(IndexError):
            q.submit_requests([1, 1], np.array([0, 99], np.int32), np.array([1, 2], np.int32))
        assert q.stats() == {"descriptors": 0, "launches": 0}
        assert q.submit([], []) == DONE
        q.wait(DONE)
        assert q.done(DONE)
        with pytest.raises(_native.NativeError):
            q.wait(0)                              # not issued
        with pytest.raises(_native.NativeError):
            q.done(5)
    assert all(torch.equal(a.view(torch.uint8), b.view(torch.uint8))
               for a, b in zip(before, dk + dv))


def test_a_queue_within_one_pool(gpu):
    """Source and destination the same pool (disjoint blocks), as a move within one
    engine's cache would be; a block that is both source and destination is refused."""
    from iekv.engine.queue import HandoffQueue

    bs, layers, heads, dim = 16, 2, 2, 16
    (sk, sv, pool), _ = pools(gpu, 64, 4, bs, layers, heads, dim, torch.bfloat16, seed=71)
    want = oracle_of(sk, sv, bs)
    with HandoffQueue(pool, pool) as q:
        with pytest.raises(ValueError):
            q.submit([1, 2], [2, 9])
        q.wait(q.submit([1, 2, 3], [40, 41, 42]))
        q.wait(q.submit([10, 11], [50, 60]))
        q.stop()
    handoff(want, want, [[1, 2, 3], [10, 11]], [[40, 41, 42], [50, 60]])
    assert_pool_equals(sk, sv, want)


def test_two_threads_submit_to_one_queue(gpu):
    from iekv.engine.queue import HandoffQueue

    bs, layers, heads, dim = 16, 2, 2, 32
    (sk, sv, src), (dk, dv, dst) = pools(gpu, 64, 256, bs, layers, heads, dim,
                                         torch.bfloat16, seed=81)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(82)
    src_tables, dst_tables = requests(rng, 64, 256, 60, 6)
    errors = []
    with HandoffQueue(src, dst) as q:
        def run(part):
            try:
                for s, d in list(zip(src_tables, dst_tables))[part::2]:
                    q.wait(q.submit(s, d))
            except Exception as err:   # reported below
                errors.append(err)

        threads = [threading.Thread(target=run, args=(p,)) for p in (0, 1)]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=60)
        assert not any(t.is_alive() for t in threads)
        q.stop()
    assert not errors, errors
    handoff(src_o, dst_o, src_tables, dst_tables)
    assert_pool_equals(dk, dv, dst_o)


def test_a_zero_timeout_raises_or_returns_and_the_request_still_completes(gpu):
    from iekv import _native
    from iekv.engine.queue import HandoffQueue

    bs, layers, heads, dim = 16, 4, 8, 128
    (sk, sv, src), (dk, dv, dst) = pools(gpu, 600, 600, bs, layers, heads, dim,
                                         torch.bfloat16, seed=91)
    src_o, dst_o = oracle_of(sk, sv, bs), oracle_of(dk, dv, bs)
    rng = np.random.default_rng(92)
    s = [int(b) for b in rng.permutation(600)[:512]]
    d = [int(b) for b in rng.permutation(600)[:512]]
    with HandoffQueue(src, dst) as q:
        t = q.submit(s, d)
        try:
            q.wait(t, timeout=0)
        except _native.NativeTimeoutError:
            pass
        q.wait(t, timeout=30)
        q.stop()
    handoff(src_o, dst_o, [s], [d])
    assert_pool_equals(dk, dv, dst_o)
