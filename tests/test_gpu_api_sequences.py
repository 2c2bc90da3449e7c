"""Random sequences of the drop-in copier's calls (GPU) against the NumPy oracle.

Two pools, A (prefill side) and B (decode side), of a random shape and cache
dtype hold random bytes; the oracle holds their NumPy images. Each seed makes
28 calls drawn at random from the HipSlotCopier surface and applies the same
moves, in the same order, to the oracle:
  - copy_blocks between the pools and within one (disjoint blocks);
  - read_blocks into device payloads and write_blocks of them elsewhere, in
    order, permuted (one block per call) or a slice;
  - host offloads (read_blocks / read_block on a host copier, deferred or not),
    kept as a tier, and restores that mix payloads of several offloads;
  - copy_requests over two streams;
  - single-block read_block / write_block protocol calls.
Ids come as Python lists, tuples, NumPy arrays, CPU tensors or device tensors;
some calls (host offloads and restores included) run on a side stream, ordered
after and before the current stream as a caller must. Reads are snapshots at call time: deferred host reads are
flushed before anything writes their pool, as the engine does. At the end both
pools equal their images byte for byte.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.copier import LayeredSlotCopier

pytestmark = pytest.mark.gpu


def _pool(n_blocks, bs, layers, heads, dim, dtype, gpu, gen):
    from iekv.engine.pools import allocate_pool

    k, v = allocate_pool(n_blocks, bs, layers, heads, dim, dtype=dtype, device=gpu, zero=False)
    slab = k[0]._base if k[0]._base is not None else k[0]
    raw = slab.view(torch.uint8)
    raw.copy_(torch.randint(0, 256, raw.shape, dtype=torch.uint8, device=gpu, generator=gen))
    return k, v


def _image(k, v, bs):
    rows = lambda t: t.contiguous().view(torch.uint8).reshape(t.shape[0], -1).cpu().numpy().copy()
    return LayeredSlotCopier([rows(t) for t in k], [rows(t) for t in v], bs)


def _ids(rng, ids, gpu):
    """The same ids in one of the forms callers pass."""
    form = int(rng.integers(5))
    if form == 0:
        return list(ids)
    if form == 1:
        return tuple(ids)
    if form == 2:
        return np.asarray(ids, dtype=np.int64)
    if form == 3:
        return torch.tensor(ids, dtype=torch.int64)
    return torch.tensor(ids, dtype=torch.int32, device=gpu)


@pytest.mark.parametrize("seed", range(40))
def test_random_call_sequences_match_the_oracle(gpu, seed):
    from iekv.engine.copier import HipSlotCopier

    rng = np.random.default_rng(1000 + seed)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(seed)
    bs = int(rng.choice([1, 2, 8, 16]))
    layers, heads = int(rng.integers(1, 4)), int(rng.integers(1, 5))
    dim = int(rng.choice([4, 8, 16, 32, 64]))
    dtype = [torch.float32, torch.bfloat16, torch.uint8][int(rng.integers(3))]
    n_a, n_b = int(rng.integers(64, 200)), int(rng.integers(64, 200))
    ka, va = _pool(n_a, bs, layers, heads, dim, dtype, gpu, gen)
    kb, vb = _pool(n_b, bs, layers, heads, dim, dtype, gpu, gen)
    print(f"seed {seed}: bs {bs} L{layers} H{heads} D{dim} {dtype} pools {n_a}/{n_b}",
          flush=True)
    oracle = {"A": _image(ka, va, bs), "B": _image(kb, vb, bs)}
    blocks = {"A": n_a, "B": n_b}
    dev = {"A": HipSlotCopier(ka, va, bs), "B": HipSlotCopier(kb, vb, bs)}
    caches = {"A": (ka, va), "B": (kb, vb)}
    host = {p: HipSlotCopier(caches[p][0], caches[p][1], bs, payload_location="host",
                             defer_reads=bool(rng.integers(2))) for p in "AB"}
    side = torch.cuda.Stream(gpu)
    tier: list = []                      # (host payload, oracle payload)

    def before_write(pool):
        host[pool].flush()               # queued reads of this pool snapshot it first

    def pick(pool, n, avoid=()):
        free = [b for b in rng.permutation(blocks[pool]) if b not in set(avoid)]
        return [int(b) for b in free[:n]]

    def run(fn):
        """On the current stream or on the side stream, ordered as a caller must."""
        if rng.integers(3):
            return fn(None)
        side.wait_stream(torch.cuda.current_stream(gpu))
        out = fn(side)
        torch.cuda.current_stream(gpu).wait_stream(side)
        return out

    ops = ["copy", "copy_same", "pack_unpack", "offload", "restore", "requests", "single"]
    for step in range(28):
        op = ops[int(rng.integers(len(ops)))]
        x, y = ("A", "B") if rng.integers(2) else ("B", "A")
        n = int(rng.integers(0, 9)) if rng.integers(4) else int(rng.integers(9, 60))
        n = min(n, blocks[x] // 2, blocks[y] // 2)
        if op == "copy":
            s, d = pick(x, n), pick(y, n)
            before_write(y)
            run(lambda st: dev[y].copy_blocks(dev[x], _ids(rng, s, gpu), _ids(rng, d, gpu),
                                              stream=st))
            payloads = [oracle[x].read_block(b) for b in s]
            for b, p in zip(d, payloads):
                oracle[y].write_block(b, p)
        elif op == "copy_same":
            s = pick(x, n)
            d = pick(x, n, avoid=s)
            before_write(x)
            run(lambda st: dev[x].copy_blocks(dev[x], _ids(rng, s, gpu), _ids(rng, d, gpu),
                                              stream=st))
            payloads = [oracle[x].read_block(b) for b in s]
            for b, p in zip(d, payloads):
                oracle[x].write_block(b, p)
        elif op == "pack_unpack":
            s, d = pick(x, n), pick(y, n)
            packed = run(lambda st: dev[x].read_blocks(_ids(rng, s, gpu), stream=st))
            want = [oracle[x].read_block(b) for b in s]
            how = int(rng.integers(3))
            if how == 1 and n > 1:               # permuted: one block per call
                perm = [int(i) for i in rng.permutation(n)]
                payloads, want = [packed[i] for i in perm], [want[i] for i in perm]
            elif how == 2 and n > 2:              # a slice of the packed payloads
                payloads, want, d = packed[1:], want[1:], d[1:]
            else:
                payloads = packed
            before_write(y)
            run(lambda st: dev[y].write_blocks(_ids(rng, d, gpu), payloads, stream=st))
            for b, p in zip(d, want):
                oracle[y].write_block(b, p)
        elif op == "offload":
            s = pick(x, max(n, 1))
            if rng.integers(2):
                payloads = list(run(lambda st: host[x].read_blocks(_ids(rng, s, gpu), stream=st)))
            else:
                payloads = [host[x].read_block(b) for b in s]
            tier.extend(zip(payloads, [oracle[x].read_block(b) for b in s]))
        elif op == "restore" and tier:
            k = min(len(tier), max(n, 1))
            chosen = [tier[int(i)] for i in rng.choice(len(tier), size=k, replace=False)]
            d = pick(y, k)
            before_write(y)
            # Host payloads carry their offload's event: a restore on any stream
            # waits for it (run() still orders the pool writes for the caller).
            run(lambda st: dev[y].write_blocks(_ids(rng, d, gpu), [h for h, _ in chosen],
                                               stream=st))
            for b, (_, p) in zip(d, chosen):
                oracle[y].write_block(b, p)
        elif op == "requests":
            reqs = []
            used_s, used_d = [], []
            for _ in range(int(rng.integers(1, 5))):
                m = int(rng.integers(0, 6))
                s = pick(x, m, avoid=used_s)[:m]
                d = pick(y, m, avoid=used_d)[:m]
                m = min(len(s), len(d))
                reqs.append((s[:m], d[:m]))
                used_s += s[:m]
                used_d += d[:m]
            before_write(y)
            dev[y].copy_requests(dev[x], reqs, streams=[torch.cuda.current_stream(gpu), side])
            torch.cuda.current_stream(gpu).wait_stream(side)
            payloads = [[oracle[x].read_block(b) for b in s] for s, _ in reqs]
            for (_, d), ps in zip(reqs, payloads):
                for b, p in zip(d, ps):
                    oracle[y].write_block(b, p)
        elif op == "single":
            b, c = pick(x, 1)[0], pick(y, 1)[0]
            payload = dev[x].read_block(b)
            before_write(y)
            dev[y].write_block(c, payload)
            oracle[y].write_block(c, oracle[x].read_block(b))
    torch.cuda.synchronize()
    for pool, (k, v) in (("A", (ka, va)), ("B", (kb, vb))):
        got = _image(k, v, bs)
        for a, (g, w) in enumerate(zip(list(got.k_caches) + list(got.v_caches),
                                       list(oracle[pool].k_caches) + list(oracle[pool].v_caches))):
            if not np.array_equal(g, w):
                rows = np.nonzero((g != w).any(axis=1))[0]
                raise AssertionError(f"seed {seed} pool {pool} array {a}: {rows.size} rows "
                                     f"differ, first at row {rows[0]}")
