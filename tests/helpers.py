"""Helpers shared by the tests (not a test module)."""
from __future__ import annotations

import numpy as np

from oracle.copier import LayeredSlotCopier


def numpy_view(tensor):
    """A NumPy view of a CPU torch tensor's memory (bf16 and fp8 as raw integer views)."""
    import torch

    if tensor.dtype == torch.bfloat16:
        return tensor.view(torch.int16).numpy()
    if tensor.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        return tensor.view(torch.uint8).numpy()
    return tensor.numpy()


def oracle_factory(k_caches, v_caches, block_size, role):
    """Engine copier factory that moves bytes with the NumPy oracle (CPU pools only)."""
    return LayeredSlotCopier([numpy_view(t) for t in k_caches],
                             [numpy_view(t) for t in v_caches], block_size)


class StringCopier:
    """A copier whose blocks hold strings: the block manager's offload wiring is
    exercised without any KV bytes. An unwritten block reads as "block-<id>";
    ``calls`` logs every protocol call as (op, block id)."""

    def __init__(self):
        self.store: dict[int, str] = {}
        self.calls: list[tuple[str, int]] = []

    def read_block(self, block_id):
        self.calls.append(("read", block_id))
        return self.store.get(block_id, f"block-{block_id}")

    def write_block(self, block_id, payload):
        self.calls.append(("write", block_id))
        self.store[block_id] = payload


class LoggingCopier:
    """Wraps a copier and logs ["r"|"w", block_id] for every protocol call.

    It offers only the reference's protocol (read_block / write_block), not the
    HIP copier's batched calls, so callers take their per-block paths and the
    log is the reference's call trace.
    """

    BATCHED = ("read_blocks", "write_blocks", "copy_blocks")

    def __init__(self, inner, log):
        self.inner = inner
        self.log = log

    def read_block(self, block_id):
        self.log.append(["r", int(block_id)])
        return self.inner.read_block(block_id)

    def write_block(self, block_id, payload):
        self.log.append(["w", int(block_id)])
        return self.inner.write_block(block_id, payload)

    def __getattr__(self, name):
        if name in self.BATCHED:
            raise AttributeError(name)
        return getattr(self.inner, name)


def cfg1_inputs():
    """The cfg1 recipe of tests/golden/make_golden.py, restated: lengths, src tables, fill."""
    layers, heads, dim, bs, pool_blocks, seqs = 4, 4, 32, 16, 4096, 64
    rng = np.random.default_rng(0)
    lengths = rng.integers(16, 512, size=seqs, endpoint=True)
    counts = [-(-int(n) // bs) for n in lengths]
    perm = rng.permutation(pool_blocks)
    tables, at = [], 0
    for c in counts:
        tables.append([int(b) for b in perm[at:at + c]])
        at += c
    fill = np.random.default_rng(1)
    shape = (pool_blocks * bs, heads, dim)
    k = [fill.standard_normal(shape, dtype=np.float32) for _ in range(layers)]
    v = [fill.standard_normal(shape, dtype=np.float32) for _ in range(layers)]
    return [int(n) for n in lengths], tables, k, v


class DirectOracleCopier(LayeredSlotCopier):
    """Oracle copier with the direct pool-to-pool call (a read then a write per block)."""

    def copy_blocks(self, source, src_ids, dst_ids):
        for s, d in zip(src_ids, dst_ids):
            self.write_block(int(d), source.read_block(int(s)))


def direct_oracle_factory(k_caches, v_caches, block_size, role):
    return DirectOracleCopier([numpy_view(t) for t in k_caches],
                              [numpy_view(t) for t in v_caches], block_size)
