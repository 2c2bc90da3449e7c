"""NumPy restatement of slot-level KV access — TEST INFRASTRUCTURE ONLY.

``write_kv`` scatters rows into a ``[N*bs, H, D]`` cache by slot
(ie/kernels/reference.py:45-51); ``gather_context`` reads a sequence's context
back through its block table (ie/kernels/reference.py:54-63). Both are pinned by
the reference's own known-answer tests (tests/test_paged_attention.py:54-70:
gather slots [12,13,14,15,4,5] for table [3,1], bs 4, context 6; writes to
slots [9,0,5]), re-run in tests/test_oracle.py.
"""
from __future__ import annotations

import numpy as np


def write_kv(k: np.ndarray, v: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
             slot_mapping) -> None:
    if len(slot_mapping) != k.shape[0]:
        raise ValueError(f"{len(slot_mapping)} slots for {k.shape[0]} tokens")
    rows = np.asarray(slot_mapping, dtype=np.int64)
    k_cache[rows] = k
    v_cache[rows] = v


def gather_context(cache: np.ndarray, block_table, context_len: int,
                   block_size: int) -> np.ndarray:
    needed = -(-context_len // block_size)
    if needed > len(block_table):
        raise IndexError(f"context of {context_len} needs {needed} blocks, "
                         f"table has {len(block_table)}")
    rows = np.concatenate([np.arange(block_table[i] * block_size,
                                     (block_table[i] + 1) * block_size)
                           for i in range(needed)]) if needed else np.zeros(0, np.int64)
    return cache[rows[:context_len]]
