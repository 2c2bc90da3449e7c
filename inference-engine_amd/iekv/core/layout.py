"""Slot addressing of a batch: the contract the destination pool must satisfy.

Token ``p`` of a sequence lives in slot ``block_table[p // bs] * bs + p % bs`` of
every layer's K and V array (the reference's addressing, ie/core/layout.py:46-53).
After a handoff, decode reads the moved blocks only through this mapping, so a
bit-exact copy of each tile under its new block id keeps decode token-identical.

``build_layout`` flattens a batch into the arrays a forward pass consumes
(ie/core/layout.py:60-93): the scheduled tokens of every sequence, their
positions and slots, per-sequence query and context lengths, and block tables
padded with -1 to the longest one. Each sequence's positions and slots are
computed as whole NumPy ranges.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .scheduler import Batch
from .sequence import Sequence


@dataclass(slots=True)
class BatchLayout:
    token_ids: list[int]
    positions: list[int]
    slot_mapping: list[int]
    context_lens: list[int]
    query_lens: list[int]
    block_tables: list[list[int]]
    is_prefill: bool

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)

    @property
    def cu_seqlens_q(self) -> list[int]:
        return np.concatenate(([0], np.cumsum(self.query_lens, dtype=np.int64))).tolist()

    @property
    def cu_seqlens_k(self) -> list[int]:
        return np.concatenate(([0], np.cumsum(self.context_lens, dtype=np.int64))).tolist()

    @property
    def max_query_len(self) -> int:
        return max(self.query_lens, default=0)

    @property
    def max_context_len(self) -> int:
        return max(self.context_lens, default=0)


def _slots(seq: Sequence, positions: np.ndarray, block_size: int) -> np.ndarray:
    blocks = positions // block_size
    held = len(seq.block_table)
    if positions.size and int(blocks[-1]) >= held:
        short = int(positions[np.argmax(blocks >= held)])
        raise IndexError(f"position {short} needs block {short // block_size} but sequence "
                         f"{seq.id} holds {held}")
    return np.asarray(seq.block_table, dtype=np.int64)[blocks] * block_size + \
        positions % block_size


def slot_for_position(seq: Sequence, position: int, block_size: int) -> int:
    """The cache row of token ``position`` of ``seq``."""
    return int(_slots(seq, np.array([position], dtype=np.int64), block_size)[0])


def computed_range(seq: Sequence) -> range:
    """Positions the current step computes for ``seq``."""
    return range(seq.num_computed, seq.num_computed + seq.num_scheduled)


def build_layout(batch: Batch, block_size: int) -> BatchLayout:
    """Flatten the scheduled tokens of ``batch``; pad block tables with -1."""
    seqs = batch.sequences
    starts = np.array([s.num_computed for s in seqs], dtype=np.int64)
    counts = np.array([s.num_scheduled for s in seqs], dtype=np.int64)
    for seq, n in zip(seqs, counts):
        if n <= 0:
            raise ValueError(f"sequence {seq.id} was scheduled with no tokens")
    tokens, positions, slots = [], [], []
    for seq, lo, n in zip(seqs, starts, counts):
        pos = np.arange(lo, lo + n, dtype=np.int64)
        positions.append(pos)
        slots.append(_slots(seq, pos, block_size))
        tokens.append(np.asarray(seq.token_ids[lo:lo + n], dtype=np.int64))
    width = max((len(s.block_table) for s in seqs), default=0)
    tables = np.full((len(seqs), width), -1, dtype=np.int64)
    for row, seq in enumerate(seqs):
        tables[row, :len(seq.block_table)] = seq.block_table

    def flat(parts: list[np.ndarray]) -> list[int]:
        return np.concatenate(parts).tolist() if parts else []

    return BatchLayout(token_ids=flat(tokens), positions=flat(positions),
                       slot_mapping=flat(slots), context_lens=(starts + counts).tolist(),
                       query_lens=counts.tolist(), block_tables=tables.tolist(),
                       is_prefill=batch.is_prefill)
