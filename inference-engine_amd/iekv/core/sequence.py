"""Per-request state carried across the handoff.

A request is its token list, how far the KV cache has caught up with it
(``num_computed``), and the physical blocks that hold that KV
(``block_table``). These are exactly what a KVTransfer hands from the prefill
pool to the decode pool, so their names and meanings are the reference's
interface (ie/core/sequence.py:13-105): the workers, the block manager and the
scheduler read and write them directly.

Block arithmetic lives in :class:`BlockGeometry`, a value shared by a
sequence and everything that asks it about blocks: with block size ``bs``,
block ``i`` covers token positions ``[i*bs, (i+1)*bs)``, ``n`` tokens occupy
``ceil(n / bs)`` blocks, and the first ``n // bs`` of them are full.
"""
from __future__ import annotations

import itertools
from dataclasses import dataclass
from enum import Enum, auto


class Status(Enum):
    """Where a sequence is in the scheduler's queues."""

    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


@dataclass(frozen=True, slots=True)
class BlockGeometry:
    """Token positions <-> logical blocks for one block size."""

    block_size: int

    def __post_init__(self) -> None:
        if self.block_size <= 0:
            raise ValueError("block_size must be positive")

    def blocks_for(self, tokens: int) -> int:
        """Blocks that ``tokens`` tokens occupy (the last may be partial)."""
        return -(-tokens // self.block_size)

    def full_blocks(self, tokens: int) -> int:
        """Leading blocks that ``tokens`` tokens fill completely."""
        return tokens // self.block_size

    def span(self, index: int) -> slice:
        """Token positions of block ``index``."""
        return slice(index * self.block_size, (index + 1) * self.block_size)

    def end(self, index: int) -> int:
        """Number of tokens up to and including block ``index``."""
        return (index + 1) * self.block_size


_sequence_ids = itertools.count()


class Sequence:
    """One request's tokens, KV progress and physical blocks.

    ``num_computed`` counts leading tokens whose KV is in the cache;
    ``num_scheduled`` the tokens the current step computes; ``block_table[i]``
    is the physical block holding logical block ``i``. ``swapped`` is set while
    a swap preemption keeps the sequence's KV in host memory:
    ``(host payload of its first ceil(num_computed / block_size) blocks,
    num_computed at swap-out)``.
    """

    def __init__(self, prompt_ids: list[int], block_size: int, max_new_tokens: int = 64,
                 temperature: float = 1.0, eos_id: int | None = None) -> None:
        if len(prompt_ids) == 0:
            raise ValueError("a sequence needs at least one prompt token")
        self.geometry = BlockGeometry(block_size)
        self.id = next(_sequence_ids)
        self.token_ids: list[int] = list(prompt_ids)
        self.num_prompt = len(self.token_ids)
        self.max_new_tokens = max_new_tokens
        self.temperature = temperature
        self.eos_id = eos_id
        self.status = Status.WAITING
        self.num_computed = 0
        self.num_scheduled = 0
        self.block_table: list[int] = []
        self.swapped: tuple | None = None

    # -- sizes ---------------------------------------------------------------------
    @property
    def block_size(self) -> int:
        return self.geometry.block_size

    def __len__(self) -> int:
        return len(self.token_ids)

    @property
    def num_generated(self) -> int:
        return len(self) - self.num_prompt

    @property
    def last_token(self) -> int:
        return self.token_ids[-1]

    @property
    def num_uncomputed(self) -> int:
        return len(self) - self.num_computed

    @property
    def prompt_is_fully_computed(self) -> bool:
        return self.num_computed >= self.num_prompt

    @property
    def is_finished(self) -> bool:
        return self.status is Status.FINISHED

    # -- blocks --------------------------------------------------------------------
    @property
    def num_blocks(self) -> int:
        """Logical blocks the tokens so far occupy."""
        return self.geometry.blocks_for(len(self))

    @property
    def num_computed_blocks(self) -> int:
        return self.geometry.full_blocks(self.num_computed)

    @property
    def block_table_is_short(self) -> bool:
        """True when the last token has no physical block yet."""
        return self.num_blocks > len(self.block_table)

    def _check_block(self, index: int) -> None:
        if index < 0 or index >= self.num_blocks:
            raise IndexError(f"block {index} out of range for {self.num_blocks} blocks")

    def block_tokens(self, index: int) -> list[int]:
        self._check_block(index)
        return self.token_ids[self.geometry.span(index)]

    def block_is_full(self, index: int) -> bool:
        self._check_block(index)
        return self.geometry.end(index) <= len(self)

    def block_is_computed(self, index: int) -> bool:
        return self.geometry.end(index) <= self.num_computed

    # -- progress ------------------------------------------------------------------
    def append(self, token_id: int) -> None:
        self.token_ids.append(token_id)

    def commit_scheduled(self) -> None:
        """The step ran: its scheduled tokens now have KV in the cache."""
        self.num_computed, self.num_scheduled = self.num_computed + self.num_scheduled, 0

    def discard_computation(self) -> None:
        """Forget all KV progress and blocks (recompute preemption)."""
        self.status = Status.WAITING
        self.num_computed = self.num_scheduled = 0
        self.block_table = []

    def stop_reason(self) -> str | None:
        """``"eos"`` after the end-of-sequence token, ``"length"`` once
        ``max_new_tokens`` tokens were generated, else None."""
        if self.eos_id is not None and self.last_token == self.eos_id:
            return "eos"
        return "length" if self.num_generated >= self.max_new_tokens else None

    def __repr__(self) -> str:
        return (f"Sequence(id={self.id}, {self.status.name}, len={len(self)}, "
                f"computed={self.num_computed}, blocks={len(self.block_table)})")
