"""Paged block allocator: free list, reference counts, prefix index, offload hooks.

This module decides the handoff's *destination* block ids, and which leading
blocks of a prompt a prefix-aware admit may share instead of moving. Block
tables after a handoff must equal the reference's entry for entry
(ie/core/block_manager.py:43-226), so the observable rules are the
reference's:

* free ids leave from the front of the free list and return at its back; a
  freed table is released last block first;
* a block whose last reference drops keeps its prefix key until it is
  claimed again, so a later request can revive it; reviving removes it from
  wherever it sits in the free list;
* a block leaving the free list first forgets its prefix key, and if it was
  the key's canonical block and a tier is attached, its payload is read and
  offered to the tier (read first: the tier may reject or deduplicate it);
* a prefix plan looks only at full blocks and never at the last block; it
  stops at the first block it cannot reuse, and at a resident block that
  follows one the tier must restore.

The data structures are this build's own:

* :class:`FreeList` is a doubly linked list threaded through two integer
  arrays indexed by block id. Taking the front, appending at the back and
  removing a revived block from the middle are all O(1) (the reference's
  deque removes from the middle in O(n)).
* Per-block state is three parallel arrays (reference counts, prefix keys,
  the tokens each key stands for); ``blocks[i]`` is a read-only view.
* The prefix index maps a chain key to its canonical block. Chain keys are
  produced by one walker (:meth:`BlockManager._chain`) that both planning and
  indexing use, and a plan is a :class:`PrefixPlan` value.
"""
from __future__ import annotations

import hashlib
import operator
from dataclasses import dataclass, field
from types import MappingProxyType
from typing import Iterable, Iterator

from .offload import KVTier, SlotCopier
from .sequence import Sequence


def chain_hash(token_ids: list[int], parent: str | None = None) -> str:
    """Prefix key of a block: hex blake2b-128 of ``"<parent>|t0,t1,..."`` (just the
    token list for the first block). The offload tier and the prefix index are keyed
    by it, so it must equal the reference's key (ie/core/block_manager.py:10-16)."""
    text = ",".join(map(str, token_ids))
    if parent is not None:
        text = parent + "|" + text
    return hashlib.blake2b(text.encode(), digest_size=16).hexdigest()


class FreeList:
    """Ordered set of free block ids over ``0..n-1`` with O(1) front, back and middle ops.

    A circular doubly linked list whose sentinel is node ``n``: ``_next[i]`` and
    ``_prev[i]`` link block ``i`` to its neighbours while it is on the list.
    """

    __slots__ = ("_next", "_prev", "_on", "_len", "_end")

    def __init__(self, n: int) -> None:
        self._end = n
        self._on = [False] * n
        self._next = [0] * (n + 1)
        self._prev = [0] * (n + 1)
        self._len = 0
        self._link(range(n))

    def _link(self, order: Iterable[int]) -> None:
        end = self._end
        tail = end
        for b in order:
            self._next[tail] = b
            self._prev[b] = tail
            self._on[b] = True
            tail = b
            self._len += 1
        self._next[tail] = end
        self._prev[end] = tail

    def __len__(self) -> int:
        return self._len

    def __bool__(self) -> bool:
        return self._len > 0

    def __contains__(self, block_id: object) -> bool:
        try:
            b = operator.index(block_id)
        except TypeError:
            return False
        return 0 <= b < self._end and self._on[b]

    def __iter__(self) -> Iterator[int]:
        b = self._next[self._end]
        while b != self._end:
            yield b
            b = self._next[b]

    def __repr__(self) -> str:
        return f"FreeList({list(self)})"

    def pop_front(self) -> int:
        if not self._len:
            raise IndexError("no free block")
        b = self._next[self._end]
        self.discard(b)
        return b

    def push_back(self, block_id: int) -> None:
        if self._on[block_id]:
            raise ValueError(f"block {block_id} is already free")
        end = self._end
        last = self._prev[end]
        self._next[last] = block_id
        self._prev[block_id] = last
        self._next[block_id] = end
        self._prev[end] = block_id
        self._on[block_id] = True
        self._len += 1

    def discard(self, block_id: int) -> None:
        """Unlink ``block_id`` wherever it is on the list."""
        if not self._on[block_id]:
            raise ValueError(f"block {block_id} is not free")
        before, after = self._prev[block_id], self._next[block_id]
        self._next[before] = after
        self._prev[after] = before
        self._on[block_id] = False
        self._len -= 1

    def reorder(self, order: Iterable[int]) -> None:
        """Relink the same set of free ids in ``order``."""
        order = [int(b) for b in order]
        if len(order) != self._len or len(set(order)) != len(order) or \
                not all(b in self for b in order):
            raise ValueError("a new free-list order must list exactly the free blocks once")
        self._len = 0
        self._link(order)


class BlockView:
    """Read-only view of one physical block's state."""

    __slots__ = ("_m", "id")

    def __init__(self, manager: "BlockManager", block_id: int) -> None:
        self._m = manager
        self.id = block_id

    @property
    def ref_count(self) -> int:
        return self._m._refs[self.id]

    @property
    def hash(self) -> str | None:
        return self._m._keys[self.id]

    @property
    def token_ids(self) -> list[int]:
        held = self._m._tokens[self.id]
        return [] if held is None else held

    @property
    def is_free(self) -> bool:
        return self.ref_count == 0

    @property
    def is_shareable(self) -> bool:
        return self.hash is not None

    def holds(self, token_ids: list[int]) -> bool:
        return self.token_ids == token_ids

    def __repr__(self) -> str:
        return f"Block({self.id}, refs={self.ref_count}, shareable={self.is_shareable})"


class _BlockViews:
    """``manager.blocks``: indexable, sized and iterable views of every block."""

    __slots__ = ("_m",)

    def __init__(self, manager: "BlockManager") -> None:
        self._m = manager

    def __len__(self) -> int:
        return len(self._m._refs)

    def __getitem__(self, block_id: int) -> BlockView:
        if not -len(self) <= block_id < len(self):
            raise IndexError(f"block {block_id} out of range for {len(self)} blocks")
        return BlockView(self._m, block_id % len(self))

    def __iter__(self) -> Iterator[BlockView]:
        return (BlockView(self._m, b) for b in range(len(self)))


@dataclass(slots=True)
class PrefixPlan:
    """Leading blocks of a sequence whose KV is already held.

    ``resident``: ids of pool blocks to share (in table order); ``restored``:
    prefix keys the tier must give back (they follow the resident blocks).
    """

    resident: list[int] = field(default_factory=list)
    restored: list[str] = field(default_factory=list)

    @property
    def cached_blocks(self) -> int:
        return len(self.resident) + len(self.restored)


class BlockManager:
    """Allocator of one pool's blocks."""

    def __init__(self, num_blocks: int, block_size: int,
                 tier: KVTier | None = None, copier: SlotCopier | None = None) -> None:
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        self.block_size = block_size
        self.tier = tier
        self.copier = copier
        self._free = FreeList(num_blocks)
        self._refs = [0] * num_blocks
        self._keys: list[str | None] = [None] * num_blocks
        self._tokens: list[list[int] | None] = [None] * num_blocks
        self._index: dict[str, int] = {}      # prefix key -> its canonical block
        self.blocks = _BlockViews(self)
        self.blocks_reused = 0
        self.blocks_computed = 0
        self.blocks_restored = 0

    # -- views and accounting ---------------------------------------------------
    @property
    def free_ids(self) -> FreeList:
        """The free list, front first."""
        return self._free

    @free_ids.setter
    def free_ids(self, order: Iterable[int]) -> None:
        """Reorder the free list (every free id exactly once), e.g. to fragment it."""
        self._free.reorder(order)

    @property
    def block_id_by_hash(self) -> MappingProxyType:
        """Prefix key -> canonical block id (read-only)."""
        return MappingProxyType(self._index)

    @property
    def offload_enabled(self) -> bool:
        return self.tier is not None and self.copier is not None

    @property
    def num_free(self) -> int:
        return len(self._free)

    @property
    def num_total(self) -> int:
        return len(self._refs)

    @property
    def utilization(self) -> float:
        return 1.0 - self.num_free / self.num_total

    @property
    def reuse_rate(self) -> float:
        looked_up = self.blocks_reused + self.blocks_computed
        return self.blocks_reused / looked_up if looked_up else 0.0

    def flush_pending(self) -> None:
        """Let a batching offload copier issue its queued reads (before a pool write)."""
        flush = getattr(self.copier, "flush", None)
        if flush is not None:
            flush()

    # -- one block's life cycle -------------------------------------------------
    def _unkey(self, block_id: int) -> None:
        """The block is about to hold other KV: drop its prefix key, offloading the
        payload first when the block is that key's canonical holder."""
        key = self._keys[block_id]
        if key is not None and self._index.get(key) == block_id:
            if self.offload_enabled:
                payload = self.copier.read_block(block_id)
                self.tier.admit(key, self._tokens[block_id], payload)
            del self._index[key]
        self._keys[block_id] = None
        self._tokens[block_id] = None

    def _key(self, block_id: int, key: str, tokens: list[int]) -> None:
        self._keys[block_id] = key
        self._tokens[block_id] = tokens
        self._index[key] = block_id

    def _claim_fresh(self) -> int:
        block_id = self._free.pop_front()
        if self._refs[block_id]:
            raise AssertionError(f"block {block_id} was free but holds "
                                 f"{self._refs[block_id]} references")
        self._unkey(block_id)
        self._refs[block_id] = 1
        return block_id

    def _share(self, block_id: int) -> None:
        if self._refs[block_id] == 0:
            self._free.discard(block_id)
        self._refs[block_id] += 1

    def _unref(self, block_id: int) -> None:
        self._refs[block_id] -= 1
        if self._refs[block_id] == 0:
            self._free.push_back(block_id)

    # -- prefix keys ------------------------------------------------------------
    def _chain(self, seq: Sequence, count: int) -> Iterator[tuple[int, list[int], str]]:
        """(index, tokens, key) of the first ``count`` blocks of ``seq``, each key
        chained on the previous block's."""
        parent = None
        for index in range(count):
            tokens = seq.block_tokens(index)
            parent = chain_hash(tokens, parent)
            yield index, tokens, parent

    def plan_prefix(self, seq: Sequence) -> PrefixPlan:
        """Which leading blocks of ``seq`` are held: in the pool, then in the tier."""
        plan = PrefixPlan()
        # Only full blocks before the last one: the last block is always computed.
        for _, tokens, key in self._chain(seq, max(0, seq.num_blocks - 1)):
            owner = self._index.get(key)
            if owner is not None and self._tokens[owner] == tokens:
                if plan.restored:
                    break
                plan.resident.append(owner)
            elif self.offload_enabled and self.tier.holds(key, tokens):
                plan.restored.append(key)
            else:
                break
        return plan

    def _pool_cost(self, seq: Sequence, plan: PrefixPlan) -> int:
        """Free blocks an allocation following ``plan`` takes off the free list."""
        revived = sum(self._refs[b] == 0 for b in plan.resident)
        return revived + len(plan.restored) + seq.num_blocks - plan.cached_blocks

    def cached_prefix_tokens(self, seq: Sequence) -> int:
        return self.plan_prefix(seq).cached_blocks * self.block_size

    def can_allocate(self, seq: Sequence) -> bool:
        return self.num_free >= self._pool_cost(seq, self.plan_prefix(seq))

    # -- tables -----------------------------------------------------------------
    def allocate(self, seq: Sequence) -> int:
        """Give ``seq`` a full block table, sharing and restoring its cached prefix.

        Returns the number of prompt tokens whose KV is already in the pool.
        """
        if seq.block_table:
            raise RuntimeError(f"sequence {seq.id} already holds blocks")
        plan = self.plan_prefix(seq)
        if self.num_free < self._pool_cost(seq, plan):
            raise RuntimeError("no capacity; call can_allocate() first")
        table = seq.block_table
        for block_id in plan.resident:
            self._share(block_id)
            table.append(block_id)
        self._restore(plan.restored, table)
        cached = plan.cached_blocks
        for _ in range(seq.num_blocks - cached):
            table.append(self._claim_fresh())
        self.blocks_reused += cached
        self.blocks_computed += seq.num_blocks - cached
        seq.num_computed = cached * self.block_size
        return seq.num_computed

    def _restore(self, keys: list[str], table: list[int]) -> None:
        """Bring the tier's entries for ``keys`` back into fresh blocks appended to ``table``.

        Each entry's block is claimed right after the entry leaves the tier, as in
        the reference (ie/core/block_manager.py:159-167); claiming may offload a
        victim out of that very block, and the victim's read is issued before the
        block is written. A copier with a batched ``write_blocks`` writes all the
        restored blocks with one call after the last claim: a restore writes only
        blocks this allocation claimed, which no later claim of it can take as a
        victim, and the HIP copier flushes queued victim reads before any write,
        so every byte ends up the same. A protocol-only copier writes each block
        as it is claimed, which is the reference's exact call order.
        """
        batched = getattr(self.copier, "write_blocks", None) if len(keys) > 1 else None
        writes: list[tuple[int, object]] = []
        for key in keys:
            token_ids, payload = self.tier.take(key)
            block_id = self._claim_fresh()
            if batched is None:
                self.copier.write_block(block_id, payload)
            else:
                writes.append((block_id, payload))
            self._key(block_id, key, list(token_ids))
            table.append(block_id)
            self.blocks_restored += 1
        if writes:
            batched([b for b, _ in writes], [p for _, p in writes])

    def free(self, seq: Sequence) -> None:
        """Drop ``seq``'s references, last block first; keyed blocks stay revivable."""
        for block_id in reversed(seq.block_table):
            self._unref(block_id)
        seq.block_table = []
        seq.num_computed = 0

    def can_append(self, seq: Sequence) -> bool:
        return self.num_free > 0 or not seq.block_table_is_short

    def append_slot(self, seq: Sequence) -> None:
        """Give ``seq`` a block for its newest token if it needs one."""
        if not seq.block_table_is_short:
            return
        if not self.num_free:
            raise RuntimeError("no free block; call can_append() first")
        seq.block_table.append(self._claim_fresh())

    def reserve(self, seq: Sequence, num_blocks: int) -> bool:
        """Grow ``seq``'s table to ``num_blocks`` fresh blocks (a handoff's destination ids).

        Returns False when the pool runs dry; the blocks claimed so far stay in
        the table, as the reference leaves them (ie/core/block_manager.py:193-198).
        """
        table = seq.block_table
        while len(table) < num_blocks:
            if not self._free:
                return False
            table.append(self._claim_fresh())
        return True

    def share_computed_blocks(self, seq: Sequence) -> None:
        """Key every full, computed leading block of ``seq`` so later requests can share it."""
        ready = seq.geometry.full_blocks(min(len(seq), seq.num_computed))
        for index, tokens, key in self._chain(seq, ready):
            block_id = seq.block_table[index]
            if self._keys[block_id] != key:
                self._unkey(block_id)
                self._key(block_id, key, tokens)

    def stats(self) -> dict[str, float | int]:
        return {
            "total": self.num_total,
            "free": self.num_free,
            "utilization": round(self.utilization, 4),
            "reused": self.blocks_reused,
            "computed": self.blocks_computed,
            "reuse_rate": round(self.reuse_rate, 4),
            "shareable": len(self._index),
            "restored": self.blocks_restored,
            "tier_held": len(self.tier) if self.tier else 0,
        }
