"""Paged block allocator: free list, refcounts, chained-hash prefix index, offload hooks.

This is the code that decides the handoff's *destination* block ids and which
blocks a prefix-aware admit may skip. Behaviour follows the reference's
``BlockManager`` (ie/core/block_manager.py:10-226) exactly, because the
block tables after a handoff must match the reference entry for entry:

* free ids are a deque handed out from the left (``popleft``) and returned on
  the right, a released table in reverse order (block_manager.py:50,87-104,178-182);
* a shared block revived from the free list is removed from the middle of
  the deque (block_manager.py:94-98);
* a block leaving the free list forgets its hash, first offloading its payload
  to the tier when it is the canonical holder of that hash (block_manager.py:79-85);
* prefix plans match only full blocks and never the last one, and stop at the
  first miss or at a resident hit that follows a tier hit (block_manager.py:106-128).
"""
from __future__ import annotations

import hashlib
from collections import deque

from .offload import KVTier, SlotCopier
from .sequence import Sequence


def chain_hash(token_ids: list[int], parent: str | None = None) -> str:
    """Hex blake2b-128 of ``parent + "|" + ",".join(tokens)`` (ie/core/block_manager.py:10-16).

    The key format must be identical to the reference's, because the offload
    tier and the prefix index are keyed by it.
    """
    h = hashlib.blake2b(digest_size=16)
    if parent is not None:
        h.update(parent.encode() + b"|")
    h.update(",".join(str(t) for t in token_ids).encode())
    return h.hexdigest()


class Block:
    """One physical block of the pool (ie/core/block_manager.py:19-40)."""

    __slots__ = ("id", "ref_count", "hash", "token_ids")

    def __init__(self, block_id: int) -> None:
        self.id = block_id
        self.ref_count = 0
        self.hash: str | None = None
        self.token_ids: list[int] = []

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


class BlockManager:
    """Allocator of one pool's blocks (ie/core/block_manager.py:43-226)."""

    def __init__(self, num_blocks: int, block_size: int,
                 tier: KVTier | None = None, copier: SlotCopier | None = None) -> None:
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        self.block_size = block_size
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.free_ids: deque[int] = deque(range(num_blocks))
        self.block_id_by_hash: dict[str, int] = {}
        self.blocks_reused = 0
        self.blocks_computed = 0
        self.blocks_restored = 0
        self.tier = tier
        self.copier = copier

    # -- pool accounting ---------------------------------------------------
    @property
    def offload_enabled(self) -> bool:
        return self.tier is not None and self.copier is not None

    @property
    def num_free(self) -> int:
        return len(self.free_ids)

    @property
    def num_total(self) -> int:
        return len(self.blocks)

    @property
    def utilization(self) -> float:
        return 1.0 - self.num_free / self.num_total

    @property
    def reuse_rate(self) -> float:
        total = self.blocks_reused + self.blocks_computed
        return self.blocks_reused / total if total else 0.0

    def flush_pending(self) -> None:
        """Let a batching offload copier issue its queued reads (before a pool write)."""
        flush = getattr(self.copier, "flush", None)
        if flush is not None:
            flush()

    # -- block life cycle --------------------------------------------------
    def _forget(self, block: Block) -> None:
        """Drop a block's hash; offload it first if it is that hash's canonical holder."""
        key = block.hash
        if key is not None and self.block_id_by_hash.get(key) == block.id:
            if self.offload_enabled:
                # The read happens before the tier decides (it may reject or dedup).
                payload = self.copier.read_block(block.id)
                self.tier.admit(key, block.token_ids, payload)
            del self.block_id_by_hash[key]
        block.hash = None
        block.token_ids = []

    def _claim_free_block(self) -> Block:
        block = self.blocks[self.free_ids.popleft()]
        assert block.is_free, f"{block} was on the free list but is still referenced"
        self._forget(block)
        block.ref_count = 1
        return block

    def _claim_shared_block(self, block_id: int) -> None:
        block = self.blocks[block_id]
        if block.is_free:
            self.free_ids.remove(block_id)
        block.ref_count += 1

    def _release(self, block_id: int) -> None:
        block = self.blocks[block_id]
        block.ref_count -= 1
        if block.ref_count == 0:
            self.free_ids.append(block_id)

    # -- prefix planning -----------------------------------------------------
    def _prefix_plan(self, seq: Sequence) -> tuple[list[int], list[str]]:
        """Leading blocks already held: resident block ids, then tier keys."""
        resident: list[int] = []
        offloaded: list[str] = []
        parent: str | None = None
        for index in range(seq.num_blocks - 1):   # the last block is always recomputed
            if not seq.block_is_full(index):
                break
            tokens = seq.block_tokens(index)
            key = chain_hash(tokens, parent)
            block_id = self.block_id_by_hash.get(key)
            if block_id is not None and self.blocks[block_id].holds(tokens):
                if offloaded:
                    break
                resident.append(block_id)
            elif self.offload_enabled and self.tier.holds(key, tokens):
                offloaded.append(key)
            else:
                break
            parent = key
        return resident, offloaded

    def _reusable_prefix(self, seq: Sequence) -> list[int]:
        return self._prefix_plan(seq)[0]

    def _blocks_taken_from_pool(self, seq: Sequence, resident: list[int],
                                offloaded: list[str]) -> int:
        revived = sum(1 for block_id in resident if self.blocks[block_id].is_free)
        fresh = seq.num_blocks - len(resident) - len(offloaded)
        return revived + len(offloaded) + fresh

    def cached_prefix_tokens(self, seq: Sequence) -> int:
        resident, offloaded = self._prefix_plan(seq)
        return (len(resident) + len(offloaded)) * self.block_size

    def can_allocate(self, seq: Sequence) -> bool:
        resident, offloaded = self._prefix_plan(seq)
        return self.num_free >= self._blocks_taken_from_pool(seq, resident, offloaded)

    # -- allocation ----------------------------------------------------------
    def allocate(self, seq: Sequence) -> int:
        """Give ``seq`` a full block table, sharing and restoring its cached prefix.

        Returns the number of prompt tokens whose KV is already in the pool.
        """
        if seq.block_table:
            raise RuntimeError(f"sequence {seq.id} already holds blocks")
        resident, offloaded = self._prefix_plan(seq)
        if self.num_free < self._blocks_taken_from_pool(seq, resident, offloaded):
            raise RuntimeError("no capacity; call can_allocate() first")

        for block_id in resident:
            self._claim_shared_block(block_id)
            seq.block_table.append(block_id)

        # A copier with a batched write restores the whole prefix in one call
        # after the last claim (see _write_restored); a protocol-only copier
        # writes each block right after claiming it, as the reference does.
        batched = getattr(self.copier, "write_blocks", None) if len(offloaded) > 1 else None
        restores: list[tuple[int, object]] = []
        for key in offloaded:
            token_ids, payload = self.tier.take(key)
            # Claiming may offload a victim out of this very block: the victim's
            # read is enqueued before this block's restore write, so it sees the
            # old bytes.
            block = self._claim_free_block()
            if batched is None:
                self.copier.write_block(block.id, payload)
            else:
                restores.append((block.id, payload))
            block.hash = key
            block.token_ids = list(token_ids)
            self.block_id_by_hash[key] = block.id
            seq.block_table.append(block.id)
            self.blocks_restored += 1
        if restores:
            self._write_restored(batched, restores)

        cached = len(resident) + len(offloaded)
        for _ in range(cached, seq.num_blocks):
            seq.block_table.append(self._claim_free_block().id)

        self.blocks_reused += cached
        self.blocks_computed += seq.num_blocks - cached
        seq.num_computed = cached * self.block_size
        return seq.num_computed

    @staticmethod
    def _write_restored(write_blocks, restores: list[tuple[int, object]]) -> None:
        """Write the tier payloads a prefix plan restored, with one batched call.

        The reference writes each block right after claiming it
        (ie/core/block_manager.py:159-167); writing them all after the last
        claim has the same effect: a restore writes only blocks this allocation
        claimed, which no later claim of it can take as a victim, and every
        victim read those claims enqueued is issued before the writes (the HIP
        copier flushes its queued reads first). The HIP copier gathers the
        payloads' host images with one iekv_restore_blocks.
        """
        write_blocks([block_id for block_id, _ in restores],
                     [payload for _, payload in restores])

    def free(self, seq: Sequence) -> None:
        for block_id in reversed(seq.block_table):
            self._release(block_id)
        seq.block_table = []
        seq.num_computed = 0

    def can_append(self, seq: Sequence) -> bool:
        return not seq.block_table_is_short or self.num_free > 0

    def append_slot(self, seq: Sequence) -> None:
        if seq.block_table_is_short:
            if self.num_free == 0:
                raise RuntimeError("no free block; call can_append() first")
            seq.block_table.append(self._claim_free_block().id)

    def reserve(self, seq: Sequence, num_blocks: int) -> bool:
        """Grow ``seq``'s table to ``num_blocks`` fresh blocks (the handoff's dst ids).

        Returns False when the pool runs dry; the blocks claimed so far stay in
        the table, as in the reference (ie/core/block_manager.py:193-198).
        """
        while len(seq.block_table) < num_blocks:
            if not self.free_ids:
                return False
            seq.block_table.append(self._claim_free_block().id)
        return True

    def share_computed_blocks(self, seq: Sequence) -> None:
        """Index every full, computed leading block of ``seq`` under its chain hash."""
        parent: str | None = None
        for index in range(seq.num_blocks):
            if not (seq.block_is_full(index) and seq.block_is_computed(index)):
                return
            block = self.blocks[seq.block_table[index]]
            tokens = seq.block_tokens(index)
            key = chain_hash(tokens, parent)
            if block.hash != key:
                self._forget(block)
                block.hash = key
                block.token_ids = tokens
                self.block_id_by_hash[key] = block.id
            parent = key

    def stats(self) -> dict[str, float | int]:
        return {
            "total": self.num_total,
            "free": self.num_free,
            "utilization": round(self.utilization, 4),
            "reused": self.blocks_reused,
            "computed": self.blocks_computed,
            "reuse_rate": round(self.reuse_rate, 4),
            "shareable": len(self.block_id_by_hash),
            "restored": self.blocks_restored,
            "tier_held": len(self.tier) if self.tier else 0,
        }
