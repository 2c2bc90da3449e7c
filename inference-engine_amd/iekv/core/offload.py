"""The copier protocol and the host offload tier.

``SlotCopier`` is the plugin boundary of the handoff (reference:
ie/core/offload.py:8-11): anything with ``read_block``/``write_block`` can move
KV blocks for the block manager and the disaggregation workers. ``KVTier`` is
the LRU store of evicted, hashed blocks (reference: ie/core/offload.py:14-69);
with the HIP copier its payloads live in pinned host memory.
"""
from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass
from typing import Any, Protocol


class SlotCopier(Protocol):
    """Moves the KV bytes of one physical block (reference: ie/core/offload.py:8-11)."""

    def read_block(self, block_id: int) -> Any: ...

    def write_block(self, block_id: int, payload: Any) -> None: ...


@dataclass(slots=True)
class TierStats:
    admitted: int = 0
    restored: int = 0
    evicted: int = 0
    rejected: int = 0

    @property
    def restore_rate(self) -> float:
        return self.restored / self.admitted if self.admitted else 0.0


class KVTier:
    """Capacity-bounded LRU map ``hash -> (token_ids, payload)``.

    Semantics of ie/core/offload.py:26-69: a zero-capacity tier rejects every
    admit; re-admitting a held key only refreshes its recency (the new payload
    is dropped); admitting into a full tier evicts the least recently admitted
    entries first.
    """

    def __init__(self, capacity_blocks: int) -> None:
        if capacity_blocks < 0:
            raise ValueError("capacity cannot be negative")
        self.capacity = capacity_blocks
        self.entries: OrderedDict[str, tuple[list[int], Any]] = OrderedDict()
        self.stats = TierStats()

    def __len__(self) -> int:
        return len(self.entries)

    def __contains__(self, key: str) -> bool:
        return key in self.entries

    @property
    def is_full(self) -> bool:
        return len(self.entries) >= self.capacity

    def admit(self, key: str, token_ids: list[int], payload: Any) -> bool:
        if self.capacity == 0:
            self.stats.rejected += 1
            return False
        if key in self.entries:
            self.entries.move_to_end(key)
            return True
        while len(self.entries) >= self.capacity:
            self.entries.popitem(last=False)
            self.stats.evicted += 1
        self.entries[key] = (list(token_ids), payload)
        self.stats.admitted += 1
        return True

    def holds(self, key: str, token_ids: list[int]) -> bool:
        entry = self.entries.get(key)
        return entry is not None and entry[0] == token_ids

    def take(self, key: str) -> tuple[list[int], Any] | None:
        entry = self.entries.pop(key, None)
        if entry is not None:
            self.stats.restored += 1
        return entry

    def peek(self, key: str) -> tuple[list[int], Any] | None:
        return self.entries.get(key)
