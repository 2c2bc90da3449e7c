"""The copier protocol and the host offload tier.

``SlotCopier`` is the plugin boundary of the handoff (the reference's
protocol, ie/core/offload.py:8-11): anything with ``read_block`` /
``write_block`` can move KV blocks for the block manager and the
disaggregation workers.

``KVTier`` keeps the payloads of evicted, hashed blocks so a later request
with the same prefix can restore them instead of recomputing them. Its
observable behaviour is the reference's (ie/core/offload.py:14-69), because
tier contents, their order and the statistics are what the golden traces
record:
* a tier of capacity 0 rejects every admission (counted);
* admitting a key it already holds refreshes the key's recency and keeps the
  payload it has (the new one is dropped);
* admitting into a full tier first evicts the least recently admitted or
  refreshed entries (counted);
* ``take`` removes an entry and counts a restore.

The store is a plain dict, whose iteration order is insertion order: the
first key is always the least recent, a refresh re-inserts a key at the end.
With the HIP copier the payloads live in pinned host memory.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, NamedTuple, Protocol


class SlotCopier(Protocol):
    """Moves the KV bytes of one physical block (ie/core/offload.py:8-11)."""

    def read_block(self, block_id: int) -> Any: ...

    def write_block(self, block_id: int, payload: Any) -> None: ...


@dataclass(slots=True)
class TierStats:
    """Counters of a tier's admissions, restores, evictions and rejections."""

    admitted: int = 0
    restored: int = 0
    evicted: int = 0
    rejected: int = 0

    @property
    def restore_rate(self) -> float:
        return self.restored / self.admitted if self.admitted else 0.0


class TierEntry(NamedTuple):
    """What the tier holds for one key: the block's tokens and its payload."""

    token_ids: list[int]
    payload: Any


class KVTier:
    """Capacity-bounded, least-recently-admitted-first store ``key -> TierEntry``."""

    def __init__(self, capacity_blocks: int) -> None:
        if capacity_blocks < 0:
            raise ValueError("capacity cannot be negative")
        self.capacity = capacity_blocks
        self.stats = TierStats()
        self._store: dict[str, TierEntry] = {}

    @property
    def entries(self) -> dict[str, TierEntry]:
        """The held entries, least recent first (read it, do not modify it)."""
        return self._store

    def __len__(self) -> int:
        return len(self._store)

    def __contains__(self, key: str) -> bool:
        return key in self._store

    @property
    def is_full(self) -> bool:
        return len(self._store) >= self.capacity

    def admit(self, key: str, token_ids: list[int], payload: Any) -> bool:
        """Hold ``payload`` under ``key``; False if the tier holds nothing at all."""
        if not self.capacity:
            self.stats.rejected += 1
            return False
        held = self._store.pop(key, None)
        if held is not None:                  # refresh: back to most recent, old payload
            self._store[key] = held
            return True
        while self.is_full:
            del self._store[next(iter(self._store))]
            self.stats.evicted += 1
        self._store[key] = TierEntry(list(token_ids), payload)
        self.stats.admitted += 1
        return True

    def holds(self, key: str, token_ids: list[int]) -> bool:
        """True if ``key`` is held for exactly these tokens."""
        entry = self._store.get(key)
        return entry is not None and entry.token_ids == token_ids

    def take(self, key: str) -> TierEntry | None:
        """Remove and return ``key``'s entry (a restore), or None."""
        entry = self._store.pop(key, None)
        if entry is not None:
            self.stats.restored += 1
        return entry

    def peek(self, key: str) -> TierEntry | None:
        return self._store.get(key)
