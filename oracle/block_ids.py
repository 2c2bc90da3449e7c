"""Brute-force restatement of the block-id flow — TEST INFRASTRUCTURE ONLY.

The handoff's destination ids are whatever the decode pool's free list hands
out: ``free_ids`` starts as ``0..N-1`` (ie/core/block_manager.py:50), a claim
takes the leftmost id (``popleft``, :87-92), a reference that drops to zero
appends the id on the right (:100-104), a freed table is released in reverse
order (:178-182), and ``reserve`` claims until the table is long enough or the
list is empty (:193-198). This model keeps only those rules (a Python list and
a refcount dict; no hashing), so the product's BlockManager can be checked
against it on long random traces.
"""
from __future__ import annotations


class FreeListModel:
    def __init__(self, num_blocks: int) -> None:
        self.free = list(range(num_blocks))
        self.refs = {b: 0 for b in range(num_blocks)}

    def claim(self) -> int:
        block = self.free.pop(0)
        assert self.refs[block] == 0
        self.refs[block] = 1
        return block

    def reserve(self, table: list[int], num_blocks: int) -> bool:
        while len(table) < num_blocks:
            if not self.free:
                return False
            table.append(self.claim())
        return True

    def release_table(self, table: list[int]) -> None:
        for block in reversed(table):
            self.refs[block] -= 1
            if self.refs[block] == 0:
                self.free.append(block)
        table.clear()

    def share(self, block: int) -> None:
        """Take one more reference on ``block`` (reviving it from the free list if needed)."""
        if self.refs[block] == 0:
            self.free.remove(block)
        self.refs[block] += 1
