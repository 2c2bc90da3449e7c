"""NumPy restatement of the reference KV handoff — TEST INFRASTRUCTURE ONLY.

The reference moves KV bytes with ``LayeredSlotCopier`` (ie/engine/copier.py:6-38):
per block, ``2L`` slice copies out of the per-layer caches (read) and ``2L``
slice assignments into them (write), driven once per block of a request by
``PrefillWorker.prefill`` (ie/serve/disaggregated.py:50) and
``DecodeWorker.admit`` (ie/serve/disaggregated.py:81-82). This module restates
exactly that, over NumPy arrays of any dtype (bf16 / fp8 caches are handed in
as uint16 / uint8 views of their bytes, so every copy is bitwise).

It is the checker for the HIP path and the timed CPU baseline; it is never
part of the product.
"""
from __future__ import annotations

from typing import Any, Sequence

import numpy as np


class LayeredSlotCopier:
    """Per-block gather/scatter over per-layer caches (ie/engine/copier.py:6-38)."""

    def __init__(self, k_caches: Sequence[np.ndarray], v_caches: Sequence[np.ndarray],
                 block_size: int) -> None:
        self.k_caches = k_caches
        self.v_caches = v_caches
        self.block_size = block_size
        self.blocks_read = 0
        self.blocks_written = 0

    def _span(self, block_id: int) -> slice:
        """Rows [b*bs, (b+1)*bs) of every layer array (ie/engine/copier.py:14-16)."""
        first = block_id * self.block_size
        return slice(first, first + self.block_size)

    def read_block(self, block_id: int) -> tuple[list[np.ndarray], list[np.ndarray]]:
        """Fresh copies of the block's K tiles, then V tiles (ie/engine/copier.py:18-22)."""
        rows = self._span(block_id)
        self.blocks_read += 1
        return ([cache[rows].copy() for cache in self.k_caches],
                [cache[rows].copy() for cache in self.v_caches])

    def write_block(self, block_id: int, payload: Any) -> None:
        """Slice-assign a payload into the block (ie/engine/copier.py:24-31)."""
        rows = self._span(block_id)
        k_tiles, v_tiles = payload
        for cache, tile in zip(self.k_caches, k_tiles):
            cache[rows] = tile
        for cache, tile in zip(self.v_caches, v_tiles):
            cache[rows] = tile
        self.blocks_written += 1

    @property
    def bytes_moved(self) -> int:
        """(reads + writes) x 2L x T (ie/engine/copier.py:33-38)."""
        if not self.k_caches:
            return 0
        per_block = self.k_caches[0][self._span(0)].nbytes * 2 * len(self.k_caches)
        return (self.blocks_read + self.blocks_written) * per_block


def pack(copier: LayeredSlotCopier, block_ids: Sequence[int]) -> list:
    """The prefill side of one request: read every block of its table (disaggregated.py:50)."""
    return [copier.read_block(int(b)) for b in block_ids]


def unpack(copier: LayeredSlotCopier, block_ids: Sequence[int], payloads: Sequence) -> None:
    """The decode side of one request: write payload i into block i (disaggregated.py:81-82)."""
    for block_id, payload in zip(block_ids, payloads):
        copier.write_block(int(block_id), payload)


def handoff(src: LayeredSlotCopier, dst: LayeredSlotCopier, src_tables: Sequence[Sequence[int]],
            dst_tables: Sequence[Sequence[int]]) -> None:
    """Request by request: pack the source table, then unpack onto the destination table."""
    for src_ids, dst_ids in zip(src_tables, dst_tables):
        unpack(dst, dst_ids, pack(src, src_ids))


def packed_image(payloads: Sequence) -> np.ndarray:
    """Reference payloads as the build's block-major byte image ``[B, 2L, T]`` (uint8).

    Entry ``[i, a]`` holds tile ``a`` of payload ``i``: K of layers 0..L-1,
    then V of layers 0..L-1, i.e. the order of ``read_block``'s lists.
    """
    if not payloads:
        return np.zeros((0, 0, 0), dtype=np.uint8)
    rows = []
    for k_tiles, v_tiles in payloads:
        tiles = [np.ascontiguousarray(t).view(np.uint8).reshape(-1) for t in (*k_tiles, *v_tiles)]
        rows.append(np.stack(tiles))
    return np.stack(rows)


def as_bytes(array: np.ndarray, block_size: int) -> np.ndarray:
    """A cache array as ``[num_blocks, T]`` uint8 (a view when contiguous)."""
    flat = np.ascontiguousarray(array).view(np.uint8)
    rows = array.shape[0]
    return flat.reshape(rows // block_size, -1)
