"""HIP slot copier: the reference's SlotCopier protocol over libiekv.

``HipSlotCopier`` is a drop-in for ``LayeredSlotCopier`` (ie/engine/copier.py:6-38):
``read_block(id)`` returns a snapshot payload, ``write_block(id, payload)``
scatters one back, ``blocks_read`` / ``blocks_written`` / ``bytes_moved`` count
exactly as the reference does. It adds the batched calls the workers use so a
request's whole block table moves in one launch instead of ``2L`` NumPy slice
copies per block:

* ``read_blocks(ids)``  -> one fused pack launch (iekv_pack), or the pinned-host
  offload pipeline (iekv_offload) when payloads live on the host;
* ``write_blocks(ids, payloads)`` -> one unpack launch (iekv_unpack), or the
  restore pipeline for host payloads (iekv_restore for one buffer's
  consecutive images, iekv_restore_blocks for images from unrelated buffers,
  such as the offload tier's entries);
* ``copy_blocks(source, src_ids, dst_ids)`` -> the direct pool-to-pool launch
  (iekv_copy_direct), which never materialises payloads.

Host block lists of up to ``HOST_IDS_MAX`` ids go to the ``*_ids`` variants of
these calls, which check them and carry them in the launches' kernel arguments;
longer lists are checked here and uploaded once.

Payloads are block-major byte images ``[n, 2L, T]`` (K tiles of layers
0..L-1, then V tiles). A single block's payload iterates as
``(k_list, v_list)`` of ``[block_size, H, D]`` tensors, the structure of the
reference payload (ie/engine/copier.py:21-22).

All work is enqueued on torch's current stream of the pool's device (host
copies on a side stream of the copier), so it is ordered with the model's
cache reads and writes exactly as the reference's synchronous copies are.
"""
from __future__ import annotations

import contextlib
import ctypes
import operator
import threading
import weakref
from array import array
from typing import Any, Iterable, Sequence as Seq

import numpy as np
import torch

from .. import _native
from .pools import (KVPool, StreamScope, check_device_ids, current_stream_handle, host_buffer,
                    integer_ids, stage_ids, stream_handle)

# Device staging the host pipelines use: two slots of at most this many bytes.
HOST_STAGING_BYTES = 256 << 20
# Longest host id list handed to the library's host-id entry points, which issue
# INLINE_IDS ids per launch: two launches cover every per-request table of the
# benchmark workloads (at most 508 blocks). A longer list is uploaded once and
# moved in one launch, where hundreds of 256-id launches would each add a launch's
# fixed cost.
HOST_IDS_MAX = 2 * _native.INLINE_IDS


class PackedBlocks:
    """Byte images of ``n`` blocks, ``[n, 2L, T]`` uint8, on a device or in pinned host memory.

    Indexing gives a :class:`BlockPayload` (an int) or a narrower
    :class:`PackedBlocks` (a slice); ``len`` is the number of blocks, so it
    stands in for the reference's ``block_payloads`` list (ie/serve/disaggregated.py:50-53).
    """

    def __init__(self, data: torch.Tensor, num_layers: int, tile_shape: tuple[int, ...],
                 dtype: torch.dtype) -> None:
        if data.dtype != torch.uint8 or data.dim() != 3 or data.shape[1] != 2 * num_layers:
            raise ValueError(f"packed data must be uint8 [n, {2 * num_layers}, T]")
        self.data = data
        self.num_layers = num_layers
        self.tile_shape = tuple(tile_shape)
        self.dtype = dtype
        self._event: torch.cuda.Event | None = None  # last async copy touching host data
        self._parent: PackedBlocks | None = None  # the buffer a slice views (kept alive)
        self._offset: int | None = 0   # first row in the root buffer (None: a strided view)
        self._pinned: bool | None = None   # the root's data is pinned host memory (None: unknown)
        self._checked = None           # the layout key of the last copier that accepted it

    @classmethod
    def _new(cls, data: torch.Tensor, num_layers: int, tile_shape: tuple[int, ...],
             dtype: torch.dtype, pinned: bool) -> "PackedBlocks":
        """A buffer a copier has just allocated in its pool's layout (no re-validation)."""
        self = cls.__new__(cls)
        self.data = data
        self.num_layers = num_layers
        self.tile_shape = tile_shape
        self.dtype = dtype
        self._event = None
        self._parent = None
        self._offset = 0
        self._pinned = pinned
        self._checked = None
        return self

    @property
    def pinned(self) -> bool:
        """Whether the data is pinned host memory (asked of torch once per buffer)."""
        root = self._root
        if root._pinned is None:
            root._pinned = bool(root.data.is_pinned())
        return root._pinned

    @property
    def _root(self) -> "PackedBlocks":
        return self._parent if self._parent is not None else self

    @property
    def on_host(self) -> bool:
        return self.data.device.type == "cpu"

    @property
    def tile_bytes(self) -> int:
        return self.data.shape[2]

    @property
    def nbytes(self) -> int:
        return self.data.numel()

    def __len__(self) -> int:
        return self.data.shape[0]

    def __getitem__(self, index):
        if isinstance(index, slice):
            view = PackedBlocks(self.data[index], self.num_layers, self.tile_shape, self.dtype)
            view._parent = self._root
            start, _, step = index.indices(len(self))
            view._offset = self._offset + start if step == 1 and self._offset is not None \
                else None
            return view
        n = len(self)
        if index < 0:
            index += n
        if not 0 <= index < n:
            raise IndexError(f"payload {index} out of range for {n} blocks")
        return BlockPayload(self, index)

    def __iter__(self):
        return (BlockPayload(self, i) for i in range(len(self)))

    def tiles(self, index: int) -> torch.Tensor:
        """Block ``index`` as typed tiles ``[2L, *tile_shape]`` (a view).

        Host data is read by the CPU as soon as the view exists, so a view of a
        buffer that an asynchronous copy is still filling waits for that copy
        first: the payload is a finished snapshot, as the reference's
        ``read_block`` returns one (ie/engine/copier.py:18-22).
        """
        if self.on_host:
            self.synchronize()
        return self.data[index].view(self.dtype).view(2 * self.num_layers, *self.tile_shape)

    def host_data(self) -> torch.Tensor:
        """``data`` of a host buffer once every pending copy into it has finished."""
        if not self.on_host:
            raise ValueError("the payload is in device memory")
        return self.synchronize().data

    def mark(self, stream: torch.cuda.Stream) -> None:
        """Record that async copies involving this (host) buffer end on ``stream``."""
        PackedBlocks.mark_all([self], stream)

    @staticmethod
    def mark_all(buffers: Seq["PackedBlocks"], stream: torch.cuda.Stream) -> None:
        """One event on ``stream`` marks the end of the copies of every buffer given."""
        ev = torch.cuda.Event()
        ev.record(stream)
        for buf in buffers:
            buf._root._event = ev

    @staticmethod
    def order_after(buffers: Seq["PackedBlocks"], stream: torch.cuda.Stream) -> None:
        """Order ``stream`` after the pending copies of every buffer given (a device-side
        wait, one per distinct event), so a restore issued on any stream reads host
        payloads only once their offload has written them."""
        seen = set()
        for buf in buffers:
            ev = buf._root._event
            if ev is not None and id(ev) not in seen:
                seen.add(id(ev))
                stream.wait_event(ev)

    def synchronize(self) -> "PackedBlocks":
        """Block the host until pending copies into or out of this buffer are done."""
        ev = self._root._event
        if ev is not None:
            ev.synchronize()
        elif not self.on_host:
            torch.cuda.current_stream(self.data.device).synchronize()
        return self

    def __del__(self) -> None:
        # The root owns the pinned memory, which goes back to torch's host cache
        # when it dies (views keep it alive); no DMA may still use it by then. A
        # buffer whose last copy is still running is held, with that copy's event,
        # until the event completes (_hold_until_done), so dying never blocks.
        if self._parent is not None:
            return
        ev = self._event
        if ev is None:
            return
        try:
            if not ev.query():
                _hold_until_done(self.data, ev)
        except Exception:
            try:
                ev.synchronize()
            except Exception:
                pass


class BlockPayload:
    """One block of a :class:`PackedBlocks`; unpacks as ``(k_list, v_list)``."""

    __slots__ = ("_packed", "_index")

    def __init__(self, packed: PackedBlocks | None, index: int) -> None:
        self._packed = packed
        self._index = index

    @property
    def packed(self) -> PackedBlocks:
        return self._packed

    @property
    def index(self) -> int:
        return self._index

    @property
    def k(self) -> list[torch.Tensor]:
        tiles = self.packed.tiles(self.index)
        return [tiles[l] for l in range(self.packed.num_layers)]

    @property
    def v(self) -> list[torch.Tensor]:
        tiles = self.packed.tiles(self.index)
        L = self.packed.num_layers
        return [tiles[L + l] for l in range(L)]

    def __iter__(self):
        yield self.k
        yield self.v

    def __len__(self) -> int:
        return 2

    def __getitem__(self, i: int) -> list[torch.Tensor]:
        return (self.k, self.v)[i]

    @property
    def nbytes(self) -> int:
        return self.packed.data[self.index].numel()


class DeferredBlockPayload(BlockPayload):
    """A host payload whose bytes are gathered at its copier's next :meth:`HipSlotCopier.flush`.

    Reading ``packed`` / ``index`` (or the tiles) before then flushes. The
    snapshot is still the block's contents at ``read_block`` time: every write
    to the pool flushes pending reads first (see ``HipSlotCopier``).
    """

    __slots__ = ("_copier", "block_id", "__weakref__")

    def __init__(self, copier: "HipSlotCopier", block_id: int) -> None:
        super().__init__(None, 0)
        self._copier = copier
        self.block_id = block_id

    def _resolve(self, packed: PackedBlocks, index: int) -> None:
        self._packed = packed
        self._index = index
        self._copier = None

    @property
    def packed(self) -> PackedBlocks:
        if self._packed is None:
            self._copier.flush()
        return self._packed

    @property
    def index(self) -> int:
        if self._packed is None:
            self._copier.flush()
        return self._index


# Pinned buffers whose PackedBlocks died while a copy still used them, each with
# that copy's event. Holding them keeps torch's pinned cache from handing the
# memory out again before the copy is done; they are dropped once it is. Payloads
# die in whatever thread drops them, even inside the pruning below (a garbage
# collection there runs their __del__ in the same thread), so the lock is
# reentrant and pruning pops entries one by one: one added meanwhile is popped
# and judged too, never lost.
_UNFINISHED: list[tuple[torch.Tensor, torch.cuda.Event]] = []
_UNFINISHED_LOCK = threading.RLock()


def _hold_until_done(data: torch.Tensor, ev: torch.cuda.Event) -> None:
    with _UNFINISHED_LOCK:
        _UNFINISHED.append((data, ev))
        crowded = len(_UNFINISHED) >= 32
    if crowded:
        _release_finished()


def _release_finished() -> None:
    """Drop the held buffers whose copies have completed (no waiting)."""
    with _UNFINISHED_LOCK:
        running = []
        while _UNFINISHED:
            held = _UNFINISHED.pop()
            if not held[1].query():
                running.append(held)
        _UNFINISHED.extend(running)


def _consecutive_views(payloads: Seq[Any]) -> PackedBlocks | None:
    """The PackedBlocks slice that ``payloads`` are consecutive rows of, if any.

    Payloads from different slices of one buffer count when their rows follow
    each other there (a staging buffer filled request by request). A strided slice
    (``payloads[::2]``) is not one run; a single payload always is (its own row,
    whatever buffer or slice it came from)."""
    if isinstance(payloads, PackedBlocks):
        return payloads if payloads.data.is_contiguous() else None
    if not payloads or not all(isinstance(p, BlockPayload) for p in payloads):
        return None
    if len(payloads) == 1:
        p = payloads[0]
        return p.packed[p.index:p.index + 1]
    first = payloads[0].packed
    if first._offset is None:
        return None
    root = first._root
    start = first._offset + payloads[0].index
    for k, p in enumerate(payloads):
        packed = p.packed
        if packed._root is not root or packed._offset is None or \
                packed._offset + p.index != start + k:
            return None
    return root[start:start + len(payloads)]


def join_payloads(parts: Seq[Any]) -> PackedBlocks | None:
    """One PackedBlocks for several payload lists whose rows follow each other in one
    buffer (so a single unpack moves them all), else None."""
    rows = [p for part in parts for p in part]
    return _consecutive_views(rows) if rows else None


def _host_id_array(ids) -> array | None:
    """A Python list or tuple of at most ``HOST_IDS_MAX`` ids as ``array('i')``, for
    the library's host-id entry points, which check the ids themselves
    (IEKV_ERR_RANGE, IEKV_ERR_IDS); None for anything else (NumPy arrays, tensors,
    longer lists, values that are not 32-bit integers), which the pool checks in
    NumPy.

    A serving loop's block tables are lists; converting one costs the host about a
    microsecond for a few hundred ids, where the NumPy checks cost 10-30 us, more
    than the launch they precede.
    """
    if type(ids) not in (list, tuple) or len(ids) > HOST_IDS_MAX:
        return None
    try:
        return array("i", ids)
    except (TypeError, OverflowError):
        return None


class _BlockIds:
    """The block ids of one call: host int32 ids, or a device tensor.

    Host ids are a NumPy int32 array the pool has checked, or an ``array('i')`` of a
    Python list that only the library's host-id entry points check. Up to
    ``HOST_IDS_MAX`` host ids go to those entry points (the ids ride in the
    launches' kernel arguments, INLINE_IDS per launch); a call that needs them on
    the device (a longer list, the host-memory pipelines) checks them here first
    (range, and distinctness for destinations) and uploads them once.
    """

    __slots__ = ("_pool", "host", "_on_device", "_unique", "_what", "_checked")

    def __init__(self, pool: KVPool, host=None, device_ids: torch.Tensor | None = None,
                 unique: bool = False, what: str = "block") -> None:
        self._pool = pool
        self._unique = unique
        self._what = what
        self._checked = None
        if host is not None and not isinstance(host, array):
            host = self._checked = np.ascontiguousarray(host, dtype=np.int32)
        self.host = host
        self._on_device = device_ids

    def __len__(self) -> int:
        return len(self.host) if self.host is not None else self._on_device.numel()

    def _host_array(self) -> np.ndarray:
        """The host ids as a checked NumPy int32 array."""
        if self._checked is None:
            ids = self._pool.host_ids(np.frombuffer(self.host, dtype=np.int32),
                                      unique=self._unique, what=self._what)
            self._checked = np.ascontiguousarray(ids, dtype=np.int32)
        return self._checked

    def __getitem__(self, index: slice) -> "_BlockIds":
        if self.host is not None:
            return _BlockIds(self._pool, host=self._host_array()[index])
        return _BlockIds(self._pool, device_ids=self._on_device[index])

    @property
    def inline(self) -> bool:
        """Host ids the host-id entry points take (in their launches' arguments)."""
        return self.host is not None and len(self.host) <= HOST_IDS_MAX

    def host_pointer(self) -> int:
        host = self.host
        if isinstance(host, array):
            return host.buffer_info()[0]
        return host.__array_interface__["data"][0]

    def on_device(self) -> torch.Tensor:
        if self._on_device is None:
            self._on_device = stage_ids(self._pool.device, self._host_array())[0]
        return self._on_device


class HipSlotCopier:
    """SlotCopier over per-layer GPU caches, backed by the HIP handoff kernels.

    ``payload_location`` chooses where ``read_block``/``read_blocks`` put
    payloads: ``"device"`` (the disaggregation transfer, a staging buffer in
    HBM) or ``"host"`` (the offload tier, pinned host memory).
    ``check_device_ids`` checks block ids given as device tensors on the GPU
    before each move (range; distinct destinations; disjoint source and
    destination within one pool) and raises as host lists do; the check waits
    for its answer, so it is for callers that prefer the error to the speed.
    Without it, device ids are taken as they are (the kernels skip ids outside
    the pool).
    """

    def __init__(self, k_caches: Seq[torch.Tensor], v_caches: Seq[torch.Tensor],
                 block_size: int, *, payload_location: str = "device",
                 defer_reads: bool | None = None, check_device_ids: bool = False) -> None:
        if payload_location not in ("device", "host"):
            raise ValueError("payload_location must be 'device' or 'host'")
        self.k_caches = k_caches
        self.v_caches = v_caches
        self.block_size = block_size
        self.pool = KVPool(k_caches, v_caches, block_size)
        self.payload_location = payload_location
        self.check_device_ids = check_device_ids
        # Single-block reads of host payloads (the offload hook's evictions) are
        # batched: they queue until flush(), which gathers every still-wanted
        # block with one iekv_offload.
        self.defer_reads = (payload_location == "host") if defer_reads is None else defer_reads
        self.blocks_read = 0
        self.blocks_written = 0
        self.offload_launches = 0       # iekv_offload calls made
        self.blocks_offloaded = 0       # blocks those calls moved to the host
        self.restore_launches = 0       # iekv_restore / iekv_restore_blocks calls made
        self._pending: list[tuple[int, weakref.ref]] = []
        self._copy_stream: torch.cuda.Stream | None = None
        self._staging: torch.Tensor | None = None
        self._staging_stream: torch.cuda.Stream | None = None   # the last call that used it
        # Payloads this copier has accepted carry this object, so a payload used
        # again (a tier entry restored in a batch) is not validated again.
        self._layout_key = (self.pool.n_arrays, self.pool.tile_bytes, self.pool.device)
        self._tile_shape = tuple(self.pool.tile_shape)

    # -- helpers -------------------------------------------------------------
    @property
    def device(self) -> torch.device:
        return self.pool.device

    def _empty_packed(self, n: int, on_host: bool) -> PackedBlocks:
        shape = (n, self.pool.n_arrays, self.pool.tile_bytes)
        if on_host:
            _release_finished()
            # A one-block buffer (a tier payload, kept for as long as the tier holds
            # it) pins exactly one block image; torch would round a block image that
            # is not a power of two up to one (2.5 MiB -> 4 MiB). Buffers of several
            # blocks live for one transfer or swap and stay with torch's cache,
            # whose power-of-two classes bound what it keeps for reuse.
            data = host_buffer(shape) if n == 1 else \
                torch.empty(shape, dtype=torch.uint8, pin_memory=True)
        else:
            data = torch.empty(shape, dtype=torch.uint8, device=self.device)
        out = PackedBlocks._new(data, self.pool.num_layers, self._tile_shape, self.pool.dtype,
                                pinned=on_host)
        out._checked = self._layout_key        # made in this pool's layout
        return out

    def copy_stream(self) -> torch.cuda.Stream:
        """The side stream host copies run on (default priority)."""
        if self._copy_stream is None:
            self._copy_stream = torch.cuda.Stream(self.device)
        return self._copy_stream

    def _host_staging(self, n_blocks: int) -> torch.Tensor:
        """Device staging for the host pipelines: up to two slots, bounded size.

        One buffer serves every host call of this copier, on whichever stream the
        call runs. The library leaves a call's compute stream ordered after its
        last use of the buffer, so a call on another stream is first ordered
        after the previous one's stream; a buffer replaced by a larger one is
        kept from reuse until the streams that used it have finished with it.
        """
        block = self.pool.block_bytes
        want = max(1, min(2 * n_blocks, max(2, HOST_STAGING_BYTES // block))) * block
        stream = torch.cuda.current_stream(self.device)
        last = self._staging_stream
        if self._staging is None or self._staging.numel() < want:
            if self._staging is not None:
                for used in (last, self._copy_stream):
                    if used is not None:
                        self._staging.record_stream(used)
            self._staging = torch.empty(want, dtype=torch.uint8, device=self.device)
        elif last is not None and last != stream:
            stream.wait_stream(last)
        self._staging_stream = stream
        return self._staging

    def _staging_for(self, n_blocks: int, direct: bool) -> tuple[int | None, int]:
        """(address, bytes) of the device staging a host call hands the library: none
        when the call moves pinned images directly (the library stages nothing then),
        so a copier whose host payloads are all pinned holds no staging buffer."""
        if direct:
            return None, 0
        staging = self._host_staging(n_blocks)
        return staging.data_ptr(), staging.numel()

    def _check_packed(self, packed: PackedBlocks) -> None:
        if packed._checked is self._layout_key:
            return
        if (packed.data.shape[1] != self.pool.n_arrays
                or packed.data.shape[2] != self.pool.tile_bytes):
            raise ValueError(
                f"payload of {packed.data.shape[1]} tiles x {packed.data.shape[2]} B does not "
                f"fit a pool of {self.pool.n_arrays} tiles x {self.pool.tile_bytes} B")
        if not packed.data.is_contiguous():
            raise ValueError("payload data must be contiguous")
        if not packed.on_host and packed.data.device != self.device:
            raise ValueError(f"payload on {packed.data.device}, pool on {self.device}")
        packed._checked = self._layout_key

    def _from_tiles(self, payload: Any) -> PackedBlocks:
        """Pack a reference-structured payload ``(k_list, v_list)`` into one block image."""
        k_list, v_list = payload
        tiles = list(k_list) + list(v_list)
        if len(tiles) != self.pool.n_arrays:
            raise ValueError(f"payload has {len(tiles)} tiles, pool needs {self.pool.n_arrays}")
        image = self._empty_packed(1, on_host=False)
        for a, tile in enumerate(tiles):
            t = tile if isinstance(tile, torch.Tensor) else torch.from_numpy(np.asarray(tile))
            if tuple(t.shape) != self.pool.tile_shape:
                raise ValueError(f"tile {a} has shape {tuple(t.shape)}, expected "
                                 f"{self.pool.tile_shape}")
            raw = t.contiguous().view(-1).view(torch.uint8)
            if raw.numel() != self.pool.tile_bytes:
                raise ValueError(f"tile {a} has {raw.numel()} bytes, expected "
                                 f"{self.pool.tile_bytes}")
            image.data[0, a].copy_(raw, non_blocking=True)
        return image

    # -- SlotCopier protocol (ie/core/offload.py:8-11) ---------------------------
    def read_block(self, block_id: int) -> BlockPayload:
        """Snapshot of one block (ie/engine/copier.py:18-22).

        With ``defer_reads`` the bytes are gathered at the next :meth:`flush`,
        batched with the other reads queued since; the counter still counts
        this read now, as the reference does.
        """
        if not self.defer_reads:
            return self.read_blocks([block_id])[0]
        block_id = operator.index(block_id)      # a float id is refused, not truncated
        if not 0 <= block_id < self.pool.num_blocks:
            raise IndexError(f"source block id {block_id} out of range for a pool of "
                             f"{self.pool.num_blocks} blocks")
        payload = DeferredBlockPayload(self, block_id)
        self._pending.append((block_id, weakref.ref(payload)))
        self.blocks_read += 1
        return payload

    @property
    def pending_reads(self) -> int:
        return len(self._pending)

    def flush(self) -> int:
        """Gather every queued read whose payload is still referenced, in one launch.

        Payloads nobody holds any more (a tier that rejected, deduplicated or
        already evicted them) are skipped. Returns the number of blocks moved.
        """
        if not self._pending:
            return 0
        pending, self._pending = self._pending, []
        live = [(block_id, p) for block_id, ref in pending if (p := ref()) is not None]
        if live and self.payload_location == "host":
            self._offload_each([b for b, _ in live], [p for _, p in live])
        elif live:
            packed = self._gather([b for b, _ in live], self.payload_location)
            for i, (_, payload) in enumerate(live):
                payload._resolve(packed, i)
        return len(live)

    def _image_group(self) -> int:
        """Most one-block host images one direct launch takes (IEKV_INLINE_IMAGES, and
        IEKV_HOST_DIRECT_MAX_BYTES together)."""
        return max(1, min(_native.INLINE_IMAGES, _native.HOST_DIRECT_MAX // self.pool.block_bytes))

    def _offload_each(self, block_ids: list[int], payloads: list) -> None:
        """Each deferred host read into a pinned buffer of its own (iekv_offload_blocks,
        one launch per group of images). A tier payload then keeps only its own
        block's bytes pinned, and buffers freed by the tier, all of one size, are
        reused by torch's pinned cache."""
        stream = torch.cuda.current_stream(self.device)
        group = self._image_group()
        for first in range(0, len(block_ids), group):
            ids = self._ids(block_ids[first:first + group], what="source block")  # host list
            n = len(ids)
            bufs = [self._empty_packed(1, on_host=True) for _ in range(n)]
            addresses = (ctypes.c_void_p * n)(*[b.data.data_ptr() for b in bufs])
            # Pinned images are written by the pack kernel itself (no staging).
            staging, staging_bytes = self._staging_for(n, True)
            fn, id_ptr = ("iekv_offload_blocks_ids", ids.host_pointer()) if ids.inline else \
                ("iekv_offload_blocks", ids.on_device().data_ptr())
            # Pinned images of one group are written by the pack kernel on `stream`;
            # the staged fallback orders `stream` after its last copy, so one event
            # on `stream` marks every buffer.
            _native.call(fn, self.pool.native.handle, id_ptr, n, addresses, staging,
                         staging_bytes, stream.cuda_stream, self.copy_stream().cuda_stream)
            PackedBlocks.mark_all(bufs, stream)
            for buf, payload in zip(bufs, payloads[first:first + group]):
                payload._resolve(buf, 0)
            self.offload_launches += 1
            self.blocks_offloaded += n

    def write_block(self, block_id: int, payload: Any) -> None:
        """Scatter one payload into ``block_id`` (ie/engine/copier.py:24-31)."""
        self.write_blocks([block_id], [payload])

    # -- batched calls -------------------------------------------------------
    def _on(self, stream: torch.cuda.Stream | None):
        """Run a call as if ``stream`` were the current stream (its launches, id uploads
        and new buffers are then ordered on it); None keeps the current stream."""
        if stream is None:
            return contextlib.nullcontext()
        if stream.device != self.device:
            raise ValueError(f"stream on {stream.device}, pool on {self.device}")
        return StreamScope(stream)

    def read_blocks(self, block_ids, *, location: str | None = None,
                    stream: torch.cuda.Stream | None = None,
                    into: PackedBlocks | None = None) -> PackedBlocks:
        """Pack ``block_ids`` (in order) into a new payload buffer with one launch.

        ``stream`` runs the call on that stream instead of the current one; the
        caller orders it after the work that wrote the blocks. Independent
        requests issued on different streams let one request's launch start
        while the previous one drains. ``into`` (device payloads of exactly
        ``len(block_ids)`` blocks, such as a slice of :meth:`empty_payloads`)
        receives the pack instead of a new buffer, and is returned.
        """
        with self._on(stream):
            out = self._gather(block_ids, location or self.payload_location, into)
        self.blocks_read += len(out)
        return out

    def empty_payloads(self, n_blocks: int) -> PackedBlocks:
        """An uninitialised device payload buffer of ``n_blocks`` blocks of this pool."""
        return self._empty_packed(n_blocks, on_host=False)

    def _ids(self, block_ids, *, unique: bool = False, what: str) -> "_BlockIds":
        if isinstance(block_ids, torch.Tensor) and block_ids.device.type == "cuda":
            ids = self.pool.block_ids(block_ids, what=what)
            if self.check_device_ids:
                if unique:
                    check_device_ids(None, None, self.pool, ids)
                else:
                    check_device_ids(self.pool, ids, None, None)
            return _BlockIds(self.pool, device_ids=ids)
        short = _host_id_array(block_ids)
        if short is not None:
            return _BlockIds(self.pool, host=short, unique=unique, what=what)
        return _BlockIds(self.pool, host=self.pool.host_ids(block_ids, unique=unique, what=what))

    def _gather(self, block_ids, location: str, into: PackedBlocks | None = None) -> PackedBlocks:
        ids = self._ids(block_ids, what="source block")
        n = len(ids)
        if into is not None:
            self._check_packed(into)
            if into.on_host:
                raise ValueError("read_blocks(into=...) takes device payloads")
            if len(into) != n:
                raise ValueError(f"read_blocks(into=...) got {len(into)} payload rows for "
                                 f"{n} blocks")
            out = into
        else:
            out = self._empty_packed(n, on_host=(location == "host"))
        if out.on_host:
            stream = torch.cuda.current_stream(self.device)
            # A pinned image is written by the pack kernel itself, at any size.
            staging, staging_bytes = self._staging_for(n, out.pinned)
            copy = self.copy_stream()
            # Short host lists ride in the launches' kernel arguments (no id upload).
            fn, id_ptr = ("iekv_offload_ids", ids.host_pointer()) if ids.inline else \
                ("iekv_offload", ids.on_device().data_ptr())
            _native.call(fn, self.pool.native.handle, id_ptr, n, out.data.data_ptr(), out.nbytes,
                         staging, staging_bytes, stream.cuda_stream, copy.cuda_stream)
            out.mark(stream)
            self.offload_launches += 1
            self.blocks_offloaded += n
        elif ids.inline:
            _native.call("iekv_pack_ids", self.pool.native.handle, ids.host_pointer(), n,
                         out.data.data_ptr(), out.nbytes, current_stream_handle(self.device))
        else:
            _native.call("iekv_pack", self.pool.native.handle, ids.on_device().data_ptr(), n,
                         out.data.data_ptr(), out.nbytes, current_stream_handle(self.device))
        return out

    def write_blocks(self, block_ids, payloads, *,
                     stream: torch.cuda.Stream | None = None) -> None:
        """Scatter ``payloads[i]`` into ``block_ids[i]`` for every i (one launch when possible).

        ``stream`` runs the call on that stream. Host payloads carry the event of
        the offload that wrote them, and the call waits for it on the device, so a
        restore may run on any stream. Device payloads carry none: the stream must
        be ordered after the work that produced them (the same stream as their
        read_blocks, say).
        """
        with self._on(stream):
            self._write_blocks(block_ids, payloads)

    def _write_blocks(self, block_ids, payloads) -> None:
        self.flush()   # queued reads see the blocks before this write
        ids = self._ids(block_ids, unique=True, what="destination block")
        n = len(ids)
        if len(payloads) != n:
            raise ValueError(f"{n} destination blocks for {len(payloads)} payloads")
        packed = _consecutive_views(payloads)
        if packed is not None:
            self._write_packed(ids, packed)
        elif n > 1 and all(isinstance(p, BlockPayload) and p.packed.on_host for p in payloads):
            self._restore_scattered(ids, payloads)
        else:
            for i, payload in enumerate(payloads):
                one = _consecutive_views([payload]) if isinstance(payload, BlockPayload) \
                    else self._from_tiles(payload)
                self._write_packed(ids[i:i + 1], one)
        self.blocks_written += n

    def _write_packed(self, ids: "_BlockIds", packed: PackedBlocks) -> None:
        self._check_packed(packed)
        n = len(ids)
        if packed.on_host:
            stream = torch.cuda.current_stream(self.device)
            PackedBlocks.order_after([packed], stream)
            # Pinned images are read by the unpack kernel itself on the compute
            # stream, whatever their size; passing that stream as the copy stream
            # spares the call a cross-stream hand-off it would not use.
            direct = packed.pinned
            staging, staging_bytes = self._staging_for(n, direct)
            copy = stream if direct else self.copy_stream()
            fn, id_ptr = ("iekv_restore_ids", ids.host_pointer()) if ids.inline else \
                ("iekv_restore", ids.on_device().data_ptr())
            _native.call(fn, self.pool.native.handle, id_ptr, n, packed.data.data_ptr(),
                         packed.nbytes, staging, staging_bytes, stream.cuda_stream,
                         copy.cuda_stream)
            packed.mark(copy)
            self.restore_launches += 1
        elif ids.inline:
            _native.call("iekv_unpack_ids", self.pool.native.handle, ids.host_pointer(), n,
                         packed.data.data_ptr(), packed.nbytes, current_stream_handle(self.device))
        else:
            _native.call("iekv_unpack", self.pool.native.handle, ids.on_device().data_ptr(), n,
                         packed.data.data_ptr(), packed.nbytes, current_stream_handle(self.device))

    def _restore_scattered(self, ids: "_BlockIds", payloads: Seq[BlockPayload]) -> None:
        """Host payloads from unrelated buffers (tier entries) -> iekv_restore_blocks, one
        call per group of images one direct launch takes."""
        # A row of a strided slice is addressed through a one-row view of itself.
        payloads = [p if p.packed.data.is_contiguous()
                    else BlockPayload(p.packed[p.index:p.index + 1], 0) for p in payloads]
        for p in payloads:
            self._check_packed(p.packed)
        stream = torch.cuda.current_stream(self.device)
        group = self._image_group()
        for first in range(0, len(ids), group):
            part = ids if len(ids) <= group else ids[first:first + group]
            chunk = payloads[first:first + group]
            n = len(part)
            packs = [p.packed for p in chunk]
            # Checked payloads are contiguous [n, 2L, T] rows: image i starts
            # index * block_bytes past its buffer's first byte.
            block = self.pool.block_bytes
            addresses = (ctypes.c_void_p * n)(*[q.data.data_ptr() + p.index * block
                                                for q, p in zip(packs, chunk)])
            PackedBlocks.order_after(packs, stream)
            # Pinned images are read by the unpack kernel itself on the compute
            # stream (IEKV_INLINE_IMAGES, IEKV_HOST_DIRECT_MAX_BYTES per launch): no
            # cross-stream hand-off.
            direct = all(q.pinned for q in packs)
            staging, staging_bytes = self._staging_for(n, direct)
            copy = stream if direct else self.copy_stream()
            fn, id_ptr = ("iekv_restore_blocks_ids", part.host_pointer()) if part.inline else \
                ("iekv_restore_blocks", part.on_device().data_ptr())
            _native.call(fn, self.pool.native.handle, id_ptr, n, addresses, staging,
                         staging_bytes, stream.cuda_stream, copy.cuda_stream)
            PackedBlocks.mark_all(list({id(q._root): q._root for q in packs}.values()), copy)
            self.restore_launches += 1

    def copy_blocks(self, source: "HipSlotCopier", src_ids, dst_ids, *,
                    stream: torch.cuda.Stream | None = None) -> None:
        """Direct pool-to-pool move: tile ``src_ids[i]`` of ``source`` -> ``dst_ids[i]`` here.

        ``stream`` runs the copy on that stream instead of the current one; the
        caller orders it after the writes of the source blocks and orders later
        readers of the destination blocks after it.
        """
        scope = self._on(stream)        # validates the stream's device
        if self._pending:
            with scope:                 # queued reads see the blocks before this write
                self.flush()
        self._copy_blocks(source, src_ids, dst_ids, stream)

    def _copy_blocks(self, source: "HipSlotCopier", src_ids, dst_ids,
                     on: torch.cuda.Stream | None) -> None:
        if not self.pool.same_shape(source.pool):
            raise ValueError("source and destination pools differ in layout")
        if source.device != self.device:
            raise ValueError(f"pools on {source.device} and {self.device}")
        on_device = (isinstance(src_ids, torch.Tensor) and src_ids.device.type == "cuda") or \
            (isinstance(dst_ids, torch.Tensor) and dst_ids.device.type == "cuda")
        stream = on.cuda_stream if on is not None else current_stream_handle(self.device)
        same_pool = source.pool.same_pool_as(self.pool)
        if on_device:
            with self._on(on):          # a host-side table's upload is ordered on the copy's stream
                src = source.pool.block_ids(src_ids, what="source block")
                dst = self.pool.block_ids(dst_ids, unique=True, what="destination block")
            if src.numel() != dst.numel():
                raise ValueError(f"{src.numel()} source blocks for {dst.numel()} destinations")
            n = dst.numel()
            if self.check_device_ids:
                with self._on(on):
                    check_device_ids(source.pool, src, self.pool, dst)
            _native.call("iekv_copy_direct", source.pool.native.handle, self.pool.native.handle,
                         src.data_ptr(), dst.data_ptr(), n, stream)
            source.blocks_read += n
            self.blocks_written += n
            return
        # Host ids, issued by destination id. Up to HOST_IDS_MAX pairs go to the
        # library, which checks and orders them, and travel in the launches' kernel
        # arguments (INLINE_IDS per launch); a serving loop's Python tables go there
        # unconverted by NumPy. Other host tables (arrays, CPU tensors) are checked
        # here first, and longer ones are uploaded together with one copy.
        s, d = _host_id_array(src_ids), _host_id_array(dst_ids)
        if s is not None and d is not None:
            if len(s) != len(d):
                raise ValueError(f"{len(s)} source blocks for {len(d)} destinations")
            n = len(d)
            _native.call("iekv_copy_direct_ids", source.pool.native.handle,
                         self.pool.native.handle, s.buffer_info()[0], d.buffer_info()[0], n,
                         stream)
            source.blocks_read += n
            self.blocks_written += n
            return
        s, d = issue_order(src_ids, dst_ids)
        s = source.pool.host_ids(s, what="source block")
        d = self.pool.host_ids(d, unique=True, what="destination block", ascending=True)
        if same_pool and bool(np.isin(s, d, assume_unique=False).any()):
            raise ValueError("a direct copy within one pool needs disjoint source "
                             "and destination blocks")
        n = int(d.size)
        if n <= HOST_IDS_MAX:
            s32 = np.ascontiguousarray(s, dtype=np.int32)
            d32 = np.ascontiguousarray(d, dtype=np.int32)
            _native.call("iekv_copy_direct_ids", source.pool.native.handle,
                         self.pool.native.handle, s32.__array_interface__["data"][0],
                         d32.__array_interface__["data"][0], n, stream)
        else:
            with self._on(on):          # the upload is ordered on the copy's stream
                src, dst = stage_ids(self.device, s, d)
            _native.call("iekv_copy_direct", source.pool.native.handle,
                         self.pool.native.handle, src.data_ptr(), dst.data_ptr(), n, stream)
        source.blocks_read += n
        self.blocks_written += n

    def copy_requests(self, source: "HipSlotCopier", tables, *,
                      streams: Seq[torch.cuda.Stream] | None = None,
                      done_events: Seq[torch.cuda.Event] | None = None) -> None:
        """Direct moves of several independent requests, one launch each, in one call.

        ``tables`` holds one ``(src_ids, dst_ids)`` pair of host tables per request
        (iekv_copy_direct_requests). Request k runs on ``streams[k % len(streams)]``
        (default: the current stream); every stream is first ordered after the
        current stream, where the ids are uploaded, and the caller orders later
        readers of the destinations after the streams, or after ``done_events[k]``,
        recorded right after request k's launch. Ids are checked as
        :meth:`copy_blocks` checks them, and requests may not share destination
        blocks. Each request's pairs are issued by destination id.
        """
        if not self.pool.same_shape(source.pool):
            raise ValueError("source and destination pools differ in layout")
        if source.device != self.device:
            raise ValueError(f"pools on {source.device} and {self.device}")
        streams = list(streams) if streams else [torch.cuda.current_stream(self.device)]
        for st in streams:
            if st.device != self.device:
                raise ValueError(f"stream on {st.device}, pool on {self.device}")
        if done_events is not None and len(done_events) != len(tables):
            raise ValueError(f"{len(done_events)} events for {len(tables)} requests")
        self.flush()
        counts, src_all, dst_all = [], [], []
        for src_ids, dst_ids in tables:
            s, d = issue_order(src_ids, dst_ids)
            counts.append(int(d.size))
            src_all.append(s)
            dst_all.append(d)
        s = source.pool.host_ids(np.concatenate(src_all) if src_all else [], what="source block")
        d = self.pool.host_ids(np.concatenate(dst_all) if dst_all else [], unique=True,
                               what="destination block")
        if source.pool.same_pool_as(self.pool) and bool(np.isin(s, d).any()):
            raise ValueError("a direct copy within one pool needs disjoint source "
                             "and destination blocks")
        if not counts:
            return
        src, dst = stage_ids(self.device, s, d)
        current = torch.cuda.current_stream(self.device)
        uploaded = torch.cuda.Event()
        uploaded.record(current)
        for st in streams:
            if st != current:
                st.wait_event(uploaded)
        events = None
        if done_events is not None:
            for ev in done_events:
                if not ev.cuda_event:         # torch creates its events at the first record
                    ev.record(current)
            events = (ctypes.c_void_p * len(done_events))(*[ev.cuda_event for ev in done_events])
        handles = (ctypes.c_void_p * len(streams))(*[st.cuda_stream for st in streams])
        count_array = array("i", counts)
        _native.call("iekv_copy_direct_requests", source.pool.native.handle,
                     self.pool.native.handle, len(counts), count_array.buffer_info()[0],
                     src.data_ptr(), dst.data_ptr(), handles, len(streams), events)
        for st in streams:          # the id buffers are freed on the current stream
            if st != current:
                src.record_stream(st)
                dst.record_stream(st)
        total = int(d.size)
        source.blocks_read += total
        self.blocks_written += total

    @property
    def bytes_moved(self) -> int:
        """(reads + writes) x 2L x T, as ie/engine/copier.py:33-38 counts."""
        return (self.blocks_read + self.blocks_written) * self.pool.block_bytes


def issue_order(src_ids, dst_ids) -> tuple[np.ndarray, np.ndarray]:
    """The (src, dst) pairs of a direct copy, reordered by ascending destination block id.

    The pairs of one copy are independent, so their order is free. Issued by
    destination id, the workgroups in flight write neighbouring tiles of each
    array. Measured on MI355X, the pool-to-pool copy of the benchmark workloads
    was then as fast or faster than in table order or source order (one launch:
    +7% on the Llama-3-8B shape, +5% with a shared prefix, +4% on the
    Qwen2.5-0.5B shape; equal where the table order already ascends).
    """
    src = integer_ids(src_ids, "source block")
    dst = integer_ids(dst_ids, "destination block")
    if src.shape != dst.shape:
        raise ValueError(f"{src.size} source blocks for {dst.size} destinations")
    order = np.argsort(dst, kind="stable")
    return src[order], dst[order]


def copier_for(k_caches, v_caches, block_size: int, role: str = "transfer") -> HipSlotCopier:
    """Default copier factory of the engine.

    ``transfer``: device payloads (the handoff); ``offload``: host payloads with
    batched (deferred) single-block reads (the tier); ``swap``: host payloads,
    read at once (swap preemption).
    """
    if role not in ("transfer", "offload", "swap"):
        raise ValueError(f"unknown copier role {role!r}")
    return HipSlotCopier(k_caches, v_caches, block_size,
                         payload_location="device" if role == "transfer" else "host",
                         defer_reads=(role == "offload"))


def stack_payloads(payloads: Iterable[BlockPayload]) -> PackedBlocks:
    """Gather arbitrary block payloads of one layout into a new contiguous PackedBlocks."""
    items = list(payloads)
    if not items:
        raise ValueError("no payloads")
    first = items[0].packed
    data = torch.stack([p.packed.data[p.index] for p in items])
    return PackedBlocks(data, first.num_layers, first.tile_shape, first.dtype)


__all__ = ["BlockPayload", "DeferredBlockPayload", "HipSlotCopier", "PackedBlocks", "copier_for",
           "issue_order", "stack_payloads", "stream_handle"]
