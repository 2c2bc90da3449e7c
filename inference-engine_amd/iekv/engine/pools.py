"""Device KV pools and their registration with libiekv.

A pool is what the reference's engine allocates per layer (ie/engine/engine.py:38-46,
ie/kernels/torch_backend.py:6-10, ie/model/torch_transformer.py:82-86): for each
layer a K and a V array of shape [num_blocks * block_size, H, D]. Here all 2L
arrays are views of ONE slab ``[2, L, num_blocks * block_size, H, D]`` (K half
first), so the library sees equally spaced arrays and addresses array ``a`` as
``base + a * stride`` with no pointer table. ``k_caches[l]`` / ``v_caches[l]``
keep the reference's per-layer shape, and the ``[N, bs, H, D]`` paged view
(ie/kernels/flash_backend.py:15-17) stays a free reshape.
"""
from __future__ import annotations

import ctypes
import math
from typing import Sequence as Seq

import numpy as np
import torch

from .. import _native


def allocate_pool(num_blocks: int, block_size: int, num_layers: int, num_kv_heads: int,
                  head_dim: int, *, dtype: torch.dtype = torch.float16,
                  device: str | torch.device = "cuda", zero: bool = True, pad_blocks: int = 0
                  ) -> tuple[list[torch.Tensor], list[torch.Tensor]]:
    """Per-layer K and V caches as views of one slab (zero-filled like the reference).

    ``pad_blocks`` leaves that many unused blocks after each array, so consecutive
    arrays start ``(num_blocks + pad_blocks)`` tiles apart instead of ``num_blocks``.
    """
    if min(num_blocks, block_size, num_layers, num_kv_heads, head_dim) <= 0 or pad_blocks < 0:
        raise ValueError("pool dimensions must be positive")
    rows = num_blocks * block_size
    shape = (2, num_layers, rows + pad_blocks * block_size, num_kv_heads, head_dim)
    slab = (torch.zeros if zero else torch.empty)(shape, dtype=dtype, device=device)
    return ([slab[0, l, :rows] for l in range(num_layers)],
            [slab[1, l, :rows] for l in range(num_layers)])


def paged_view(cache: torch.Tensor, block_size: int) -> torch.Tensor:
    """The ``[N, bs, H, D]`` view of one ``[N * bs, H, D]`` cache array
    (ie/kernels/flash_backend.py:15-17): entry ``b`` is block ``b``'s tile, the
    bytes the handoff kernels move for that block. No copy."""
    slots, heads, dim = cache.shape
    if block_size <= 0 or slots % block_size:
        raise ValueError(f"{slots} slots are not whole blocks of {block_size}")
    return cache.view(slots // block_size, block_size, heads, dim)


def allocate_pool_pair(first_blocks: int, second_blocks: int, block_size: int,
                       num_layers: int, num_kv_heads: int, head_dim: int, *,
                       dtype: torch.dtype = torch.float16,
                       device: str | torch.device = "cuda", zero: bool = True,
                       pad_blocks: int = 0):
    """Two pools of the same layout carved from ONE allocation, the first at the lower addresses.

    Returns ``((k_first, v_first), (k_second, v_second))``; each pool is the slab
    ``[2, L, N*bs, H, D]`` that :func:`allocate_pool` makes, and the second slab
    starts right after the first. Give the prefill (source) pool the first slot
    and the decode (destination) pool the second: on MI355X a direct copy from
    the lower pool of one reservation into the upper one measured 3% faster on
    the Llama-3-8B-shape handoff (6.29 against 6.11 TB/s for two separate
    allocations, three boxes) and 10-18% faster with 37 GB pools, and 5% slower
    in the opposite direction; splitting each array into halves instead gained
    nothing. ``pad_blocks`` pads every array of both pools as :func:`allocate_pool` does.
    """
    if min(first_blocks, second_blocks, block_size, num_layers, num_kv_heads,
           head_dim) <= 0 or pad_blocks < 0:
        raise ValueError("pool dimensions must be positive")
    row = num_kv_heads * head_dim
    n_first = 2 * num_layers * (first_blocks + pad_blocks) * block_size * row
    n_second = 2 * num_layers * (second_blocks + pad_blocks) * block_size * row
    flat = (torch.zeros if zero else torch.empty)(n_first + n_second, dtype=dtype, device=device)
    pools = []
    for start, blocks in ((0, first_blocks), (n_first, second_blocks)):
        stride = (blocks + pad_blocks) * block_size
        n = 2 * num_layers * stride * row
        slab = flat[start:start + n].view(2, num_layers, stride, num_kv_heads, head_dim)
        rows = blocks * block_size
        pools.append(([slab[0, l, :rows] for l in range(num_layers)],
                      [slab[1, l, :rows] for l in range(num_layers)]))
    return pools[0], pools[1]


# Exact-size pinned host buffers (iekv_host_alloc). torch's caching host allocator
# rounds every pinned request up to a power of two and keeps the block when the
# tensor dies: a 2.5 MiB block image then pins 4 MiB and a 43 GB image 64 GiB.
# Buffers made here pin exactly their size; one that dies goes back to a free list
# of its size, so a tier that recycles its payloads allocates only while it grows.
_PINNED_FREE: dict[int, list[int]] = {}
_PINNED_TYPES: dict[int, type] = {}


def _pinned_type(nbytes: int) -> type:
    """A ctypes byte array type of ``nbytes`` whose instances hand their memory back
    to the free list when the last tensor over them dies."""
    t = _PINNED_TYPES.get(nbytes)
    if t is None:
        free = _PINNED_FREE.setdefault(nbytes, [])
        addressof = ctypes.addressof

        class _Pinned(ctypes.c_ubyte * nbytes):
            __slots__ = ()

            def __del__(self, _free=free, _addressof=addressof) -> None:
                _free.append(_addressof(self))

        t = _PINNED_TYPES[nbytes] = _Pinned
    return t


def pinned_empty(nbytes: int) -> torch.Tensor:
    """A uint8 CPU tensor of exactly ``nbytes`` bytes of pinned host memory mapped for
    the GPU (uninitialised). Its memory is reused by later calls of the same size once
    every view of it is gone; :func:`release_pinned` returns unused buffers."""
    if nbytes <= 0:
        raise ValueError("nbytes must be positive")
    try:   # the pop alone: another thread may take the last free buffer first
        ptr = _PINNED_FREE[nbytes].pop()
    except (KeyError, IndexError):
        out = ctypes.c_void_p()
        _native.call("iekv_host_alloc", nbytes, ctypes.byref(out))
        ptr = out.value
    return torch.frombuffer(_pinned_type(nbytes).from_address(ptr), dtype=torch.uint8)


def pinned_bytes_cached() -> int:
    """Bytes of pinned buffers :func:`pinned_empty` holds for reuse."""
    return sum(size * len(ptrs) for size, ptrs in list(_PINNED_FREE.items()))


def release_pinned() -> int:
    """Free every unused buffer :func:`pinned_empty` holds (no copy may use them: a
    buffer is unused once its last tensor died, and host payloads keep their tensors
    alive until their copies finish). Returns the bytes freed."""
    freed = 0
    for size, ptrs in list(_PINNED_FREE.items()):   # sizes other threads add are skipped
        while True:
            try:
                ptr = ptrs.pop()
            except IndexError:
                break
            _native.call("iekv_host_free", ptr)
            freed += size
    return freed


def host_buffer(shape: tuple[int, ...], *, pinned: bool = True) -> torch.Tensor:
    """A uint8 host buffer of ``shape``: pinned memory of exactly its size when its size
    is not a power of two (:func:`pinned_empty`), else torch's pinned memory, which is
    then exact and cached by torch; pageable memory when ``pinned`` is false."""
    nbytes = math.prod(shape)
    if not pinned or nbytes <= 0:
        return torch.empty(shape, dtype=torch.uint8, pin_memory=pinned and nbytes > 0)
    if nbytes & (nbytes - 1) == 0:
        return torch.empty(shape, dtype=torch.uint8, pin_memory=True)
    return pinned_empty(nbytes).view(shape)


class KVPool:
    """A validated, registered set of per-layer caches (K arrays then V arrays)."""

    def __init__(self, k_caches: Seq[torch.Tensor], v_caches: Seq[torch.Tensor],
                 block_size: int) -> None:
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        if not k_caches or len(k_caches) != len(v_caches):
            raise ValueError("need one K and one V cache per layer")
        arrays = list(k_caches) + list(v_caches)
        first = arrays[0]
        for t in arrays:
            if not isinstance(t, torch.Tensor):
                raise TypeError(f"caches must be torch tensors, got {type(t).__name__}")
            if t.device.type != "cuda":
                raise ValueError(f"the HIP copier needs GPU caches, got one on {t.device}")
            if t.device != first.device or t.dtype != first.dtype or t.shape != first.shape:
                raise ValueError("all caches must share device, dtype and shape")
            if not t.is_contiguous():
                raise ValueError("caches must be contiguous")
        if first.dim() < 1 or first.shape[0] % block_size:
            raise ValueError(f"cache rows {tuple(first.shape)} are not a multiple of "
                             f"block_size {block_size}")
        self.num_layers = len(k_caches)
        self.block_size = block_size
        self.num_blocks = first.shape[0] // block_size
        self.tile_shape = (block_size, *first.shape[1:])
        self.tile_bytes = math.prod(self.tile_shape) * first.element_size()
        self.dtype = first.dtype
        self.device = first.device
        self._arrays = arrays  # keeps the memory alive while the handle exists
        # Array addresses and the byte range they span, for comparing pools by memory
        # (memory_relation) without asking torch again on every call.
        self._ptrs = tuple(t.data_ptr() for t in arrays)
        self._span = (min(self._ptrs), max(self._ptrs) + self.num_blocks * self.tile_bytes)
        self.native = _native.Pool(list(self._ptrs), self.tile_bytes, self.num_blocks,
                                   self.device.index or 0)
        self._check_buffers: tuple[torch.Tensor, torch.Tensor] | None = None

    @property
    def n_arrays(self) -> int:
        return 2 * self.num_layers

    def memory_relation(self, other: "KVPool") -> str:
        """How this pool's arrays share memory with ``other``'s: ``"same"`` (the same
        arrays, also through another KVPool made over the same caches), ``"partial"``
        (arrays that overlap without being the same) or ``"separate"``. Block ids of one
        pool mean the same blocks of the other only when they are the same."""
        if other is self:
            return "same"
        if self.device != other.device or self._span[1] <= other._span[0] or \
                other._span[1] <= self._span[0]:
            return "separate"          # the usual case, decided without a sort
        mine, theirs = self._ptrs, other._ptrs
        if mine == theirs and (self.tile_bytes, self.num_blocks) == (other.tile_bytes,
                                                                     other.num_blocks):
            return "same"
        span = self.num_blocks * self.tile_bytes
        other_span = other.num_blocks * other.tile_bytes
        spans = sorted([(a, a + span, 0) for a in mine] + [(b, b + other_span, 1)
                                                          for b in theirs])
        reach = [0, 0]
        for lo, hi, owner in spans:
            if reach[1 - owner] > lo:
                return "partial"
            reach[owner] = max(reach[owner], hi)
        return "separate"

    def same_pool_as(self, other: "KVPool") -> bool:
        """Whether ``other`` describes this pool's memory (see :meth:`memory_relation`);
        ValueError for pools that overlap without being the same."""
        relation = self.memory_relation(other)
        if relation == "partial":
            raise ValueError("the source and destination pools overlap in memory without "
                             "being the same pool")
        return relation == "same"

    @property
    def block_bytes(self) -> int:
        """Bytes of one block across all layers, K and V (2L * T)."""
        return self.n_arrays * self.tile_bytes

    def check_buffers(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The device workspace (a bitmap of this pool's blocks) and status word that
        :func:`check_device_ids` hands iekv_check_ids, made on first use."""
        if self._check_buffers is None:
            words = _native.check_workspace_bytes(self.num_blocks) // 4
            self._check_buffers = (torch.empty(words, dtype=torch.int32, device=self.device),
                                   torch.empty(1, dtype=torch.int32, device=self.device))
        return self._check_buffers

    def same_shape(self, other: "KVPool") -> bool:
        return (self.n_arrays == other.n_arrays and self.tile_bytes == other.tile_bytes
                and self.tile_shape == other.tile_shape and self.dtype == other.dtype)

    def block_ids(self, ids, *, unique: bool = False, what: str = "block") -> torch.Tensor:
        """Block ids as a contiguous int32 tensor on this pool's device.

        Host-side ids (lists, arrays, CPU tensors) are range-checked here and
        raise IndexError before anything is launched, then uploaded
        (:func:`stage_ids`). Device int32 tensors are taken as they are: the
        kernels skip ids outside the pool.
        """
        if isinstance(ids, torch.Tensor) and ids.device.type == "cuda":
            if ids.dtype != torch.int32 or ids.dim() != 1 or not ids.is_contiguous():
                raise TypeError("device block ids must be a contiguous 1-D int32 tensor")
            if ids.device != self.device:
                raise ValueError(f"block ids on {ids.device}, pool on {self.device}")
            return ids
        return stage_ids(self.device, self.host_ids(ids, unique=unique, what=what))[0]

    def host_ids(self, ids, *, unique: bool = False, what: str = "block",
                 ascending: bool = False) -> np.ndarray:
        """Host-side ids as int64 NumPy, range-checked against this pool (IndexError)
        and, with ``unique``, checked for repeats (ValueError). ``ascending`` says the
        ids are already sorted, so repeats are adjacent."""
        host = integer_ids(ids, what)
        if host.size:
            lo, hi = (int(host[0]), int(host[-1])) if ascending else \
                (int(host.min()), int(host.max()))
            if lo < 0 or hi >= self.num_blocks:
                bad = lo if lo < 0 else hi
                raise IndexError(f"{what} id {bad} out of range for a pool of "
                                 f"{self.num_blocks} blocks")
            if unique:
                ordered = host if ascending else np.sort(host)
                if host.size > 1 and bool((ordered[1:] == ordered[:-1]).any()):
                    raise ValueError(f"{what} ids must be distinct")
        return host


def integer_ids(ids, what: str = "block") -> np.ndarray:
    """Host-side ids (a sequence, NumPy array or CPU tensor) as a flat int64 array.

    Block ids index the pool as the reference's slices do (ie/engine/copier.py:14-16),
    which refuse non-integers: floats and other non-integer values raise TypeError
    instead of being truncated (booleans count as 0 and 1, as they do there)."""
    if isinstance(ids, torch.Tensor):
        if ids.numel() and (ids.dtype.is_floating_point or ids.dtype.is_complex):
            raise TypeError(f"{what} ids must be integers, not {ids.dtype}")
        return ids.detach().to(torch.int64).numpy().reshape(-1)
    given = np.asarray(ids)
    if given.size and given.dtype.kind not in "iub":
        raise TypeError(f"{what} ids must be integers, not {given.dtype}")
    return given.astype(np.int64, copy=False).reshape(-1)


def _device_list(ids: torch.Tensor, pool: KVPool, what: str) -> torch.Tensor:
    if not (isinstance(ids, torch.Tensor) and ids.device.type == "cuda"):
        raise TypeError(f"{what} ids must be a device tensor")
    if ids.dtype != torch.int32 or ids.dim() != 1 or not ids.is_contiguous():
        raise TypeError("device block ids must be a contiguous 1-D int32 tensor")
    if ids.device != pool.device:
        raise ValueError(f"block ids on {ids.device}, pool on {pool.device}")
    return ids


def check_device_ids(src_pool: KVPool | None, src_ids: torch.Tensor | None,
                     dst_pool: KVPool | None, dst_ids: torch.Tensor | None) -> None:
    """Check block ids held on the GPU (iekv_check_ids) and wait for the answer.

    Source ids are checked against ``src_pool``'s size, destination ids against
    ``dst_pool``'s and for repeats, and when both pools are the same registered
    pool (the same arrays, whichever handles describe them), that no block is
    both a source and a destination. The check runs on
    the current stream, ordered after whatever wrote the ids, and this call
    synchronises that stream to read the result: IndexError for an id outside
    its pool, ValueError for a repeated destination or an overlap.
    """
    if src_pool is None and dst_pool is None:
        raise ValueError("no pool to check against")
    n = None
    if src_pool is not None:
        src_ids = _device_list(src_ids, src_pool, "source")
        n = src_ids.numel()
    if dst_pool is not None:
        dst_ids = _device_list(dst_ids, dst_pool, "destination")
        if n is not None and dst_ids.numel() != n:
            raise ValueError(f"{n} source blocks for {dst_ids.numel()} destinations")
        n = dst_ids.numel()
    owner = dst_pool if dst_pool is not None else src_pool
    workspace, status = owner.check_buffers()
    _native.call("iekv_check_ids",
                 src_pool.native.handle if src_pool is not None else None,
                 src_ids.data_ptr() if src_pool is not None else None,
                 dst_pool.native.handle if dst_pool is not None else None,
                 dst_ids.data_ptr() if dst_pool is not None else None,
                 n, workspace.data_ptr() if dst_pool is not None else None,
                 workspace.numel() * 4 if dst_pool is not None else 0, status.data_ptr(),
                 current_stream_handle(owner.device))
    bits = int(status.item())
    if bits & _native.IEKV_IDS_SRC_RANGE:
        raise IndexError(f"source block id out of range for a pool of "
                         f"{src_pool.num_blocks} blocks")
    if bits & _native.IEKV_IDS_DST_RANGE:
        raise IndexError(f"destination block id out of range for a pool of "
                         f"{dst_pool.num_blocks} blocks")
    if bits & _native.IEKV_IDS_DST_REPEATED:
        raise ValueError("destination block ids must be distinct")
    if bits & _native.IEKV_IDS_OVERLAP:
        raise ValueError("a direct copy within one pool needs disjoint source and "
                         "destination blocks")


def stage_ids(device: torch.device, *arrays: np.ndarray) -> list[torch.Tensor]:
    """Copy host id arrays to ``device`` as int32 with ONE host-to-device copy.

    The arrays go through one pinned buffer, so a call that needs source and
    destination ids puts one copy on the stream instead of two (measured on
    the drop-in direct copy of the Llama-3-8B-shape workload: 5.69 -> 6.00
    TB/s). Uploading on a side stream with an event wait instead measured
    slower (5.86 TB/s) and tripled the host time per call. Returns one
    contiguous device view per array.
    """
    sizes = [a.size for a in arrays]
    flat = np.concatenate(arrays).astype(np.int32) if len(arrays) > 1 else \
        arrays[0].astype(np.int32)
    staged = torch.from_numpy(flat)
    if torch.cuda.is_available():
        staged = staged.pin_memory()
    on_device = staged.to(device, non_blocking=True)
    out, at = [], 0
    for n in sizes:
        out.append(on_device[at:at + n])
        at += n
    return out


def stream_handle(device: torch.device, stream: torch.cuda.Stream | None = None) -> int:
    """The raw hipStream_t of ``stream`` (default: torch's current stream on ``device``)."""
    return stream.cuda_stream if stream is not None else current_stream_handle(device)


_raw_current_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream_handle(device: torch.device) -> int:
    """The raw hipStream_t of torch's current stream on ``device`` (a CUDA device;
    without an index, the current one).

    torch's own ``current_stream(device)`` builds a Stream object and costs the
    host about 3 us, longer than issuing the launch the handle is for; the raw
    accessor skips that.
    """
    if _raw_current_stream is not None:
        index = device.index
        return _raw_current_stream(torch.cuda.current_device() if index is None else index)
    return torch.cuda.current_stream(device).cuda_stream


_get_stream = getattr(torch._C, "_cuda_getCurrentStream", None)
_set_stream = getattr(torch._C, "_cuda_setStream", None)
_get_device = getattr(torch._C, "_cuda_getDevice", None)
_set_device = getattr(torch._C, "_cuda_setDevice", None)
_LIGHT_SCOPE = None not in (_get_stream, _set_stream, _get_device, _set_device)


class StreamScope:
    """Make ``stream`` torch's current stream on its device for a ``with`` block.

    What ``torch.cuda.stream(stream)`` does for one device (launches, id uploads
    and new buffers inside the block are ordered on ``stream``), through torch's
    raw stream accessors: the public context manager costs the host about 6 us
    per use, more than the launch it wraps. The current device is restored too.
    Falls back to ``torch.cuda.stream`` where the raw accessors are missing.
    """

    __slots__ = ("stream", "_prev", "_device", "_fallback")

    def __init__(self, stream: torch.cuda.Stream) -> None:
        self.stream = stream
        self._fallback = None if _LIGHT_SCOPE else torch.cuda.stream(stream)

    def __enter__(self) -> torch.cuda.Stream:
        if self._fallback is not None:
            return self._fallback.__enter__()
        s = self.stream
        self._device = _get_device()
        self._prev = _get_stream(s.device_index)
        _set_stream(stream_id=s.stream_id, device_index=s.device_index,
                    device_type=s.device_type)
        return s

    def __exit__(self, *exc) -> None:
        if self._fallback is not None:
            self._fallback.__exit__(*exc)
            return
        stream_id, device_index, device_type = self._prev
        _set_stream(stream_id=stream_id, device_index=device_index, device_type=device_type)
        if _get_device() != self._device:
            _set_device(self._device)
