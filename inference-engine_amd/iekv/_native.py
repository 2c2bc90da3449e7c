"""ctypes binding of libiekv.so, the HIP KV-handoff library (C-ABI in include/iekv.h).

Loading imports torch first, so the library binds to the HIP runtime torch
already uses and torch's streams are valid handles for it. There is no
fallback: if the library is missing or fails to load, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_int, c_int32, c_int64, c_uint64, c_void_p
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "libiekv.so"
ABI_VERSION = 21

INLINE_IDS = 256   # IEKV_INLINE_IDS: most host ids one launch carries in its arguments
HOST_DIRECT_MAX = 64 << 20   # IEKV_HOST_DIRECT_MAX_BYTES: largest direct offload; restore launch size
INLINE_IMAGES = 128          # IEKV_INLINE_IMAGES: scattered host images restored in one launch
STATIC_STAGING = 32 << 20    # IEKV_STATIC_STAGING_BYTES: staging of iekv_offload_static
QUEUE_SLOTS = 256            # IEKV_QUEUE_SLOTS: queue descriptors in flight at once
QUEUE_MAX_BLOCKS = 1024      # IEKV_QUEUE_MAX_BLOCKS: blocks per queue descriptor
QUEUE_DONE = (1 << 64) - 1   # IEKV_QUEUE_DONE: ticket of an empty request

IEKV_OK = 0
IEKV_ERR_INVALID = -1
IEKV_ERR_HIP = -2
IEKV_ERR_CAPACITY = -3
IEKV_ERR_RANGE = -4      # a host block id outside its pool
IEKV_ERR_IDS = -5        # host ids that conflict (a destination twice; overlap within a pool)
IEKV_ERR_TIMEOUT = -6    # iekv_queue_wait: the requests did not finish in time
# Bits iekv_check_ids writes to its status word.
IEKV_IDS_SRC_RANGE = 1
IEKV_IDS_DST_RANGE = 2
IEKV_IDS_DST_REPEATED = 4
IEKV_IDS_OVERLAP = 8


def check_workspace_bytes(num_blocks: int) -> int:
    """Workspace iekv_check_ids needs for a destination pool of num_blocks blocks."""
    return (num_blocks + 31) // 32 * 4

# Every entry point of include/iekv.h: name -> (restype, argtypes).
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "iekv_abi_version": (c_int, []),
    "iekv_last_error": (c_char_p, []),
    "iekv_pool_create": (c_int, [POINTER(c_uint64), c_int32, c_int64, c_int64, c_int32,
                                 POINTER(c_void_p)]),
    "iekv_pool_destroy": (c_int, [c_void_p]),
    "iekv_copy_direct": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_void_p]),
    "iekv_copy_direct_requests": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p,
                                          c_void_p, c_void_p, c_int32, c_void_p]),
    "iekv_pack": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_void_p]),
    "iekv_unpack": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_void_p]),
    "iekv_copy_direct_ids": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_void_p]),
    "iekv_pack_ids": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_void_p]),
    "iekv_unpack_ids": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_void_p]),
    "iekv_write_slots": (c_int, [c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
                                 c_int32, c_void_p]),
    "iekv_gather_rows": (c_int, [c_void_p, c_int32, c_int32, c_void_p, c_int32, c_void_p,
                                 c_int64, c_void_p]),
    "iekv_write_slots_layers": (c_int, [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                        c_int64, c_void_p, c_int32, c_void_p]),
    "iekv_gather_rows_arrays": (c_int, [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_int32,
                                        c_void_p, c_int64, c_void_p]),
    "iekv_offload": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_void_p, c_int64,
                             c_void_p, c_void_p]),
    "iekv_offload_static": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_void_p,
                                    c_void_p]),
    "iekv_restore": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_void_p, c_int64,
                             c_void_p, c_void_p]),
    "iekv_restore_blocks": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int64,
                                    c_void_p, c_void_p]),
    "iekv_offload_ids": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_void_p,
                                 c_int64, c_void_p, c_void_p]),
    "iekv_restore_ids": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_void_p,
                                 c_int64, c_void_p, c_void_p]),
    "iekv_restore_blocks_ids": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p,
                                        c_int64, c_void_p, c_void_p]),
    "iekv_offload_blocks": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int64,
                                    c_void_p, c_void_p]),
    "iekv_offload_blocks_ids": (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p,
                                        c_int64, c_void_p, c_void_p]),
    "iekv_set_launch": (c_int, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32]),
    "iekv_set_direct_chunk": (c_int, [c_int32]),
    "iekv_get_direct_chunk": (c_int, [POINTER(c_int32)]),
    "iekv_get_launch": (c_int, [POINTER(c_int32), POINTER(c_int32), POINTER(c_int32),
                                POINTER(c_int32), POINTER(c_int32), POINTER(c_int32)]),
    "iekv_check_ids": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_void_p,
                               c_int64, c_void_p, c_void_p]),
    "iekv_host_alloc": (c_int, [c_int64, POINTER(c_void_p)]),
    "iekv_host_free": (c_int, [c_void_p]),
    "iekv_noop": (c_int, [c_int32, c_int32, c_void_p]),
    "iekv_profile_start": (c_int, [c_int32]),
    "iekv_profile_stop": (c_int, [POINTER(ctypes.c_float), c_int32, POINTER(c_int32)]),
    "iekv_queue_create": (c_int, [c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int64,
                                  POINTER(c_void_p)]),
    "iekv_queue_submit": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, POINTER(c_uint64)]),
    "iekv_queue_submit_requests": (c_int, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p,
                                           c_void_p]),
    "iekv_queue_wait": (c_int, [c_void_p, c_uint64, c_int64]),
    "iekv_queue_poll": (c_int, [c_void_p, c_uint64, POINTER(c_int32)]),
    "iekv_queue_stop": (c_int, [c_void_p]),
    "iekv_queue_destroy": (c_int, [c_void_p]),
    "iekv_queue_stats": (c_int, [c_void_p, POINTER(c_uint64), POINTER(c_uint64)]),
}

_lib: ctypes.CDLL | None = None


class NativeError(RuntimeError):
    """A libiekv call returned a non-zero status."""

    def __init__(self, function: str, code: int, message: str) -> None:
        super().__init__(f"{function} failed ({code}): {message}")
        self.function = function
        self.code = code


class NativeIndexError(NativeError, IndexError):
    """IEKV_ERR_RANGE: a block id outside its pool (Python's IndexError kind)."""


class NativeValueError(NativeError, ValueError):
    """IEKV_ERR_IDS: ids that conflict (a destination twice; overlap within a pool)."""


class NativeTimeoutError(NativeError, TimeoutError):
    """IEKV_ERR_TIMEOUT: queued requests that did not finish in time."""


_ERRORS = {IEKV_ERR_RANGE: NativeIndexError, IEKV_ERR_IDS: NativeValueError,
           IEKV_ERR_TIMEOUT: NativeTimeoutError}


def library_path() -> Path:
    override = os.environ.get("IEKV_LIBRARY")
    return Path(override) if override else LIBRARY


def lib() -> ctypes.CDLL:
    """The loaded library (loaded on first use)."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  (binds the library to torch's HIP runtime)

    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"{path} is missing: build it with `python -m iekv.build` or "
            "`python -c 'import __graft_entry__ as g; g.build()'` before using the HIP path")
    handle = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = handle.iekv_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
    _lib = handle
    return handle


def check(function: str, code: int) -> None:
    """Raise for a non-zero status: IndexError / ValueError kinds for the id checks
    (IEKV_ERR_RANGE, IEKV_ERR_IDS), NativeError (a RuntimeError) for the rest."""
    if code != IEKV_OK:
        message = lib().iekv_last_error().decode(errors="replace")
        raise _ERRORS.get(code, NativeError)(function, code, message)


_functions: dict[str, ctypes._CFuncPtr] = {}


def call(function: str, *args) -> None:
    """Call an entry point and raise NativeError on a non-zero status.

    The bound function is looked up once per name: issuing a launch costs the
    host about 2.3 us in HIP itself, and a per-call attribute lookup on the
    library would add to every request.
    """
    f = _functions.get(function)
    if f is None:
        f = _functions[function] = getattr(lib(), function)
    code = f(*args)
    if code:
        check(function, code)


class Pool:
    """A registered paged pool: 2L array base addresses, tile bytes, block count."""

    def __init__(self, array_ptrs: list[int], tile_bytes: int, num_blocks: int,
                 device: int) -> None:
        table = (c_uint64 * len(array_ptrs))(*array_ptrs)
        out = c_void_p()
        call("iekv_pool_create", table, len(array_ptrs), tile_bytes, num_blocks, device,
             ctypes.byref(out))
        self.handle = out
        self.n_arrays = len(array_ptrs)
        self.tile_bytes = tile_bytes
        self.num_blocks = num_blocks
        self.device = device

    @property
    def block_bytes(self) -> int:
        return self.n_arrays * self.tile_bytes

    def close(self) -> None:
        if self.handle is not None and self.handle.value and _lib is not None:
            _lib.iekv_pool_destroy(self.handle)
        self.handle = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


def set_launch(run_blocks: int = -1, unroll: int = 0, nontemporal: int = -1,
               order: int = -1, pack_order: int = -1, chunk_bytes: int = -1,
               direct_chunk_bytes: int = -1) -> None:
    """Launch shape of the move kernels; see iekv_set_launch in include/iekv.h.

    ``chunk_bytes`` sets the chunk size of every move; ``direct_chunk_bytes``
    (iekv_set_direct_chunk) then sets that of the launches that write a pool
    (pool-to-pool moves and unpacks), when not -1.
    """
    call("iekv_set_launch", run_blocks, unroll, nontemporal, order, pack_order, chunk_bytes)
    call("iekv_set_direct_chunk", direct_chunk_bytes)


def get_launch() -> dict[str, int]:
    run, unroll, nt, order, pack_order, chunk = (c_int32() for _ in range(6))
    call("iekv_get_launch", ctypes.byref(run), ctypes.byref(unroll), ctypes.byref(nt),
         ctypes.byref(order), ctypes.byref(pack_order), ctypes.byref(chunk))
    direct = c_int32()
    call("iekv_get_direct_chunk", ctypes.byref(direct))
    return {"run_blocks": run.value, "unroll": unroll.value, "nontemporal": nt.value,
            "order": order.value, "pack_order": pack_order.value, "chunk_bytes": chunk.value,
            "direct_chunk_bytes": direct.value}


class LaunchTimer:
    """Times every kernel launch the library makes inside a ``with`` block (this thread).

    Uses iekv_profile_start/stop: the start/stop events ride in each launch's
    own dispatch, so timing adds nothing to the stream between launches.
    ``durations_ms`` holds one entry per launch, in launch order.
    """

    def __init__(self, max_launches: int) -> None:
        self.max_launches = max_launches
        self.durations_ms: list[float] = []

    def __enter__(self) -> "LaunchTimer":
        call("iekv_profile_start", self.max_launches)
        return self

    def __exit__(self, *exc) -> None:
        out = (ctypes.c_float * self.max_launches)()
        count = c_int32()
        call("iekv_profile_stop", out, self.max_launches, ctypes.byref(count))
        self.durations_ms = list(out[:min(count.value, self.max_launches)])
