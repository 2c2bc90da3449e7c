"""Per-request direct handoffs served by a resident kernel (``iekv_queue_*`` in include/iekv.h).

The reference hands prefilled requests to the decode pool one at a time
(``DisaggregatedEngine.generate``, ie/serve/disaggregated.py:106-116; each handoff
is a disaggregated.py:50 read and a :81-82 write). Issued as one kernel launch per
request, a request of a few MB costs the launch (3.9 us of dispatch and 2-4 us of
host time) rather than its bytes. :class:`HandoffQueue` serves the same requests
through a kernel that stays resident: a submission writes a descriptor into a ring
in pinned host memory, the kernel's movers claim the request's tiles, and the
request's ticket completes when its last tile has moved.

The queue moves a request as soon as it is submitted, in no order with any
stream: submit only requests whose source blocks are written (synchronize the
stream that wrote them first), read a destination only after :meth:`wait` (or
:meth:`done`) says its ticket is done, and keep requests in flight together on
distinct destination blocks. ``torch.cuda.synchronize()`` and ``hipFree`` wait for
every stream of the device, the queue's included, so they wait for its kernel to
end (at most the idle limit after the last submission); :meth:`stop` ends it at
once.
"""
from __future__ import annotations

import ctypes
import weakref
from ctypes import c_int32, c_uint64, c_void_p

import numpy as np

from .. import _native
from .pools import KVPool, integer_ids

DONE = _native.QUEUE_DONE


def _destroy(handle: c_void_p) -> None:
    if handle.value and _native._lib is not None:
        _native._lib.iekv_queue_destroy(handle)
        handle.value = None


def _id_array(ids, what: str) -> np.ndarray:
    """Host ids as a contiguous int32 array (type-checked as the copier's ids are)."""
    if isinstance(ids, np.ndarray) and ids.dtype == np.int32 and ids.flags.c_contiguous:
        return ids
    host = integer_ids(ids, what)
    out = host.astype(np.int32)
    if out.size and not np.array_equal(out, host):
        raise IndexError(f"{what} ids do not fit int32")
    return out


class HandoffQueue:
    """Direct handoffs from ``src`` to ``dst`` (two :class:`KVPool` of one shape).

    ``workers``: mover workgroups, each wave of which is a mover (0: one per compute
    unit, the leader's included); ``claim_bytes``: most bytes a mover claims at once
    (0: 512 KiB); ``idle_ms`` / ``life_ms``: the
    kernel's idle and lifetime limits (0: 200 ms / 60 s). The library restarts the
    kernel by itself when a submission comes near either limit.
    """

    def __init__(self, src: KVPool, dst: KVPool, *, workers: int = 0, claim_bytes: int = 0,
                 idle_ms: float = 0.0, life_ms: float = 0.0) -> None:
        if not src.same_shape(dst):
            raise ValueError("the pools differ in shape")
        handle = c_void_p()
        _native.call("iekv_queue_create", src.native.handle, dst.native.handle, workers,
                     claim_bytes, int(idle_ms * 1000), int(life_ms * 1000),
                     ctypes.byref(handle))
        self.handle = handle
        self.src, self.dst = src, dst
        self.last_ticket = DONE
        # The pools stay alive until the queue is destroyed: its kernel addresses them.
        self._finalizer = weakref.finalize(self, HandoffQueue._release, handle, src, dst)

    @staticmethod
    def _release(handle: c_void_p, src: KVPool, dst: KVPool) -> None:
        _destroy(handle)

    def _live(self) -> c_void_p:
        if not self.handle.value:
            raise RuntimeError("the queue is closed")
        return self.handle

    def submit(self, src_ids, dst_ids) -> int:
        """Submit one request (host ids, checked as iekv_copy_direct_ids checks them);
        its ticket. An empty request gives :data:`DONE`."""
        s = _id_array(src_ids, "source")
        d = _id_array(dst_ids, "destination")
        if s.size != d.size:
            raise ValueError(f"{s.size} source ids for {d.size} destination ids")
        ticket = c_uint64()
        _native.call("iekv_queue_submit", self._live(), s.ctypes.data, d.ctypes.data, s.size,
                     ctypes.byref(ticket))
        if ticket.value != DONE:
            self.last_ticket = ticket.value
        return ticket.value

    def submit_requests(self, counts, src_ids: np.ndarray, dst_ids: np.ndarray) -> list[int]:
        """Submit several requests in one call: request k moves counts[k] blocks, its
        ids following request k-1's in the concatenated int32 arrays. Their tickets."""
        counts = np.ascontiguousarray(counts, dtype=np.int32)
        s = _id_array(src_ids, "source")
        d = _id_array(dst_ids, "destination")
        if s.size != d.size or s.size != int(counts.sum()):
            raise ValueError("the id arrays must each hold sum(counts) ids")
        tickets = np.empty(counts.size, dtype=np.uint64)
        _native.call("iekv_queue_submit_requests", self._live(), counts.size, counts.ctypes.data,
                     s.ctypes.data, d.ctypes.data, tickets.ctypes.data)
        issued = tickets[tickets != np.uint64(DONE)]
        if issued.size:
            self.last_ticket = int(issued.max())
        return [int(t) for t in tickets]

    def wait(self, ticket: int | None = None, timeout: float | None = None) -> None:
        """Wait until every request up to and including ``ticket`` (default: the last
        submitted) is done; TimeoutError (NativeTimeoutError) after ``timeout`` s."""
        t = self.last_ticket if ticket is None else ticket
        _native.call("iekv_queue_wait", self._live(), t,
                     -1 if timeout is None else int(timeout * 1e6))

    def done(self, ticket: int) -> bool:
        """Whether every request up to and including ``ticket`` is done."""
        flag = c_int32()
        _native.call("iekv_queue_poll", self._live(), ticket, ctypes.byref(flag))
        return bool(flag.value)

    def stop(self) -> None:
        """Finish every submitted request and end the kernel (the next submission
        starts it again)."""
        if self.handle.value:
            _native.call("iekv_queue_stop", self.handle)

    def stats(self) -> dict[str, int]:
        """Descriptors submitted over the queue's life and kernel launches."""
        descriptors, launches = c_uint64(), c_uint64()
        _native.call("iekv_queue_stats", self._live(), ctypes.byref(descriptors),
                     ctypes.byref(launches))
        return {"descriptors": descriptors.value, "launches": launches.value}

    def close(self) -> None:
        """Stop the queue and release it."""
        self._finalizer()

    def __enter__(self) -> "HandoffQueue":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
