"""Disaggregated prefill -> decode serving over one GPU's HBM.

Public API as in the reference (ie/serve/disaggregated.py:16-130): a
``PrefillWorker`` runs a prompt to completion in its own pool and hands a
``KVTransfer`` to a ``DecodeWorker``, which places the blocks under freshly
reserved ids in its pool and continues decoding. The KV bytes move through
the copier the workers own: by default the HIP copier, so a request's whole
block table moves in one launch.

Transfer modes (``mode=``):

``"pack"`` (default, reference-exact)
    prefill packs the blocks into a device staging buffer (one fused pack
    launch, iekv_pack), frees its blocks, and the transfer carries the packed
    payloads; admit reserves fresh ids (``BlockManager.reserve``) and
    unpacks them (one launch, iekv_unpack). Block tables, counters and
    ``bytes_moved`` are those of the reference.
``"direct"``
    prefill keeps its blocks referenced and the transfer carries their ids;
    admit copies pool to pool (iekv_copy_direct, no staging, 2P bytes instead
    of 4P) and only then releases the prefill blocks. Destination ids and
    decode output are the same as in "pack" mode; the prefill pool's blocks
    are released at admit instead of at the end of prefill.

``"queue"``
    as "direct", but each admitted request's copy is submitted to a resident
    request queue (iekv_queue_*, :class:`iekv.engine.queue.HandoffQueue`) instead
    of being launched: its own descriptor, ticket and completion, no launch. The
    current stream is synchronized first (the prefill's writes of the sources and
    any earlier reads of the destinations are done), and the decode worker waits
    for the ticket before the request decodes, so admission stays synchronous per
    request as in the reference. ``generate`` ends the queue's kernel once every
    prompt is admitted, before decoding.

``prefix_aware=True`` (any mode)
    the decode worker is asked first which leading full blocks of the prompt
    its pool already holds under the same chain hashes; prefill moves only
    the blocks after them, and admit claims the held ones by reference count
    (``BlockManager.allocate`` rules, ie/core/block_manager.py:106-176) instead
    of reserving fresh blocks for them. The reference always moves every block
    (ie/serve/disaggregated.py:50); this mode is the build's addition for
    prefix-sharing workloads.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

from ..core.sequence import Sequence, Status
from ..engine.copier import join_payloads
from ..engine.engine import CopierFactory, Engine, EngineConfig

MODES = ("pack", "direct", "queue")

# Largest device staging buffer a batched pack-mode generate() fills before it
# unpacks what it holds (then it starts again at the beginning).
STAGING_ARENA_BYTES = 4 << 30


@dataclass(slots=True)
class DirectSource:
    """Where a direct-mode transfer copies from: a copier and its block ids."""

    copier: Any
    block_ids: list[int]
    release: Callable[[], None]
    released: bool = False

    def done(self) -> None:
        if not self.released:
            self.released = True
            self.release()


@dataclass(slots=True)
class PendingMove:
    """A move ``admit`` deferred for :meth:`DisaggregatedEngine.flush_moves`: a direct
    copy from ``source``, or an unpack of ``payloads``, into ``dst_ids`` of ``copier``."""

    copier: Any
    dst_ids: list[int]
    source: DirectSource | None = None
    payloads: Any = None


class _StagingArena:
    """Consecutive device payload slices for a batched pack-mode ``generate``.

    Each prefill packs into the next slice, so the payloads of every admitted
    request lie one after another and one unpack moves them all. When the
    buffer is full the pending unpacks are issued (stream-ordered before the
    packs that then reuse the buffer) and filling starts again.
    """

    def __init__(self, engine: "DisaggregatedEngine", capacity: int, pending: list) -> None:
        self.engine = engine
        self.capacity = capacity
        self.pending = pending
        self.buffer = None
        self.used = 0

    def take(self, n_blocks: int):
        if n_blocks == 0 or n_blocks > self.capacity:
            return None                        # a payload of its own
        if self.used + n_blocks > self.capacity:
            self.engine.flush_moves(self.pending)
            self.used = 0
        if self.buffer is None:
            self.buffer = self.engine.prefill.copier.empty_payloads(self.capacity)
        view = self.buffer[self.used:self.used + n_blocks]
        self.used += n_blocks
        return view


@dataclass(slots=True)
class KVTransfer:
    """The handoff record (ie/serve/disaggregated.py:16-25).

    ``block_payloads`` holds one payload per moved block, in block-table order
    (None for a direct-mode transfer, whose ``source`` names the blocks).
    ``first_block`` is the index in the sequence's table of the first moved
    block (non-zero only for prefix-aware transfers). ``bytes_moved`` is the
    payload size of the moved blocks, one direction (B x 2L x T).
    """

    token_ids: list[int]
    num_computed: int
    block_payloads: Any
    bytes_moved: int = 0
    first_block: int = 0
    source: DirectSource | None = None

    @property
    def num_blocks(self) -> int:
        if self.block_payloads is not None:
            return len(self.block_payloads)
        return len(self.source.block_ids) if self.source is not None else 0

    @property
    def table_length(self) -> int:
        return self.first_block + self.num_blocks


@dataclass(slots=True)
class DisaggregationStats:
    prefills: int = 0
    decodes: int = 0
    transfers: int = 0
    blocks_transferred: int = 0
    bytes_transferred: int = 0
    prefill_tokens: int = 0
    decode_tokens: int = 0
    blocks_skipped: int = 0


def _per_block_bytes(engine: Engine) -> int:
    """Payload bytes of one block, 2L x T (ie/serve/disaggregated.py:60-66)."""
    if not engine.k_caches:
        return 0
    bs = engine.config.block_size
    tile = engine.k_caches[0][0:bs]
    nbytes = tile.nbytes if hasattr(tile, "nbytes") else tile.numel() * tile.element_size()
    return int(nbytes) * 2 * len(engine.k_caches)


class PrefillWorker:
    """Runs prompts to completion and packages their KV (ie/serve/disaggregated.py:39-66)."""

    def __init__(self, model, config: EngineConfig, *, mode: str = "pack",
                 copier_factory: CopierFactory | None = None, caches=None) -> None:
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}")
        self.engine = Engine(model, config, copier_factory=copier_factory, caches=caches)
        self.copier = self.engine.make_copier("transfer")
        self.mode = mode

    def prefill(self, prompt_ids: list[int], temperature: float = 0.0,
                skip_blocks: int = 0, payload_buffer: Callable | None = None) -> KVTransfer:
        """Run a prompt to completion and package its KV (ie/serve/disaggregated.py:45-57).

        In pack mode ``payload_buffer(n)`` may supply the device payloads the
        ``n`` moved blocks are packed into (None: a new buffer).
        """
        seq = self.engine.submit(prompt_ids, max_new_tokens=1 << 30, temperature=temperature)
        while not seq.prompt_is_fully_computed:
            self.engine.step()
        if not 0 <= skip_blocks <= len(seq.block_table):
            raise ValueError(f"cannot skip {skip_blocks} of {len(seq.block_table)} blocks")
        moved = seq.block_table[skip_blocks:]
        nbytes = self._payload_bytes(len(moved))
        if self.mode in ("direct", "queue"):
            source = DirectSource(self.copier, list(moved), release=lambda: self._retire(seq))
            return KVTransfer(token_ids=list(seq.token_ids), num_computed=seq.num_computed,
                              block_payloads=None, bytes_moved=nbytes,
                              first_block=skip_blocks, source=source)
        payloads = self._read(moved, payload_buffer)
        transfer = KVTransfer(token_ids=list(seq.token_ids), num_computed=seq.num_computed,
                              block_payloads=payloads, bytes_moved=nbytes,
                              first_block=skip_blocks)
        self._retire(seq)
        return transfer

    def _read(self, block_ids: list[int], payload_buffer: Callable | None = None):
        if hasattr(self.copier, "read_blocks"):
            into = payload_buffer(len(block_ids)) if payload_buffer is not None else None
            if into is not None:
                return self.copier.read_blocks(block_ids, into=into)
            return self.copier.read_blocks(block_ids)          # one fused pack launch
        return [self.copier.read_block(b) for b in block_ids]  # generic SlotCopier

    def _retire(self, seq: Sequence) -> None:
        self.engine.blocks.free(seq)
        if seq in self.engine.scheduler.running:
            self.engine.scheduler.running.remove(seq)

    def _payload_bytes(self, num_blocks: int) -> int:
        return num_blocks * _per_block_bytes(self.engine)


class DecodeWorker:
    """Admits transfers into its pool and decodes them (ie/serve/disaggregated.py:69-96)."""

    def __init__(self, model, config: EngineConfig, *, prefix_aware: bool = False,
                 copier_factory: CopierFactory | None = None, caches=None) -> None:
        self.engine = Engine(model, config, copier_factory=copier_factory, caches=caches)
        self.copier = self.engine.make_copier("transfer")
        self.prefix_aware = prefix_aware
        self.use_queue = False      # direct transfers through a request queue ("queue" mode)
        self._queues: dict[int, Any] = {}

    def cached_prefix_blocks(self, prompt_ids: list[int]) -> int:
        """Leading full blocks of ``prompt_ids`` this pool already holds (0 unless prefix-aware).

        Only resident blocks count; a plan that would restore from the offload
        tier stops there, so the transfer carries those blocks instead.
        """
        if not self.prefix_aware:
            return 0
        probe = Sequence(prompt_ids, block_size=self.engine.config.block_size)
        return len(self.engine.blocks.plan_prefix(probe).resident)

    def admit(self, transfer: KVTransfer, max_new_tokens: int,
              temperature: float = 0.0, pending: list | None = None) -> Sequence:
        """Place a transfer's blocks under fresh ids (ie/serve/disaggregated.py:75-96).

        With ``pending`` (a list) the transfer's move (a direct copy, or the
        unpack of its payloads) is not issued here: a :class:`PendingMove` is
        appended for :meth:`DisaggregatedEngine.flush_moves` to issue together
        with others. A sequence that finishes on arrival is then not moved at
        all (its blocks are freed at once and never read).
        """
        engine = self.engine
        seq = engine.submit(transfer.token_ids[:-1], max_new_tokens=max_new_tokens,
                            temperature=temperature)
        if transfer.first_block:
            dst_ids = self._claim_with_prefix(seq, transfer)
        else:
            if not engine.blocks.reserve(seq, transfer.num_blocks):
                raise RuntimeError("decode worker has no room for the transferred cache")
            dst_ids = list(seq.block_table)

        engine.flush_offloads()   # evictions made room for dst_ids: read them first
        deferred = pending is not None
        if not deferred:
            self._move(transfer, dst_ids)

        seq.token_ids = list(transfer.token_ids)
        seq.num_computed = transfer.num_computed
        engine.scheduler.waiting.remove(seq)
        copied = True
        if deferred:
            if seq.stop_reason() is None:
                pending.append(PendingMove(self.copier, list(dst_ids), transfer.source,
                                           transfer.block_payloads))
            else:
                if transfer.source is not None:
                    transfer.source.done()
                copied = False      # never moved: its blocks hold no KV to share
        if (transfer.first_block or self.prefix_aware) and copied:
            engine.blocks.share_computed_blocks(seq)   # later requests can share these
        if seq.stop_reason() is not None:
            seq.status = Status.FINISHED
            engine.blocks.free(seq)
            engine.scheduler.finished.append(seq)
            return seq
        seq.status = Status.RUNNING
        engine.scheduler.running.append(seq)
        return seq

    def _claim_with_prefix(self, seq: Sequence, transfer: KVTransfer) -> list[int]:
        blocks = self.engine.blocks
        # A tier hit after the resident prefix is restored by allocate() and then
        # overwritten by the transfer's payload for the same tokens.
        resident = len(blocks.plan_prefix(seq).resident)
        if resident != transfer.first_block:
            self.engine.scheduler.waiting.remove(seq)
            raise RuntimeError(
                f"decode pool holds {resident} prefix blocks, the transfer assumed "
                f"{transfer.first_block}")
        if not blocks.can_allocate(seq):
            self.engine.scheduler.waiting.remove(seq)
            raise RuntimeError("decode worker has no room for the transferred cache")
        blocks.allocate(seq)
        if len(seq.block_table) != transfer.table_length:
            raise RuntimeError(f"admitted table has {len(seq.block_table)} blocks, transfer "
                               f"carries {transfer.table_length}")
        return seq.block_table[transfer.first_block:]

    def queue_from(self, source_copier):
        """The request queue from ``source_copier``'s pool into this worker's (made on
        first use); the current stream is synchronized, so the queue's moves see
        every write issued before."""
        import torch

        from ..engine.queue import HandoffQueue

        q = self._queues.get(id(source_copier))
        if q is None:
            if not (hasattr(source_copier, "pool") and hasattr(self.copier, "pool")):
                raise TypeError("queue transfers need HIP copiers on both sides")
            q = self._queues[id(source_copier)] = HandoffQueue(source_copier.pool,
                                                                self.copier.pool)
        torch.cuda.current_stream(self.copier.pool.device).synchronize()
        return q

    def stop_queues(self) -> None:
        """End the request queues' kernels (the next submission starts them again)."""
        for q in self._queues.values():
            q.stop()

    def _move(self, transfer: KVTransfer, dst_ids: list[int]) -> None:
        if transfer.source is not None:
            src = transfer.source
            if self.use_queue:
                q = self.queue_from(src.copier)
                q.wait(q.submit(src.block_ids, dst_ids))
                _count_copy(src.copier, self.copier, len(dst_ids))
                src.done()   # the copy has finished
                return
            if not hasattr(self.copier, "copy_blocks"):
                raise TypeError("direct transfers need a copier with copy_blocks()")
            self.copier.copy_blocks(src.copier, src.block_ids, dst_ids)
            src.done()   # stream-ordered after the copy's reads
        else:
            _write(self.copier, dst_ids, transfer.block_payloads)


def _count_copy(source, copier, n: int) -> None:
    """Count a queued copy of n blocks as copy_blocks counts its own: n blocks read
    from the source copier's pool and n written to the destination's."""
    source.blocks_read += n
    copier.blocks_written += n


def _write(copier, dst_ids: list[int], payloads) -> None:
    """Scatter payloads into dst_ids: one batched call, or the protocol's per-block writes."""
    if hasattr(copier, "write_blocks"):
        copier.write_blocks(dst_ids, payloads)
    else:
        for block_id, payload in zip(dst_ids, payloads):
            copier.write_block(block_id, payload)


class DisaggregatedEngine:
    """Prefill worker + decode worker over one model (ie/serve/disaggregated.py:99-130)."""

    def __init__(self, model, config: EngineConfig | None = None, *, mode: str = "pack",
                 prefix_aware: bool = False,
                 copier_factory: CopierFactory | None = None,
                 paired_pools: bool = True) -> None:
        config = config or EngineConfig()
        # Both pools live in one GPU's HBM: with a model that can allocate them
        # as one reservation (prefill pool first), the handoff copies run from
        # the lower pool into the upper one, the faster orientation on MI355X.
        pair = getattr(model, "allocate_cache_pair", None) if paired_pools else None
        caches = (pair(config.num_blocks, config.num_blocks, config.block_size)
                  if pair is not None else (None, None))
        self.prefill = PrefillWorker(model, config, mode=mode, copier_factory=copier_factory,
                                     caches=caches[0])
        self.decode = DecodeWorker(model, config, prefix_aware=prefix_aware,
                                   copier_factory=copier_factory, caches=caches[1])
        self.decode.use_queue = mode == "queue"
        self.stats = DisaggregationStats()

    def handoff(self, prompt: list[int], max_new_tokens: int, temperature: float = 0.0,
                pending: list | None = None, payload_buffer: Callable | None = None
                ) -> Sequence:
        """Prefill one prompt and admit it into the decode pool (its move deferred into
        ``pending`` when given; pack-mode payloads from ``payload_buffer`` when given)."""
        skip = self.decode.cached_prefix_blocks(prompt)
        transfer = self.prefill.prefill(prompt, temperature, skip_blocks=skip,
                                        payload_buffer=payload_buffer)
        self.stats.prefills += 1
        self.stats.transfers += 1
        self.stats.blocks_transferred += transfer.num_blocks
        self.stats.bytes_transferred += transfer.bytes_moved
        self.stats.prefill_tokens += len(prompt)
        self.stats.blocks_skipped += transfer.first_block
        return self.decode.admit(transfer, max_new_tokens, temperature, pending=pending)

    def flush_moves(self, pending: list) -> int:
        """Issue deferred moves and return the number of blocks moved.

        Direct copies: one pool-to-pool launch per (source, destination) copier
        pair, then the prefill blocks are released. Unpacks: per destination
        copier, one launch when the payloads lie one after another in one buffer
        (a batched pack-mode ``generate``), else one per transfer.
        """
        copies: dict[tuple[int, int], tuple[Any, Any, list[int], list[int], list]] = {}
        unpacks: dict[int, tuple[Any, list[list[int]], list]] = {}
        for move in pending:
            if move.source is not None:
                key = (id(move.source.copier), id(move.copier))
                if key not in copies:
                    copies[key] = (move.source.copier, move.copier, [], [], [])
                _, _, src_all, dst_all, sources = copies[key]
                src_all.extend(move.source.block_ids)
                dst_all.extend(move.dst_ids)
                sources.append(move.source)
            else:
                entry = unpacks.setdefault(id(move.copier), (move.copier, [], []))
                entry[1].append(move.dst_ids)
                entry[2].append(move.payloads)
        moved = 0
        for src_copier, dst_copier, src_all, dst_all, sources in copies.values():
            if src_all and self.decode.use_queue:
                # one request per move, submitted together, then waited for
                import numpy as np

                q = self.decode.queue_from(src_copier)
                q.submit_requests([len(x.block_ids) for x in sources],
                                  np.asarray(src_all, dtype=np.int32),
                                  np.asarray(dst_all, dtype=np.int32))
                q.wait()
                _count_copy(src_copier, dst_copier, len(src_all))
                moved += len(src_all)
            elif src_all:
                dst_copier.copy_blocks(src_copier, src_all, dst_all)
                moved += len(src_all)
            for source in sources:
                source.done()     # stream-ordered after the copy's reads
        for dst_copier, dst_lists, payload_lists in unpacks.values():
            joined = join_payloads(payload_lists) if hasattr(dst_copier, "write_blocks") else None
            if joined is not None:
                dst_copier.write_blocks([b for ids in dst_lists for b in ids], joined)
            else:
                for ids, payloads in zip(dst_lists, payload_lists):
                    _write(dst_copier, ids, payloads)
            moved += sum(len(ids) for ids in dst_lists)
        pending.clear()
        return moved

    def _prefill_has_room(self, prompt: list[int]) -> bool:
        blocks = self.prefill.engine.blocks
        probe = Sequence(prompt, block_size=self.prefill.engine.config.block_size)
        return blocks.can_allocate(probe)

    def generate(self, prompts: list[list[int]], max_new_tokens: int = 16,
                 temperature: float = 0.0, *, batch_moves: bool = False) -> list[list[int]]:
        """Prefill, hand off and decode ``prompts`` (ie/serve/disaggregated.py:106-130).

        ``batch_moves=True`` admits every prompt as the reference does — same
        block tables, same order — but moves the KV of all of them together
        before decoding starts:
        - direct mode: one copy launch (earlier only if the prefill pool runs
          short of room for the next prompt, its blocks being held until then);
        - pack mode: each prompt is still packed with one launch and its prefill
          blocks freed at once, as in the reference, but into the next slice of
          one device staging buffer, so a single unpack launch places every
          request (earlier only when that buffer, at most STAGING_ARENA_BYTES,
          is full).
        """
        pending: list | None = [] if batch_moves else None
        payload_buffer = None
        if batch_moves and self.prefill.mode == "pack" and \
                hasattr(self.prefill.copier, "empty_payloads"):
            bs = self.prefill.engine.config.block_size
            need = sum(-(-(len(p) + 1) // bs) for p in prompts)
            block = max(1, _per_block_bytes(self.prefill.engine))
            capacity = max(1, min(need, STAGING_ARENA_BYTES // block))
            payload_buffer = _StagingArena(self, capacity, pending).take
        sequences = []
        for prompt in prompts:
            if pending and self.prefill.mode in ("direct", "queue") and \
                    not self._prefill_has_room(prompt):
                self.flush_moves(pending)
            sequences.append(self.handoff(prompt, max_new_tokens, temperature, pending,
                                          payload_buffer))
        if pending:
            self.flush_moves(pending)
        self.decode.stop_queues()   # every prompt is admitted: the GPU is the decode's
        self.decode_until_done()
        return [s.token_ids[s.num_prompt:] for s in sequences]

    def decode_until_done(self) -> None:
        """Step the decode worker until every admitted sequence has finished
        (the decode loop of ie/serve/disaggregated.py:117-129)."""
        engine = self.decode.engine
        while engine.scheduler.has_work:
            batch, _ = engine._advance()
            if batch is None:
                break
            self.stats.decodes += 1
            self.stats.decode_tokens += len(batch)
