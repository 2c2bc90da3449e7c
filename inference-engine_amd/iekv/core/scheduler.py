"""Prefill-first continuous-batching scheduler.

Only the parts the handoff touches need to be reproduced exactly: the queue
transitions the workers rely on (``waiting`` -> ``running`` -> ``finished``),
decode-time ``append_slot`` growth of block tables, recompute preemption, and
hashing of computed blocks after every step. Behaviour follows
ie/core/scheduler.py:38-162.

With a ``swapper`` (a copier whose payloads live in host memory), preemption
swaps instead of recomputing: the victim's computed blocks are packed out to
the host and freed, and when the sequence is scheduled again they are
restored into fresh blocks, so its KV is never recomputed. Without one the
reference's recompute preemption is used unchanged.
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

from .block_manager import BlockManager
from .sequence import Sequence, Status


@dataclass(slots=True)
class Batch:
    sequences: list[Sequence] = field(default_factory=list)
    is_prefill: bool = False

    @property
    def num_tokens(self) -> int:
        return sum(seq.num_scheduled for seq in self.sequences)

    def __bool__(self) -> bool:
        return bool(self.sequences)

    def __len__(self) -> int:
        return len(self.sequences)


@dataclass(slots=True)
class SchedulerStats:
    steps: int = 0
    prefill_steps: int = 0
    decode_steps: int = 0
    preemptions: int = 0
    finished: int = 0
    tokens_prefilled: int = 0
    tokens_decoded: int = 0
    tokens_reused_from_cache: int = 0
    swapped_out: int = 0
    swapped_in: int = 0


class Scheduler:
    """ie/core/scheduler.py:38-162."""

    def __init__(self, block_manager: BlockManager, max_batch_sequences: int = 256,
                 max_batch_tokens: int = 8192, swapper=None) -> None:
        self.blocks = block_manager
        self.swapper = swapper
        self.max_batch_sequences = max_batch_sequences
        self.max_batch_tokens = max_batch_tokens
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()
        self.finished: list[Sequence] = []
        self.stats = SchedulerStats()

    @property
    def has_work(self) -> bool:
        return bool(self.waiting) or bool(self.running)

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    def schedule(self) -> Batch:
        """A prefill batch if any prompt can start or continue, else a decode batch."""
        batch = self._schedule_prefill()
        if batch:
            self.stats.steps += 1
            self.stats.prefill_steps += 1
            self.stats.tokens_prefilled += batch.num_tokens
            return batch
        batch = self._schedule_decode()
        if batch:
            self.stats.steps += 1
            self.stats.decode_steps += 1
            self.stats.tokens_decoded += batch.num_tokens
        return batch

    def _schedule_prefill(self) -> Batch:
        batch = Batch(is_prefill=True)
        budget = self.max_batch_tokens
        while self.waiting and len(batch) < self.max_batch_sequences and budget > 0:
            seq = self.waiting[0]
            if not seq.block_table:
                if seq.swapped is not None:
                    if not self._swap_in(seq):
                        break
                elif not self.blocks.can_allocate(seq):
                    break
            remaining = self._uncomputed_after_cache(seq)
            if remaining > budget and batch:
                break
            if not seq.block_table:
                self.stats.tokens_reused_from_cache += self.blocks.allocate(seq)
            seq.num_scheduled = min(remaining, budget)   # chunked prefill when over budget
            budget -= seq.num_scheduled
            if seq.num_computed + seq.num_scheduled >= seq.num_prompt:
                self.waiting.popleft()
                seq.status = Status.RUNNING
                self.running.append(seq)
            batch.sequences.append(seq)
        return batch

    def _uncomputed_after_cache(self, seq: Sequence) -> int:
        if seq.block_table:
            return seq.num_uncomputed
        return len(seq) - self.blocks.cached_prefix_tokens(seq)

    def _schedule_decode(self) -> Batch:
        batch = Batch(is_prefill=False)
        while self.running and len(batch) < self.max_batch_sequences:
            seq = self.running.popleft()
            while not self.blocks.can_append(seq):
                if self.running:
                    self._preempt(self.running.pop())      # youngest first
                else:
                    self._preempt(seq)
                    seq = None
                    break
            if seq is None:
                break
            self.blocks.append_slot(seq)
            seq.num_scheduled = 1
            batch.sequences.append(seq)
        self.running.extendleft(reversed(batch.sequences))
        return batch

    def _preempt(self, seq: Sequence) -> None:
        if self.swapper is not None and seq.num_computed > 0:
            self._swap_out(seq)
            return
        self.blocks.free(seq)
        seq.discard_computation()
        self.waiting.appendleft(seq)
        self.stats.preemptions += 1

    # -- swap preemption ---------------------------------------------------------
    def _swap_out(self, seq: Sequence) -> None:
        kept = -(-seq.num_computed // self.blocks.block_size)
        ids = seq.block_table[:kept]
        if hasattr(self.swapper, "read_blocks"):
            payload = self.swapper.read_blocks(ids, location="host")   # one batched offload
        else:
            payload = [self.swapper.read_block(b) for b in ids]
        seq.swapped = (payload, seq.num_computed)
        self.blocks.free(seq)                 # the blocks may be reused at once
        seq.status = Status.WAITING
        seq.num_scheduled = 0
        self.waiting.appendleft(seq)
        self.stats.preemptions += 1
        self.stats.swapped_out += 1

    def _swap_in(self, seq: Sequence) -> bool:
        if self.blocks.num_free < seq.num_blocks:
            return False
        payload, num_computed = seq.swapped
        if not self.blocks.reserve(seq, seq.num_blocks):
            raise RuntimeError("free blocks vanished during swap-in")
        kept = -(-num_computed // self.blocks.block_size)
        self.blocks.flush_pending()           # evictions above read their victims first
        if hasattr(self.swapper, "write_blocks"):
            self.swapper.write_blocks(seq.block_table[:kept], payload)
        else:
            for block_id, block_payload in zip(seq.block_table[:kept], payload):
                self.swapper.write_block(block_id, block_payload)
        seq.num_computed = num_computed
        seq.swapped = None
        self.stats.swapped_in += 1
        return True

    def finish_step(self, batch: Batch, token_ids: list[int]) -> list[Sequence]:
        if len(token_ids) != len(batch):
            raise ValueError(f"expected {len(batch)} tokens, got {len(token_ids)}")
        done: list[Sequence] = []
        for seq, token_id in zip(batch.sequences, token_ids):
            seq.commit_scheduled()
            self.blocks.share_computed_blocks(seq)
            if not seq.prompt_is_fully_computed:
                continue                                   # mid-prompt chunk: no token yet
            seq.append(token_id)
            if seq.stop_reason() is not None:
                self._retire(seq)
                done.append(seq)
        return done

    def _retire(self, seq: Sequence) -> None:
        seq.status = Status.FINISHED
        self.blocks.free(seq)
        if seq in self.running:
            self.running.remove(seq)
        self.finished.append(seq)
        self.stats.finished += 1
