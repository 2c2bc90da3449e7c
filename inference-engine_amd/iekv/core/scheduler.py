"""Prefill-first continuous-batching scheduler.

The handoff observes only part of the scheduler, and that part keeps the
reference's rules (ie/core/scheduler.py:38-162) so block tables and tokens
match it: queue transitions (``waiting`` -> ``running`` -> ``finished``,
which the disaggregation workers also drive by hand), a step that prefills
whenever some waiting prompt can start or continue and decodes otherwise,
chunked prefill under a token budget, decode-time growth of block tables
(``append_slot``), preemption of the most recently scheduled running
sequence when a decode step needs a block the pool lacks, and keying of the
computed blocks after every step.

A step is built by one of two phases, :meth:`Scheduler._prefill_phase` and
:meth:`Scheduler._decode_phase`; preemption has one policy,
:meth:`Scheduler._make_room`.

With a ``swapper`` (a copier whose payloads live in host memory) preemption
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
    """The sequences one step computes, and whether it is a prefill step."""

    sequences: list[Sequence] = field(default_factory=list)
    is_prefill: bool = False

    @property
    def num_tokens(self) -> int:
        return sum(s.num_scheduled for s in self.sequences)

    def __len__(self) -> int:
        return len(self.sequences)

    def __bool__(self) -> bool:
        return len(self.sequences) > 0


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
    """Queues of one engine's sequences and the policy that batches them."""

    def __init__(self, block_manager: BlockManager, max_batch_sequences: int = 256,
                 max_batch_tokens: int = 8192, swapper=None) -> None:
        self.blocks = block_manager
        self.max_batch_sequences = max_batch_sequences
        self.max_batch_tokens = max_batch_tokens
        self.swapper = swapper
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()
        self.finished: list[Sequence] = []
        self.stats = SchedulerStats()

    @property
    def has_work(self) -> bool:
        return len(self.waiting) + len(self.running) > 0

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    def schedule(self) -> Batch:
        """A prefill batch if any waiting prompt can start or continue, else a decode
        batch (empty when nothing can run)."""
        batch = self._prefill_phase()
        if not batch:
            batch = self._decode_phase()
        if batch:
            st = self.stats
            st.steps += 1
            if batch.is_prefill:
                st.prefill_steps += 1
                st.tokens_prefilled += batch.num_tokens
            else:
                st.decode_steps += 1
                st.tokens_decoded += batch.num_tokens
        return batch

    # -- prefill ------------------------------------------------------------------
    def _placed(self, seq: Sequence) -> bool:
        """Make sure a waiting sequence without blocks can get them: swap its KV back
        in, or check that the pool can allocate it. False if it cannot start now."""
        if seq.block_table:
            return True
        if seq.swapped is not None:
            return self._swap_in(seq)
        return self.blocks.can_allocate(seq)

    def _prompt_work(self, seq: Sequence) -> int:
        """Tokens still to compute: those past the cached prefix for a sequence yet to
        be allocated, else those past its computed KV."""
        if seq.block_table:
            return seq.num_uncomputed
        return len(seq) - self.blocks.cached_prefix_tokens(seq)

    def _prefill_phase(self) -> Batch:
        batch = Batch(is_prefill=True)
        budget = self.max_batch_tokens
        while budget > 0 and self.waiting and len(batch) < self.max_batch_sequences:
            seq = self.waiting[0]
            if not self._placed(seq):
                break
            work = self._prompt_work(seq)
            if batch and work > budget:      # an oversized prompt starts a batch of its own
                break
            if not seq.block_table:
                self.stats.tokens_reused_from_cache += self.blocks.allocate(seq)
            seq.num_scheduled = min(work, budget)      # a chunk when over budget
            budget -= seq.num_scheduled
            batch.sequences.append(seq)
            if seq.num_computed + seq.num_scheduled >= seq.num_prompt:
                self.waiting.popleft()
                seq.status = Status.RUNNING
                self.running.append(seq)
        return batch

    # -- decode -------------------------------------------------------------------
    def _make_room(self, seq: Sequence) -> bool:
        """Preempt the most recently queued running sequences until ``seq`` can grow by
        one token; with none left, preempt ``seq`` itself and return False."""
        while not self.blocks.can_append(seq):
            if not self.running:
                self._preempt(seq)
                return False
            self._preempt(self.running.pop())
        return True

    def _decode_phase(self) -> Batch:
        batch = Batch(is_prefill=False)
        while self.running and len(batch) < self.max_batch_sequences:
            seq = self.running.popleft()
            if not self._make_room(seq):
                break
            self.blocks.append_slot(seq)
            seq.num_scheduled = 1
            batch.sequences.append(seq)
        # The batch goes back to the front of the queue, in its order.
        self.running.extendleft(reversed(batch.sequences))
        return batch

    def _preempt(self, seq: Sequence) -> None:
        self.stats.preemptions += 1
        if self.swapper is not None and seq.num_computed > 0:
            self._swap_out(seq)
        else:
            self.blocks.free(seq)
            seq.discard_computation()
        self.waiting.appendleft(seq)

    # -- swap preemption ------------------------------------------------------------
    def _swap_out(self, seq: Sequence) -> None:
        kept = seq.geometry.blocks_for(seq.num_computed)
        ids = seq.block_table[:kept]
        if hasattr(self.swapper, "read_blocks"):
            payload = self.swapper.read_blocks(ids, location="host")   # one batched offload
        else:
            payload = [self.swapper.read_block(b) for b in ids]
        seq.swapped = (payload, seq.num_computed)
        self.blocks.free(seq)                 # the blocks may be reused at once
        seq.status = Status.WAITING
        seq.num_scheduled = 0
        self.stats.swapped_out += 1

    def _swap_in(self, seq: Sequence) -> bool:
        if self.blocks.num_free < seq.num_blocks:
            return False
        payload, num_computed = seq.swapped
        if not self.blocks.reserve(seq, seq.num_blocks):
            raise RuntimeError("free blocks vanished during swap-in")
        kept = seq.geometry.blocks_for(num_computed)
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

    # -- after the forward pass -------------------------------------------------------
    def finish_step(self, batch: Batch, token_ids: list[int]) -> list[Sequence]:
        """Commit a step: record computed KV, key full blocks, append each sampled token
        to the sequences whose prompt is done, and retire those that stop. A chunk in
        the middle of a prompt gets no token."""
        if len(token_ids) != len(batch):
            raise ValueError(f"expected {len(batch)} tokens, got {len(token_ids)}")
        done: list[Sequence] = []
        for seq, token_id in zip(batch.sequences, token_ids):
            seq.commit_scheduled()
            self.blocks.share_computed_blocks(seq)
            if seq.prompt_is_fully_computed:
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
