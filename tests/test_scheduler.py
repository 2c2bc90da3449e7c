"""The scheduler behaviour the handoff depends on (CPU).

The disaggregation workers drive the scheduler's queues and rely on when block
tables are made: a prompt gets its blocks only when a step places it, so a prefix
published by an earlier step is visible to it, and a prompt deferred by the token
budget holds nothing meanwhile. These tests pin those rules and the step
accounting against the reference's scheduler behaviour
(ie/core/scheduler.py:38-162; its tests at tests/test_scheduler.py:190,216,228).
"""
from __future__ import annotations

import numpy as np
import pytest

from iekv.core.block_manager import BlockManager
from iekv.core.scheduler import Scheduler
from iekv.core.sequence import Sequence, Status

BS = 4


def make(num_blocks: int = 64, batch_sequences: int = 8, batch_tokens: int = 32) -> Scheduler:
    return Scheduler(BlockManager(num_blocks, BS), max_batch_sequences=batch_sequences,
                     max_batch_tokens=batch_tokens)


def request(tokens, new_tokens: int = 4) -> Sequence:
    return Sequence(list(tokens), BS, max_new_tokens=new_tokens)


def drain(sched: Scheduler, token: int = 5, limit: int = 10_000) -> int:
    """Step until nothing can run; every sampled token is ``token``."""
    steps = 0
    while sched.has_work and steps < limit:
        batch = sched.schedule()
        if not batch:
            break
        sched.finish_step(batch, [token] * len(batch))
        steps += 1
    return steps


def test_a_prompt_moves_from_waiting_to_running_to_finished():
    sched = make()
    s = request(range(1, 7), new_tokens=3)
    sched.add(s)
    assert s.status == Status.WAITING and s.block_table == []
    first = sched.schedule()
    assert first.is_prefill and first.sequences == [s] and first.num_tokens == 6
    assert s.status == Status.RUNNING and len(s.block_table) == 2
    sched.finish_step(first, [11])
    for expected in (12, 13):
        step = sched.schedule()
        assert not step.is_prefill and step.num_tokens == 1
        sched.finish_step(step, [expected])
    assert s.status == Status.FINISHED and s.token_ids[6:] == [11, 12, 13]
    assert sched.finished == [s] and not sched.has_work
    assert sched.blocks.num_free == sched.blocks.num_total


def test_a_prompt_over_the_budget_is_prefilled_in_chunks_without_a_token_between():
    sched = make(batch_tokens=5)
    s = request(range(12), new_tokens=1)
    sched.add(s)
    sizes = []
    while s.status == Status.WAITING:
        step = sched.schedule()
        sizes.append(step.num_tokens)
        sched.finish_step(step, [99])
        if s.status == Status.WAITING:
            assert len(s) == 12                # no token for a chunk mid-prompt
    assert sizes == [5, 5, 2]
    assert s.token_ids[12:] == [99]


def test_later_prompts_with_a_shared_prefix_prefill_less():
    shared = list(range(100, 132))             # 8 full blocks
    sched = make(num_blocks=128, batch_tokens=256)
    prefilled = []
    for tail in range(4):
        before = sched.stats.tokens_prefilled
        sched.add(request(shared + [tail], new_tokens=1))
        drain(sched)
        prefilled.append(sched.stats.tokens_prefilled - before)
    assert prefilled[0] == 33
    assert all(p < prefilled[0] for p in prefilled[1:])
    assert sched.stats.tokens_reused_from_cache == sum(33 - p for p in prefilled[1:])
    assert sched.stats.tokens_reused_from_cache > 0


def test_a_token_count_that_does_not_match_the_batch_is_refused():
    sched = make()
    sched.add(request([1, 2]))
    step = sched.schedule()
    computed = step.sequences[0].num_computed
    with pytest.raises(ValueError):
        sched.finish_step(step, [1, 2, 3])
    assert step.sequences[0].num_computed == computed     # nothing committed


def test_a_prompt_deferred_by_the_budget_holds_no_blocks():
    sched = make(batch_tokens=12)
    first, waiting = request(range(1, 9)), request([9] * 8)
    sched.add(first)
    sched.add(waiting)
    step = sched.schedule()
    assert step.sequences == [first]
    assert waiting.block_table == [] and waiting.status == Status.WAITING
    assert sched.blocks.num_free == sched.blocks.num_total - 2


def test_a_deferred_prompt_reuses_a_prefix_published_while_it_waited():
    sched = make(batch_tokens=12)
    prompt = list(range(1, 9))
    first, later = request(prompt, new_tokens=1), request(prompt, new_tokens=1)
    sched.add(first)
    sched.add(later)
    opening = sched.schedule()
    assert opening.sequences == [first]        # `later` does not fit the rest of the budget
    assert sched.stats.tokens_reused_from_cache == 0
    first_blocks = list(first.block_table)
    sched.finish_step(opening, [0])            # keys first's full blocks, then retires it
    warm = sched.schedule()
    assert later in warm.sequences
    # The first full block is shared; the prompt's last block is computed again.
    assert sched.stats.tokens_reused_from_cache == BS
    assert later.block_table[0] == first_blocks[0]
    assert later.num_scheduled == len(prompt) - BS


def test_a_decode_that_runs_out_of_blocks_preempts_and_both_requests_finish():
    sched = make(num_blocks=6, batch_tokens=64)
    a, b = request(range(8), new_tokens=8), request(range(50, 58), new_tokens=8)
    sched.add(a)
    sched.add(b)
    drain(sched)
    assert sched.stats.preemptions >= 1
    assert a.status == Status.FINISHED and b.status == Status.FINISHED
    assert a.num_generated == 8 and b.num_generated == 8
    assert sched.blocks.num_free == sched.blocks.num_total


@pytest.mark.parametrize("seed", range(6))
def test_random_workloads_finish_and_return_every_block(seed):
    rng = np.random.default_rng(seed)
    sched = make(num_blocks=int(rng.integers(24, 64)), batch_sequences=int(rng.integers(1, 6)),
                 batch_tokens=int(rng.integers(8, 48)))
    shared = [int(t) for t in rng.integers(0, 50, size=int(rng.integers(0, 12)))]
    reqs = []
    for _ in range(int(rng.integers(3, 10))):
        tail = [int(t) for t in rng.integers(0, 50, size=int(rng.integers(1, 20)))]
        reqs.append(request(shared + tail, new_tokens=int(rng.integers(1, 6))))
        sched.add(reqs[-1])
    drain(sched)
    assert not sched.has_work
    assert all(r.status == Status.FINISHED for r in reqs)
    assert all(r.num_generated == r.max_new_tokens for r in reqs)
    assert sched.stats.finished == len(reqs)
    assert sched.blocks.num_free == sched.blocks.num_total
