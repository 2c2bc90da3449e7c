"""Slot addressing, batch-layout sizes and per-block state of sequences and blocks (CPU).

The reference's interface on either side of the handoff (ie/core/layout.py:20-53,
ie/core/sequence.py:65-77, ie/core/block_manager.py:19-40): each check compares the
build's answer with a different formulation of the same fact (rows enumerated block
by block, running sums, token slices), or with the reference's own known answer.
"""
from __future__ import annotations

import numpy as np
import pytest

from iekv.core.block_manager import BlockManager
from iekv.core.layout import BatchLayout, build_layout, computed_range, slot_for_position
from iekv.core.scheduler import Batch
from iekv.core.sequence import Sequence


def test_slots_reproduce_the_references_gather_known_answer():
    """tests/test_paged_attention.py:54-60 of the reference gathers a 6-token context
    through block table [3, 1] with 4-token blocks and reads rows 12, 13, 14, 15, 4, 5:
    the slots of positions 0..5. A position past the table raises IndexError."""
    seq = Sequence([7] * 6, 4)
    seq.block_table = [3, 1]
    assert [slot_for_position(seq, p, 4) for p in range(6)] == [12, 13, 14, 15, 4, 5]
    with pytest.raises(IndexError):
        slot_for_position(seq, 8, 4)


@pytest.mark.parametrize("seed", range(4))
def test_slots_and_layouts_of_random_batches(seed):
    """Every scheduled token's slot is its row in the sequence's blocks laid end to
    end (rows enumerated block by block); the layout's lengths and cumulative
    lengths are the running sums of the scheduled and context tokens."""
    rng = np.random.default_rng(seed)
    bs = int(rng.choice([1, 3, 4, 16]))
    seqs = []
    for _ in range(int(rng.integers(1, 6))):
        seq = Sequence([int(t) for t in rng.integers(0, 1000, int(rng.integers(1, 60)))], bs)
        seq.block_table = [int(b) for b in rng.permutation(200)[:seq.num_blocks]]
        seq.num_computed = int(rng.integers(0, len(seq)))
        seq.num_scheduled = len(seq) - seq.num_computed
        seqs.append(seq)
    layout = build_layout(Batch(seqs, is_prefill=True), bs)
    at = 0
    for seq in seqs:
        rows = [b * bs + o for b in seq.block_table for o in range(bs)]
        for p in computed_range(seq):
            assert slot_for_position(seq, p, bs) == rows[p] == layout.slot_mapping[at]
            assert layout.positions[at] == p and layout.token_ids[at] == seq.token_ids[p]
            at += 1
    assert at == layout.num_tokens
    running_q, running_k = [0], [0]
    for seq in seqs:
        running_q.append(running_q[-1] + seq.num_scheduled)
        running_k.append(running_k[-1] + seq.num_computed + seq.num_scheduled)
    assert layout.cu_seqlens_q == running_q and layout.cu_seqlens_k == running_k
    assert layout.max_query_len == max(s.num_scheduled for s in seqs)
    assert layout.max_context_len == max(len(s) for s in seqs)
    width = max(len(s.block_table) for s in seqs)
    for row, seq in zip(layout.block_tables, seqs):
        assert row == seq.block_table + [-1] * (width - len(seq.block_table))


def test_an_empty_layout_has_zero_sizes():
    empty = BatchLayout([], [], [], [], [], [], False)
    assert empty.cu_seqlens_q == [0] and empty.cu_seqlens_k == [0]
    assert empty.max_query_len == 0 and empty.max_context_len == 0 and empty.num_tokens == 0


def test_a_step_that_schedules_no_tokens_for_a_sequence_is_refused():
    seq = Sequence([1, 2, 3], 4)
    seq.block_table = [0]
    with pytest.raises(ValueError, match="no tokens"):
        build_layout(Batch([seq]), 4)


@pytest.mark.parametrize("seed", range(4))
def test_per_block_state_of_a_sequence(seed):
    """block_is_full(i) is whether block i's token slice is a whole block (the
    reference's definition), block_is_computed(i) whether every position of the
    block has KV, num_computed_blocks how many leading blocks do; an index past
    the last block raises IndexError."""
    rng = np.random.default_rng(100 + seed)
    bs = int(rng.choice([1, 2, 5, 16]))
    seq = Sequence(list(range(int(rng.integers(1, 80)))), bs)
    seq.num_computed = int(rng.integers(0, len(seq) + 1))
    assert seq.block_size == bs
    for i in range(seq.num_blocks):
        tokens = seq.token_ids[i * bs:(i + 1) * bs]
        assert seq.block_tokens(i) == tokens
        assert seq.block_is_full(i) == (len(tokens) == bs)
        assert seq.block_is_computed(i) == all(p < seq.num_computed
                                               for p in range(i * bs, (i + 1) * bs))
    computed = [seq.block_is_computed(i) for i in range(seq.num_blocks)]
    assert seq.num_computed_blocks == (computed + [False]).index(False)
    for bad in (-1, seq.num_blocks):
        with pytest.raises(IndexError):
            seq.block_is_full(bad)


def test_block_views_report_what_each_block_holds():
    """A full computed block, once shared, holds its tokens and is shareable; the
    partial last block holds none. After the sequence is freed the shared block is
    free but keeps its tokens (the prefix cache can revive it). Views index from
    either end and iterate over every block."""
    manager = BlockManager(8, 4)
    seq = Sequence(list(range(10)), 4)
    manager.allocate(seq)
    seq.num_computed = 10
    manager.share_computed_blocks(seq)
    first, last = manager.blocks[seq.block_table[0]], manager.blocks[seq.block_table[2]]
    assert first.token_ids == [0, 1, 2, 3] and first.holds([0, 1, 2, 3])
    assert not first.holds([0, 1, 2]) and not first.is_free and first.is_shareable
    assert repr(first) == f"Block({first.id}, refs=1, shareable=True)"
    assert last.token_ids == [] and not last.is_shareable and not last.is_free
    manager.free(seq)
    assert first.is_free and first.holds([0, 1, 2, 3]) and last.is_free
    assert manager.blocks[-1].id == 7 and [b.id for b in manager.blocks] == list(range(8))
    with pytest.raises(IndexError):
        manager.blocks[8]
    assert repr(manager.free_ids).startswith("FreeList([")
