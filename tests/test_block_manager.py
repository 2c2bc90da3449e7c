"""The block manager: free list, allocation geometry, prefix keys and sharing (CPU).

What is pinned here is the behaviour the handoff's destination tables depend
on (ie/core/block_manager.py:43-226): ids leave the free list at the front and
come back at the back, a freed table comes back last block first, a revived
block leaves from the middle, prefix keys are blake2b-128 chains, and a
prefix plan shares only full, computed blocks other than the last. Long random
traces are checked against the brute-force free-list model in oracle/, and
the golden traces in test_disaggregation / test_offload check the same rules
against tables the reference itself produced.
"""
from __future__ import annotations

import hashlib

import numpy as np
import pytest

from iekv.core.block_manager import BlockManager, FreeList, chain_hash
from iekv.core.sequence import Sequence
from oracle.block_ids import FreeListModel


def cached(bm: BlockManager, tokens: list[int]) -> Sequence:
    """A sequence that was allocated, fully computed and keyed (a finished prefill)."""
    s = Sequence(tokens, bm.block_size)
    bm.allocate(s)
    s.num_computed = len(tokens)
    bm.share_computed_blocks(s)
    return s


# -- the free list ------------------------------------------------------------------
@pytest.mark.parametrize("seed", range(4))
def test_free_list_matches_a_python_list_under_random_operations(seed):
    rng = np.random.default_rng(seed)
    n = 50
    fl, model = FreeList(n), list(range(n))
    for _ in range(2000):
        op = rng.integers(4)
        if op == 0 and model:
            assert fl.pop_front() == model.pop(0)
        elif op == 1 and len(model) < n:
            b = int(rng.choice(sorted(set(range(n)) - set(model))))
            fl.push_back(b)
            model.append(b)
        elif op == 2 and model:
            b = int(rng.choice(model))
            fl.discard(b)
            model.remove(b)
        elif op == 3 and model:
            order = [int(b) for b in rng.permutation(model)]
            fl.reorder(order)
            model = order
        assert list(fl) == model and len(fl) == len(model)
        probe = int(rng.integers(n))
        assert (probe in fl) == (probe in model)
        assert (np.int64(probe) in fl) == (probe in model)


def test_free_list_refuses_inconsistent_operations():
    fl = FreeList(4)
    with pytest.raises(ValueError):
        fl.push_back(2)                    # already free
    fl.discard(2)
    with pytest.raises(ValueError):
        fl.discard(2)                      # not free any more
    with pytest.raises(ValueError):
        fl.reorder([0, 1, 2])              # 2 is not free
    with pytest.raises(ValueError):
        fl.reorder([0, 0, 1])
    assert [fl.pop_front() for _ in range(3)] == [0, 1, 3]
    with pytest.raises(IndexError):
        fl.pop_front()


# -- allocation geometry ------------------------------------------------------------------
@pytest.mark.parametrize("bs", [1, 3, 4, 16])
def test_a_table_has_one_block_per_started_block_of_tokens(bs):
    bm = BlockManager(num_blocks=64, block_size=bs)
    for n in range(1, 5 * bs + 2):
        s = Sequence(list(range(100, 100 + n)), bs)
        bm.allocate(s)
        assert len(s.block_table) == -(-n // bs) == s.num_blocks
        assert 0 <= len(s.block_table) * bs - n < bs           # at most one partial block
        assert bm.num_free == 64 - len(s.block_table)
        bm.free(s)
        assert bm.num_free == 64 and s.block_table == [] and s.num_computed == 0


def test_a_sequence_the_pool_cannot_hold_is_refused_without_side_effects():
    bm = BlockManager(num_blocks=3, block_size=4)
    s = Sequence(list(range(13)), 4)                # 4 blocks
    assert not bm.can_allocate(s)
    with pytest.raises(RuntimeError, match="no capacity"):
        bm.allocate(s)
    assert s.block_table == [] and list(bm.free_ids) == [0, 1, 2]
    with pytest.raises(RuntimeError, match="already holds"):
        t = Sequence([1], 4)
        bm.allocate(t)
        bm.allocate(t)


def test_decode_growth_takes_a_block_only_when_a_token_starts_one():
    bm = BlockManager(num_blocks=3, block_size=4)
    s = Sequence([7, 7, 7], 4)
    bm.allocate(s)
    grown = []
    for token in range(6):                          # positions 3..8 of the sequence
        s.append(token)
        assert bm.can_append(s)
        before = bm.num_free
        bm.append_slot(s)
        grown.append(before - bm.num_free)
    assert grown == [0, 1, 0, 0, 0, 1]              # positions 4 and 8 start blocks
    for token in range(4):                          # positions 9..12: 12 needs a 4th block
        s.append(token)
    assert bm.num_free == 0 and not bm.can_append(s)
    with pytest.raises(RuntimeError, match="no free block"):
        bm.append_slot(s)


def test_reserve_stops_at_an_empty_pool_and_keeps_what_it_claimed():
    bm = BlockManager(num_blocks=3, block_size=4)
    s = Sequence(list(range(40)), 4)
    assert bm.reserve(s, 5) is False
    assert s.block_table == [0, 1, 2] and bm.num_free == 0
    t = Sequence([1], 4)
    assert bm.reserve(t, 0) is True and t.block_table == []


# -- prefix keys --------------------------------------------------------------------------
def test_prefix_keys_are_blake2b_128_chains():
    first = chain_hash([1, 2, 3, 4])
    assert first == hashlib.blake2b(b"1,2,3,4", digest_size=16).hexdigest()
    second = chain_hash([5, 6, 7, 8], first)
    assert second == hashlib.blake2b(f"{first}|5,6,7,8".encode(), digest_size=16).hexdigest()
    assert chain_hash([5, 6, 7, 8], chain_hash([9, 9, 9, 9])) != second   # depends on the parent
    assert len(first) == 32 and chain_hash([1, 2, 3, 4]) == first


def test_only_full_computed_blocks_get_keys():
    bm = BlockManager(num_blocks=16, block_size=4)
    s = Sequence(list(range(10)), 4)                # blocks: full, full, partial
    bm.allocate(s)
    for computed, keyed in [(0, 0), (3, 0), (4, 1), (7, 1), (8, 2), (10, 2)]:
        s.num_computed = computed
        bm.share_computed_blocks(s)
        assert len(bm.block_id_by_hash) == keyed
    keys = [bm.blocks[b].hash for b in s.block_table]
    assert keys[0] == chain_hash([0, 1, 2, 3]) and keys[1] == chain_hash([4, 5, 6, 7], keys[0])
    assert keys[2] is None


# -- sharing ---------------------------------------------------------------------------------
def test_a_cached_prefix_is_shared_by_reference_and_its_last_block_recomputed():
    bm = BlockManager(num_blocks=16, block_size=4)
    a = cached(bm, list(range(8)))                  # two full blocks
    free_before = bm.num_free
    b = Sequence(list(range(8)) + [99], 4)
    assert bm.cached_prefix_tokens(b) == 8
    assert bm.allocate(b) == 8 == b.num_computed
    assert b.block_table[:2] == a.block_table and b.block_table[2] not in a.block_table
    assert [bm.blocks[x].ref_count for x in a.block_table] == [2, 2]
    assert bm.num_free == free_before - 1
    # The same prompt again: its last block is recomputed, never shared.
    c = Sequence(list(range(8)), 4)
    assert bm.allocate(c) == 4
    assert c.block_table[0] == a.block_table[0] and c.block_table[1] != a.block_table[1]
    assert c.num_uncomputed == 4
    st = bm.stats()
    assert (st["reused"], st["computed"], st["shareable"]) == (3, 4, 2)
    assert st["reuse_rate"] == round(3 / 7, 4)


def test_a_shared_block_returns_to_the_free_list_with_its_last_owner():
    bm = BlockManager(num_blocks=8, block_size=4)
    a = cached(bm, [1, 2, 3, 4, 5])
    b = Sequence([1, 2, 3, 4, 6], 4)
    bm.allocate(b)
    shared = a.block_table[0]
    bm.free(a)
    assert bm.blocks[shared].ref_count == 1 and shared not in bm.free_ids
    bm.free(b)
    assert bm.blocks[shared].ref_count == 0 and shared in bm.free_ids
    assert bm.blocks[shared].is_shareable          # keyed, so a later request can revive it


def test_a_freed_keyed_block_is_revived_from_the_middle_of_the_free_list():
    bm = BlockManager(num_blocks=6, block_size=2)
    a = cached(bm, [1, 2, 3, 4, 5])                 # blocks 0, 1 keyed; 2 partial
    bm.free(a)                                      # released last first: 2, 1, 0
    assert list(bm.free_ids) == [3, 4, 5, 2, 1, 0]
    b = Sequence([1, 2, 3, 4, 9], 2)
    assert bm.allocate(b) == 4
    assert b.block_table == [0, 1, 3]               # 0 and 1 revived, 3 from the front
    assert list(bm.free_ids) == [4, 5, 2]


def test_a_divergence_ends_sharing_at_the_block_it_falls_in():
    bm = BlockManager(num_blocks=16, block_size=4)
    a = cached(bm, list(range(12)))
    same_first = Sequence([0, 1, 2, 3, 4, 5, 99, 7, 8, 9, 10, 11, 12], 4)
    assert bm.allocate(same_first) == 4
    assert same_first.block_table[0] == a.block_table[0]
    assert not set(same_first.block_table[1:]) & set(a.block_table)
    other = Sequence([0, 1, 2, 99] + list(range(4, 13)), 4)
    assert bm.allocate(other) == 0 and not set(other.block_table) & set(a.block_table)


def test_a_reclaimed_block_drops_its_key():
    bm = BlockManager(num_blocks=2, block_size=4)
    a = cached(bm, [1, 2, 3, 4])
    key = chain_hash([1, 2, 3, 4])
    assert bm.block_id_by_hash[key] == a.block_table[0]
    bm.free(a)
    filler = Sequence(list(range(100, 108)), 4)    # takes both blocks, the keyed one too
    bm.allocate(filler)
    assert key not in bm.block_id_by_hash and bm.block_id_by_hash.get(key) is None
    bm.free(filler)
    assert bm.allocate(Sequence([1, 2, 3, 4, 5], 4)) == 0


def test_a_block_rekeyed_for_new_tokens_leaves_the_old_key_behind():
    bm = BlockManager(num_blocks=4, block_size=2)
    s = Sequence([1, 2, 3], 2)
    bm.allocate(s)
    s.num_computed = 2
    bm.share_computed_blocks(s)
    old = chain_hash([1, 2])
    assert bm.block_id_by_hash == {old: s.block_table[0]}
    s.token_ids[:2] = [5, 6]                         # the same block now stands for 5, 6
    bm.share_computed_blocks(s)
    assert bm.block_id_by_hash == {chain_hash([5, 6]): s.block_table[0]}


# -- long random traces against the brute-force model ---------------------------------------
@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_reserve_share_and_free_follow_the_free_list_model(seed):
    """Destination ids of long random traces of reserve, revive-by-prefix and free equal
    the brute-force model's (oracle/block_ids.py), as does the free list after every step."""
    rng = np.random.default_rng(seed)
    pool, bs = 97, 4
    bm = BlockManager(num_blocks=pool, block_size=bs)
    model = FreeListModel(pool)
    live: list[tuple[Sequence, list[int]]] = []
    prefix = cached(bm, list(range(1000, 1000 + 2 * bs)))       # two keyed blocks
    model_prefix = [model.claim(), model.claim()]
    assert prefix.block_table == model_prefix
    for _ in range(500):
        r = rng.random()
        if live and (r < 0.4 or bm.num_free < 10):
            s, table = live.pop(int(rng.integers(len(live))))
            bm.free(s)
            model.release_table(table)
        elif r < 0.55 and bm.num_free >= 3:
            # a request that shares the two keyed prefix blocks and computes its last block
            s = Sequence(list(range(1000, 1000 + 2 * bs)) + [int(rng.integers(50))], bs)
            assert bm.allocate(s) == 2 * bs
            table = []
            for b in prefix.block_table[:2]:
                model.share(b)
                table.append(b)
            table.append(model.claim())
            assert s.block_table == table
            live.append((s, table))
        else:
            n = int(rng.integers(1, 9))
            s = Sequence(list(range(n * bs)), bs)
            table: list[int] = []
            ok = bm.reserve(s, n)
            assert ok == model.reserve(table, n) and s.block_table == table
            if ok:
                live.append((s, table))
            else:
                bm.free(s)
                model.release_table(table)
        assert list(bm.free_ids) == model.free
