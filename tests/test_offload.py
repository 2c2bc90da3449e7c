"""The offload tier and its wiring into the block manager (CPU).

``KVTier`` is checked against a brute-force LRU model over random admit / take
/ peek traces (the reference's rules, ie/core/offload.py:26-69: reject
everything at capacity 0, refresh without replacing on a repeated key, evict
least-recent first), then through the block manager with a copier that moves
strings, and finally against the exact offload / restore trace the reference
recorded for a small engine run (tests/golden/offload.json).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden
from helpers import LoggingCopier, StringCopier, oracle_factory
from iekv.core.block_manager import BlockManager, chain_hash
from iekv.core.offload import KVTier
from iekv.core.sequence import Sequence


class LruModel:
    """Least-recent-first list of [key, tokens, payload] with the tier's counters."""

    def __init__(self, capacity):
        self.capacity, self.items = capacity, []
        self.counts = {"admitted": 0, "restored": 0, "evicted": 0, "rejected": 0}

    def find(self, key):
        return next((i for i, item in enumerate(self.items) if item[0] == key), None)

    def admit(self, key, tokens, payload):
        if self.capacity == 0:
            self.counts["rejected"] += 1
            return False
        at = self.find(key)
        if at is not None:
            self.items.append(self.items.pop(at))
            return True
        while len(self.items) >= self.capacity:
            self.items.pop(0)
            self.counts["evicted"] += 1
        self.items.append([key, list(tokens), payload])
        self.counts["admitted"] += 1
        return True

    def take(self, key):
        at = self.find(key)
        if at is None:
            return None
        self.counts["restored"] += 1
        _, tokens, payload = self.items.pop(at)
        return tokens, payload


@pytest.mark.parametrize("capacity", [0, 1, 2, 5])
@pytest.mark.parametrize("seed", [0, 1])
def test_the_tier_follows_a_brute_force_lru_model(capacity, seed):
    rng = np.random.default_rng(seed)
    tier, model = KVTier(capacity), LruModel(capacity)
    keys = [f"k{i}" for i in range(8)]
    for step in range(600):
        key = keys[int(rng.integers(len(keys)))]
        tokens = [int(t) for t in rng.integers(0, 3, size=2)]
        op = rng.random()
        if op < 0.55:
            assert tier.admit(key, tokens, f"p{step}") == model.admit(key, tokens, f"p{step}")
        elif op < 0.8:
            assert tier.take(key) == model.take(key)
        else:
            at = model.find(key)
            want = None if at is None else tuple(model.items[at][1:])
            assert tier.peek(key) == want
            assert tier.holds(key, tokens) == (at is not None and model.items[at][1] == tokens)
        assert list(tier.entries) == [item[0] for item in model.items]
        assert len(tier) == len(model.items) and tier.is_full == (len(model.items) >= capacity)
        assert {k: getattr(tier.stats, k) for k in model.counts} == model.counts


def test_tier_edge_cases():
    with pytest.raises(ValueError):
        KVTier(capacity_blocks=-1)
    tier = KVTier(2)
    assert tier.admit("a", [1], "A") and tier.admit("b", [2], "B")
    assert tier.admit("a", [1], "A-again")          # a repeat keeps the held payload ...
    assert tier.peek("a") == ([1], "A")
    tier.admit("c", [3], "C")                       # ... and makes "b" the least recent
    assert "b" not in tier and list(tier.entries) == ["a", "c"]
    assert tier.take("missing") is None and tier.stats.restored == 0
    assert tier.take("c") == ([3], "C") and tier.stats.restore_rate == 1 / 3


def parked(manager, tokens, copier=None, payload=None):
    """Allocate ``tokens``, mark them computed, key their full blocks, write
    ``payload`` into the first block and release the sequence again."""
    s = Sequence(tokens, manager.block_size)
    manager.allocate(s)
    s.num_computed = len(tokens)
    if payload is not None:
        copier.store[s.block_table[0]] = payload
    manager.share_computed_blocks(s)
    table = list(s.block_table)
    manager.free(s)
    return table


def test_a_keyed_block_is_offloaded_when_its_block_is_claimed_again():
    copier, tier = StringCopier(), KVTier(8)
    manager = BlockManager(num_blocks=2, block_size=4, tier=tier, copier=copier)
    table = parked(manager, [1, 2, 3, 4, 5], copier, payload="first-block-kv")
    key = chain_hash([1, 2, 3, 4])
    assert len(tier) == 0 and manager.block_id_by_hash[key] == table[0]
    crowd = Sequence(list(range(50, 58)), 4)        # needs both blocks
    manager.allocate(crowd)
    # the keyed block is read exactly once, when it is claimed for the crowd
    assert copier.calls == [("read", table[0])]
    assert tier.peek(key) == ([1, 2, 3, 4], "first-block-kv")
    assert key not in manager.block_id_by_hash and tier.stats.admitted == 1
    # the partial second block was never keyed: nothing else went to the tier
    assert len(tier) == 1


def test_a_tier_hit_is_restored_into_a_fresh_block_with_its_payload():
    copier, tier = StringCopier(), KVTier(8)
    manager = BlockManager(num_blocks=2, block_size=4, tier=tier, copier=copier)
    parked(manager, [1, 2, 3, 4, 5], copier, payload="first-block-kv")
    crowd = Sequence(list(range(50, 58)), 4)
    manager.allocate(crowd)
    manager.free(crowd)
    again = Sequence([1, 2, 3, 4, 5], 4)
    assert manager.cached_prefix_tokens(again) == 4
    assert manager.allocate(again) == 4
    assert manager.blocks_restored == 1 and tier.stats.restored == 1
    assert copier.store[again.block_table[0]] == "first-block-kv"
    assert copier.calls[-1] == ("write", again.block_table[0])
    assert manager.block_id_by_hash[chain_hash([1, 2, 3, 4])] == again.block_table[0]


def run_offload_scenario(capacity, factory):
    import torch  # noqa: F401

    from iekv.engine.engine import Engine, EngineConfig
    from iekv.engine.toy_model import ModelConfig, ToyTransformer

    g = golden("offload")
    model = ToyTransformer(ModelConfig(**g["model"]), seed=g["model_seed"], device="cpu")
    engine = Engine(model, EngineConfig(block_size=16, num_blocks=12, max_batch_tokens=512,
                                        offload_blocks=capacity), copier_factory=factory)
    log: list = []
    if engine.blocks.copier is not None:
        engine.blocks.copier = LoggingCopier(engine.blocks.copier, log)
    steps = []
    for prompt in g["prompts"]:
        tokens = engine.generate([prompt], max_new_tokens=2, temperature=0.0)[0]
        steps.append({"tokens": tokens, "free_ids": list(engine.blocks.free_ids),
                      "tier_keys": list(engine.blocks.tier.entries) if engine.blocks.tier else []})
    revisit = engine.generate([g["prompts"][0]], max_new_tokens=2, temperature=0.0)[0]
    return g, engine, log, steps, revisit


@pytest.mark.parametrize("capacity", [0, 64])
def test_offload_trace_matches_the_reference(capacity):
    g, engine, log, steps, revisit = run_offload_scenario(capacity, oracle_factory)
    want = g[str(capacity)]
    assert steps == want["steps"]
    assert revisit == want["revisit"]
    assert log == want["copier_log"]
    assert engine.blocks.stats() == want["stats"]
    assert list(engine.blocks.free_ids) == want["free_ids"]
    if capacity:
        tier = engine.blocks.tier
        assert list(tier.entries) == want["tier_keys"]
        assert {k: getattr(tier.stats, k) for k in want["tier_stats"]} == want["tier_stats"]


def test_offload_does_not_change_generated_tokens():
    _, off_engine, _, _, without = run_offload_scenario(0, oracle_factory)
    _, on_engine, _, _, with_tier = run_offload_scenario(64, oracle_factory)
    assert without == with_tier
    assert off_engine.blocks.stats()["restored"] == 0
    assert on_engine.blocks.stats()["restored"] > 0
    assert on_engine.blocks.stats()["computed"] < off_engine.blocks.stats()["computed"]


def test_offload_is_off_by_default():
    from iekv.engine.engine import Engine, EngineConfig
    from iekv.engine.toy_model import ModelConfig, ToyTransformer

    model = ToyTransformer(ModelConfig(vocab_size=2048, hidden_size=32, num_layers=2,
                                       num_heads=4, num_kv_heads=2, head_dim=8,
                                       intermediate_size=64), device="cpu")
    engine = Engine(model, EngineConfig(block_size=16, num_blocks=32),
                    copier_factory=oracle_factory)
    assert not engine.blocks.offload_enabled
    assert engine.blocks.stats()["tier_held"] == 0
