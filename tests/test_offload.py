"""Offload tier: the reference's assertions (tests/test_offload.py:35-127) run against this
build, and the exact offload/restore trace the reference recorded (tests/golden/offload.json)."""
from __future__ import annotations

import pytest

from conftest import golden
from helpers import LoggingCopier, RecordingCopier, oracle_factory
from iekv.core.block_manager import BlockManager, chain_hash
from iekv.core.offload import KVTier
from iekv.core.sequence import Sequence

BS = 4


def seq(tokens, block_size=BS):
    return Sequence(tokens, block_size=block_size)


def test_tier_holds_and_returns_a_payload():
    tier = KVTier(capacity_blocks=4)
    assert tier.admit("k", [1, 2], "payload")
    assert "k" in tier
    assert tier.holds("k", [1, 2])
    assert not tier.holds("k", [9, 9])
    assert tier.take("k") == ([1, 2], "payload")
    assert "k" not in tier


def test_tier_evicts_the_least_recently_admitted():
    tier = KVTier(capacity_blocks=2)
    tier.admit("a", [1], "A")
    tier.admit("b", [2], "B")
    tier.admit("c", [3], "C")
    assert "a" not in tier
    assert "b" in tier and "c" in tier
    assert tier.stats.evicted == 1


def test_readmitting_a_key_keeps_the_old_payload_and_refreshes_it():
    tier = KVTier(capacity_blocks=2)
    tier.admit("a", [1], "A")
    tier.admit("b", [2], "B")
    assert tier.admit("a", [1], "A2")
    assert tier.peek("a") == ([1], "A")
    tier.admit("c", [3], "C")            # evicts "b", the least recent now
    assert "b" not in tier and "a" in tier


def test_a_zero_capacity_tier_rejects_everything():
    tier = KVTier(capacity_blocks=0)
    assert not tier.admit("a", [1], "A")
    assert tier.stats.rejected == 1
    assert len(tier) == 0


def test_tier_rejects_a_negative_capacity():
    with pytest.raises(ValueError):
        KVTier(capacity_blocks=-1)


def test_an_evicted_block_lands_in_the_tier():
    tier = KVTier(capacity_blocks=8)
    copier = RecordingCopier()
    manager = BlockManager(num_blocks=2, block_size=BS, tier=tier, copier=copier)
    first = seq([1, 2, 3, 4, 5])
    manager.allocate(first)
    first.num_computed = len(first)
    manager.share_computed_blocks(first)
    manager.free(first)
    manager.allocate(seq(list(range(50, 58))))
    assert len(tier) >= 1
    assert copier.reads >= 1


def test_a_block_restored_from_the_tier_carries_its_payload_back():
    tier = KVTier(capacity_blocks=8)
    copier = RecordingCopier()
    manager = BlockManager(num_blocks=2, block_size=BS, tier=tier, copier=copier)
    original = seq([1, 2, 3, 4, 5])
    manager.allocate(original)
    original.num_computed = len(original)
    copier.contents[original.block_table[0]] = "the-first-block"
    manager.share_computed_blocks(original)
    manager.free(original)
    crowd = seq(list(range(50, 58)))
    manager.allocate(crowd)
    stored = chain_hash([1, 2, 3, 4])
    assert tier.holds(stored, [1, 2, 3, 4])
    assert tier.peek(stored)[1] == "the-first-block"

    manager.free(crowd)
    revisit = seq([1, 2, 3, 4, 5])
    assert manager.allocate(revisit) == BS
    assert manager.blocks_restored == 1
    assert copier.contents[revisit.block_table[0]] == "the-first-block"


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
