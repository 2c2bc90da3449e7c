"""The reference's serving invariants over seeded random workloads (CPU).

The reference asserts, on fixed prompts, that splitting prefill from decode does
not change the tokens (tests/test_disaggregation.py:23-30), that the offload
tier does not (tests/test_offload.py:103-121) and that preemption does not
(tests/test_engine.py:136-147). Here the same equalities are checked on seeded
random workloads: prompts sharing a prefix, a random block size, cache dtype
and generation length, and pools from ample down to just large enough. KV bytes
move through the NumPy oracle copier, so these check the host logic (block
manager, scheduler, workers, tier, swap) against the reference's invariants,
independently of the HIP copier.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import direct_oracle_factory, oracle_factory

MODEL = dict(vocab_size=256, hidden_size=32, num_layers=2, num_heads=4, num_kv_heads=2,
             head_dim=8, intermediate_size=64)


def workload(seed):
    rng = np.random.default_rng(7000 + seed)
    bs = int(rng.choice([2, 4, 8]))
    prefix = [int(x) for x in rng.integers(0, 250, size=int(rng.integers(0, 3 * bs)))]
    prompts = [prefix + [int(x) for x in rng.integers(0, 250, size=int(rng.integers(1, 4 * bs)))]
               for _ in range(int(rng.integers(2, 6)))]
    max_new = int(rng.integers(1, 12))
    need_one = max(-(-(len(p) + max_new) // bs) for p in prompts)
    need_all = sum(-(-(len(p) + max_new) // bs) for p in prompts)
    return {
        "bs": bs, "prompts": prompts, "max_new": max_new,
        "ample": need_all + 8,
        # enough for any one sequence and for the prompts, not for everything at once
        "tight": max(need_one, sum(-(-(len(p) + 1) // bs) for p in prompts)) + int(rng.integers(0, 2)),
        "cache_dtype": [torch.float32, torch.bfloat16][int(rng.integers(2))],
        "max_batch_tokens": int(rng.choice([16, 64, 256])),
    }


def model(w):
    from iekv.engine.toy_model import ModelConfig, ToyTransformer

    return ToyTransformer(ModelConfig(**MODEL), seed=11, device="cpu", cache_dtype=w["cache_dtype"])


def config(w, num_blocks, **over):
    from iekv.engine.engine import EngineConfig

    return EngineConfig(block_size=w["bs"], num_blocks=num_blocks,
                        max_batch_tokens=w["max_batch_tokens"], **over)


def colocated(w, num_blocks, **over):
    from iekv.engine.engine import Engine

    return Engine(model(w), config(w, num_blocks, **over), copier_factory=oracle_factory).generate(
        w["prompts"], max_new_tokens=w["max_new"], temperature=0.0)


@pytest.mark.parametrize("seed", range(10))
def test_splitting_prefill_from_decode_never_changes_the_tokens(seed):
    from iekv.serve.disaggregated import DisaggregatedEngine

    w = workload(seed)
    want = colocated(w, w["ample"])
    for kw in (dict(mode="pack", copier_factory=oracle_factory),
               dict(mode="direct", copier_factory=direct_oracle_factory),
               dict(mode="direct", prefix_aware=True, copier_factory=direct_oracle_factory),
               dict(mode="pack", prefix_aware=True, copier_factory=oracle_factory)):
        engine = DisaggregatedEngine(model(w), config(w, w["ample"]), **kw)
        got = engine.generate(w["prompts"], max_new_tokens=w["max_new"], temperature=0.0)
        assert got == want, (seed, kw)
    engine = DisaggregatedEngine(model(w), config(w, w["ample"]), mode="direct",
                                 copier_factory=direct_oracle_factory)
    got = engine.generate(w["prompts"], max_new_tokens=w["max_new"], temperature=0.0,
                          batch_moves=True)
    assert got == want, (seed, "batch_moves")
    for kw in (dict(), dict(prefix_aware=True)):
        engine = DisaggregatedEngine(model(w), config(w, w["ample"]), mode="pack",
                                     copier_factory=oracle_factory, **kw)
        got = engine.generate(w["prompts"], max_new_tokens=w["max_new"], temperature=0.0,
                              batch_moves=True)
        assert got == want, (seed, "pack batch_moves", kw)


@pytest.mark.parametrize("seed", range(10))
def test_offload_and_preemption_never_change_the_tokens(seed):
    w = workload(seed)
    want = colocated(w, w["ample"])
    for over in (dict(), dict(offload_blocks=4), dict(offload_blocks=64),
                 dict(preemption="swap"), dict(preemption="swap", offload_blocks=16)):
        assert colocated(w, w["tight"], **over) == want, (seed, over, w["tight"])


def test_the_tight_pools_force_preemption_swaps_and_tier_restores():
    """The workloads above are not quiet: in their tight pools the engine
    preempts (by swap and by recompute), evicts into the tier and restores
    from it."""
    from iekv.engine.engine import Engine

    preempted = swapped = restored = 0
    for seed in range(10):
        w = workload(seed)
        for over in (dict(offload_blocks=64), dict(preemption="swap")):
            engine = Engine(model(w), config(w, w["tight"], **over), copier_factory=oracle_factory)
            engine.generate(w["prompts"], max_new_tokens=w["max_new"], temperature=0.0)
            preempted += engine.scheduler.stats.preemptions
            swapped += engine.scheduler.stats.swapped_out
            restored += engine.blocks.stats()["restored"]
    assert preempted > swapped > 0 and restored > 0, (preempted, swapped, restored)
