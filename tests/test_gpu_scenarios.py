"""Randomized serving scenarios on the GPU: the HIP copier against a plain PyTorch one (GPU).

Each seeded scenario runs the disaggregated engine twice on the same model
weights and prompts: once with the default HIP copiers (batched packs, kernel-
argument ids, deferred offload reads, batched restores, swap pipelines) and once
with ``TorchSlotCopier``, the reference's per-block ``LayeredSlotCopier``
(ie/engine/copier.py:6-38) restated over torch tensors. Small pools force
evictions into the offload tier, restores, and preemption. Both runs must give
the same tokens, block tables, free lists, tier contents and statistics; the
model runs the same torch operations on the same bytes in both, so any
difference is a byte the handoff moved differently.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


class TorchSlotCopier:
    """ie/engine/copier.py:6-38 over torch tensors: per-block slice copies."""

    def __init__(self, k_caches, v_caches, block_size):
        self.k_caches, self.v_caches, self.block_size = k_caches, v_caches, block_size
        self.blocks_read = 0
        self.blocks_written = 0

    def _span(self, block_id):
        return slice(block_id * self.block_size, (block_id + 1) * self.block_size)

    def read_block(self, block_id):
        span = self._span(block_id)
        self.blocks_read += 1
        return ([k[span].clone() for k in self.k_caches], [v[span].clone() for v in self.v_caches])

    def write_block(self, block_id, payload):
        span = self._span(block_id)
        k_list, v_list = payload
        for cache, data in zip(self.k_caches, k_list):
            cache[span] = data
        for cache, data in zip(self.v_caches, v_list):
            cache[span] = data
        self.blocks_written += 1

    def copy_blocks(self, source, src_ids, dst_ids):
        for s, d in zip(src_ids, dst_ids):
            self.write_block(int(d), source.read_block(int(s)))


def torch_factory(k_caches, v_caches, block_size, role):
    return TorchSlotCopier(k_caches, v_caches, block_size)


def scenario(seed):
    """Three rounds of prompts sharing a prefix, the third revisiting the first; pools
    just large enough for a round's prompts (and for any one sequence's generation),
    so blocks are evicted into the tier, restored from it, and preempted."""
    rng = np.random.default_rng(5000 + seed)
    bs = int(rng.choice([4, 8, 16]))
    mode = str(rng.choice(["pack", "direct"]))
    prefix = list(range(1000, 1000 + int(rng.integers(1, 3)) * bs + int(rng.integers(0, bs))))

    def prompt():
        return prefix + [int(x) for x in rng.integers(0, 900, size=int(rng.integers(1, 3 * bs)))]

    first = [prompt() for _ in range(int(rng.integers(3, 6)))]
    second = [prompt() for _ in range(int(rng.integers(3, 6)))]
    third = [first[int(i)] for i in rng.choice(len(first), size=2, replace=False)] + [prompt()]
    rounds = [first, second, third]
    max_new = int(rng.integers(4, 17))
    need_prompts = max(sum(-(-(len(p) + 1) // bs) for p in r) for r in rounds)
    need_one = max(-(-(len(p) + max_new) // bs) for r in rounds for p in r)
    return {
        "bs": bs,
        "num_blocks": max(need_prompts, need_one) + int(rng.integers(0, 3)),
        "offload": int(rng.choice([8, 64])),
        "preemption": str(rng.choice(["recompute", "swap"])),
        "mode": mode,
        "prefix_aware": bool(rng.integers(2)),
        "batch_moves": bool(rng.integers(2)),
        "cache_dtype": [torch.float32, torch.bfloat16][int(rng.integers(2))],
        "rounds": rounds,
        "max_new": max_new,
        "max_batch_tokens": int(rng.choice([32, 256])),
    }


def run(gpu, sc, factory):
    from iekv.engine.engine import EngineConfig
    from iekv.engine.toy_model import ModelConfig, ToyTransformer
    from iekv.serve.disaggregated import DisaggregatedEngine

    model = ToyTransformer(ModelConfig(vocab_size=2048, hidden_size=32, num_layers=2,
                                       num_heads=4, num_kv_heads=2, head_dim=8,
                                       intermediate_size=64), seed=3, device=gpu,
                           cache_dtype=sc["cache_dtype"])
    config = EngineConfig(block_size=sc["bs"], num_blocks=sc["num_blocks"],
                          max_batch_tokens=sc["max_batch_tokens"],
                          offload_blocks=sc["offload"], preemption=sc["preemption"])
    engine = DisaggregatedEngine(model, config, mode=sc["mode"], prefix_aware=sc["prefix_aware"],
                                 copier_factory=factory)
    tokens = []
    try:
        for prompts in sc["rounds"]:
            tokens.append(engine.generate(prompts, max_new_tokens=sc["max_new"], temperature=0.0,
                                          batch_moves=sc["batch_moves"]))
    except RuntimeError as err:
        return {"error": str(err), "tokens": tokens}
    out = {"tokens": tokens, "disagg": [engine.stats.transfers, engine.stats.blocks_transferred,
                                        engine.stats.bytes_transferred, engine.stats.blocks_skipped]}
    for side in ("prefill", "decode"):
        eng = getattr(engine, side).engine
        out[side] = {"stats": eng.blocks.stats(), "free": list(eng.blocks.free_ids),
                     "tier": list(eng.blocks.tier.entries) if eng.blocks.tier else [],
                     "sched": (eng.scheduler.stats.preemptions, eng.scheduler.stats.swapped_out)}
    return out


@pytest.mark.parametrize("seed", range(24))
def test_random_serving_scenarios_match_a_plain_torch_copier(gpu, seed):
    from iekv.engine.engine import default_copier_factory

    sc = scenario(seed)
    hip = run(gpu, sc, default_copier_factory)
    plain = run(gpu, sc, torch_factory)
    label = {k: v for k, v in sc.items() if k != "rounds"}
    assert hip == plain, label
    assert "error" not in hip, (label, hip)


def test_the_scenarios_exercise_offload_restore_and_preemption(gpu):
    """The seeded scenarios above are not all quiet: between them they evict into
    the offload tier, restore from it, and preempt by swap and by recompute."""
    from iekv.engine.engine import default_copier_factory

    restored = tier_held = swapped = recomputed = skipped = 0
    for seed in range(24):
        sc = scenario(seed)
        out = run(gpu, sc, default_copier_factory)
        for side in ("prefill", "decode"):
            restored += out[side]["stats"]["restored"]
            tier_held += out[side]["stats"]["tier_held"]
            preempted, swaps = out[side]["sched"]
            swapped += swaps
            recomputed += preempted - swaps
        skipped += out["disagg"][3]
    assert restored > 0 and tier_held > 0, (restored, tier_held)
    assert swapped > 0 and recomputed > 0, (swapped, recomputed)
    assert skipped > 0
