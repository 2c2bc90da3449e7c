"""Engine invariants around the handoff (CPU): the reference's equivalence tests
(tests/test_engine.py:104-147) on this build's scheduler and block manager, plus
swap preemption, which must give the same tokens as recompute preemption while
computing fewer tokens."""
from __future__ import annotations

import pytest

from helpers import oracle_factory

SMALL = dict(vocab_size=64, hidden_size=32, num_layers=2, num_heads=4, num_kv_heads=2,
             head_dim=8, intermediate_size=64)


def engine(**kw):
    from iekv.engine.engine import Engine, EngineConfig
    from iekv.engine.toy_model import ModelConfig, ToyTransformer

    cfg = dict(block_size=8, num_blocks=256, max_batch_tokens=128)
    cfg.update(kw)
    return Engine(ToyTransformer(ModelConfig(**SMALL), seed=0, device="cpu"),
                  EngineConfig(**cfg), copier_factory=oracle_factory)


def test_batched_generation_matches_one_at_a_time():
    prompts = [[1, 2, 3], [9, 8, 7, 6], [4, 4, 4, 4, 4, 4]]
    batch = engine()
    together = batch.generate(prompts, max_new_tokens=5, temperature=0.0)
    apart = [engine().generate([p], max_new_tokens=5, temperature=0.0)[0] for p in prompts]
    assert together == apart
    # every finished request gave its blocks back (tests/test_engine.py:170-173)
    assert batch.blocks.num_free == batch.blocks.num_total


def test_chunked_prefill_does_not_change_the_output():
    prompt = [list(range(40))]
    whole = engine(max_batch_tokens=512).generate(prompt, max_new_tokens=6, temperature=0.0)
    chunked = engine(max_batch_tokens=12).generate(prompt, max_new_tokens=6, temperature=0.0)
    assert whole == chunked


def test_prefix_cache_does_not_change_the_output():
    shared = list(range(24))
    cold = engine().generate([shared + [7]], max_new_tokens=6, temperature=0.0)
    warm = engine()
    warm.generate([shared + [1]], max_new_tokens=6, temperature=0.0)
    reused = warm.generate([shared + [7]], max_new_tokens=6, temperature=0.0)
    assert warm.blocks.blocks_reused > 0
    assert reused == cold


PROMPTS = [list(range(i, i + 12)) for i in range(4)]


def test_preemption_does_not_change_the_output():
    roomy = engine(num_blocks=256, max_batch_tokens=256)
    expected = roomy.generate(PROMPTS, max_new_tokens=10, temperature=0.0)
    # with room for every sequence, blocks are taken only as tokens need them and
    # nothing is preempted (tests/test_engine.py:162-168)
    assert roomy.scheduler.stats.preemptions == 0
    tight = engine(num_blocks=8, max_batch_tokens=256)
    assert tight.generate(PROMPTS, max_new_tokens=10, temperature=0.0) == expected
    assert tight.scheduler.stats.preemptions > 0
    assert tight.scheduler.stats.swapped_out == 0


def test_swap_preemption_keeps_tokens_and_skips_recomputation():
    expected = engine(num_blocks=256, max_batch_tokens=256).generate(PROMPTS, max_new_tokens=10,
                                                                     temperature=0.0)
    recompute = engine(num_blocks=8, max_batch_tokens=256)
    swap = engine(num_blocks=8, max_batch_tokens=256, preemption="swap")
    assert recompute.generate(PROMPTS, max_new_tokens=10, temperature=0.0) == expected
    assert swap.generate(PROMPTS, max_new_tokens=10, temperature=0.0) == expected
    st = swap.scheduler.stats
    assert st.preemptions > 0 and st.swapped_out == st.preemptions == st.swapped_in
    assert st.tokens_prefilled < recompute.scheduler.stats.tokens_prefilled
    assert swap.blocks.num_free == swap.blocks.num_total


def test_unknown_preemption_mode_is_rejected():
    with pytest.raises(ValueError):
        engine(preemption="teleport")


def test_a_pool_pair_is_one_allocation_with_the_first_pool_below():
    import torch

    from iekv.engine.pools import allocate_pool_pair

    (ak, av), (bk, bv) = allocate_pool_pair(5, 7, 4, 3, 2, 8, dtype=torch.bfloat16, device="cpu")
    assert len(ak) == len(av) == len(bk) == len(bv) == 3
    assert all(t.shape == (20, 2, 8) for t in ak + av)
    assert all(t.shape == (28, 2, 8) for t in bk + bv)
    assert all(t.is_contiguous() for t in ak + av + bk + bv)
    # one reservation: each pool is a [2, L, N*bs, H, D] slab, the second right after the first
    assert ak[0].untyped_storage().data_ptr() == bk[0].untyped_storage().data_ptr()
    first_bytes = 2 * 3 * 20 * 2 * 8 * 2
    assert bk[0].data_ptr() - ak[0].data_ptr() == first_bytes
    assert av[0].data_ptr() - ak[0].data_ptr() == 3 * 20 * 2 * 8 * 2
    assert all(not t.any() for t in ak + av + bk + bv)
    av[2].fill_(1)
    assert all(not t.any() for t in bk + bv + ak)


def test_the_engine_accepts_preallocated_caches_of_its_size():
    import torch

    from iekv.engine.engine import Engine, EngineConfig
    from iekv.engine.pools import allocate_pool
    from iekv.engine.toy_model import ModelConfig, ToyTransformer

    model = ToyTransformer(ModelConfig(**SMALL), seed=0, device="cpu")
    caches = allocate_pool(16, 8, 2, 2, 8, dtype=torch.float32, device="cpu")
    e = Engine(model, EngineConfig(block_size=8, num_blocks=16), copier_factory=oracle_factory,
               caches=caches)
    assert e.k_caches is caches[0]
    with pytest.raises(ValueError):
        Engine(model, EngineConfig(block_size=8, num_blocks=17), copier_factory=oracle_factory,
               caches=caches)
