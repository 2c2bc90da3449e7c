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


def _prompts(seed, n, lo, hi):
    import numpy as np

    rng = np.random.default_rng(seed)
    return [[int(t) for t in rng.integers(0, SMALL["vocab_size"], size=int(rng.integers(lo, hi)))]
            for _ in range(n)]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_a_batch_decodes_as_its_requests_would_alone(seed):
    """Requests sharing the scheduler's steps get the tokens each gets alone, and the
    pool gets every block back once they finish (the reference's batching invariant,
    tests/test_engine.py:104-110, 168-171)."""
    prompts = _prompts(seed, 4, 1, 20)
    shared = engine()
    together = shared.generate(prompts, max_new_tokens=6, temperature=0.0)
    assert together == [engine().generate([p], max_new_tokens=6, temperature=0.0)[0]
                        for p in prompts]
    assert shared.blocks.num_free == shared.blocks.num_total


@pytest.mark.parametrize("budget", [5, 8, 13, 64])
def test_prefill_split_over_steps_decodes_the_same(budget):
    """A prompt prefilled a few tokens per step decodes what one full-prompt step
    decodes (tests/test_engine.py:113-122)."""
    prompt = _prompts(7, 1, 30, 31)
    one_step = engine(max_batch_tokens=1024).generate(prompt, max_new_tokens=5, temperature=0.0)
    assert engine(max_batch_tokens=budget).generate(prompt, max_new_tokens=5,
                                                    temperature=0.0) == one_step


def test_a_cached_prefix_decodes_as_a_fresh_one():
    """A prompt whose leading full blocks are already cached (shared from an earlier
    request) decodes what it decodes in an empty engine (tests/test_engine.py:124-133);
    the shared blocks are reused, not recomputed."""
    head = _prompts(11, 1, 32, 33)[0]                 # four full blocks of 8
    first, second = head + [3, 1], head + [5]
    fresh = engine().generate([second], max_new_tokens=5, temperature=0.0)
    primed = engine()
    primed.generate([first], max_new_tokens=5, temperature=0.0)
    before = primed.blocks.blocks_reused
    assert primed.generate([second], max_new_tokens=5, temperature=0.0) == fresh
    assert primed.blocks.blocks_reused - before == 4


PROMPTS = [list(range(i, i + 12)) for i in range(4)]


def test_preemption_does_not_change_the_output():
    roomy = engine(num_blocks=256, max_batch_tokens=256)
    expected = roomy.generate(PROMPTS, max_new_tokens=10, temperature=0.0)
    # with room for every sequence, blocks are taken only as tokens need them and
    # nothing is preempted (tests/test_engine.py:160-165)
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


def test_padded_pools_space_their_arrays_by_the_padding():
    """pad_blocks leaves unused blocks after every array: arrays keep the reference's
    [N*bs, H, D] shape and stay contiguous, consecutive arrays start (N + pad) tiles
    apart, and the second pool of a pair starts after the first's padded slab."""
    import torch

    from iekv.engine.pools import allocate_pool, allocate_pool_pair

    tile = 4 * 2 * 8 * 2                               # bs 4, H 2, D 8, bf16
    k, v = allocate_pool(6, 4, 3, 2, 8, dtype=torch.bfloat16, device="cpu", pad_blocks=1)
    assert all(t.shape == (24, 2, 8) and t.is_contiguous() for t in k + v)
    arrays = k + v
    for a, b in zip(arrays, arrays[1:]):
        assert b.data_ptr() - a.data_ptr() == 7 * tile
    (ak, av), (bk, bv) = allocate_pool_pair(5, 7, 4, 3, 2, 8, dtype=torch.bfloat16,
                                            device="cpu", pad_blocks=3)
    assert all(t.shape == (20, 2, 8) for t in ak + av)
    assert all(t.shape == (28, 2, 8) for t in bk + bv)
    assert av[0].data_ptr() - ak[0].data_ptr() == 3 * 8 * tile
    assert bk[0].data_ptr() - ak[0].data_ptr() == 2 * 3 * 8 * tile
    assert bk[1].data_ptr() - bk[0].data_ptr() == 10 * tile
    with pytest.raises(ValueError):
        allocate_pool(6, 4, 3, 2, 8, device="cpu", pad_blocks=-1)


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


def test_an_eos_token_ends_a_request_before_its_token_limit():
    """Greedy decoding of the same prompt, once to learn its third token, then with
    that token as eos: the request stops right after emitting it."""
    free = engine().generate([[1, 2, 3]], max_new_tokens=12, temperature=0.0)[0]
    eos = free[2]
    stop = free.index(eos) + 1                  # the first time eos comes out
    e = engine()
    seq = e.submit([1, 2, 3], max_new_tokens=12, temperature=0.0, eos_id=eos)
    e.run()
    assert seq.token_ids[3:] == free[:stop]
    assert seq.num_generated == stop < 12
    assert e.blocks.num_free == e.blocks.num_total


def test_every_block_is_free_again_when_all_requests_finish():
    e = engine()
    e.generate([[1, 2, 3], [4, 5, 6, 7], [8, 9]], max_new_tokens=4)
    assert e.blocks.num_free == e.blocks.num_total
    assert not e.scheduler.has_work


def test_a_pool_that_just_fits_the_batch_preempts_nothing():
    """Four 12-token prompts with 5 new tokens need two 8-token blocks each at the end
    (16 tokens); nine blocks hold them, since a block is taken only when a token
    will be computed in it."""
    e = engine(num_blocks=9, max_batch_tokens=256)
    prompts = [list(range(i, i + 12)) for i in range(4)]
    e.generate(prompts, max_new_tokens=5, temperature=0.0)
    assert e.scheduler.stats.preemptions == 0


def test_the_paged_view_indexes_block_tiles_without_a_copy():
    import torch

    from iekv.engine.pools import allocate_pool, paged_view

    k, v = allocate_pool(6, 4, 2, 3, 8, dtype=torch.float32, device="cpu")
    k[1].copy_(torch.arange(k[1].numel(), dtype=torch.float32).view_as(k[1]))
    view = paged_view(k[1], 4)
    assert view.shape == (6, 4, 3, 8) and view.data_ptr() == k[1].data_ptr()
    for b in range(6):
        assert torch.equal(view[b], k[1][4 * b:4 * (b + 1)])
    view[2].fill_(-1)                            # writes land in the cache itself
    assert (k[1][8:12] == -1).all() and (k[1][:8] >= 0).all()
    with pytest.raises(ValueError):
        paged_view(k[1], 5)
