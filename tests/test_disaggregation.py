"""Disaggregated serving on the CPU, with KV bytes moved by the NumPy oracle: the
reference's serving invariants (disaggregated == colocated, whole-cache transfers,
released prefill pools, the undersized-pool failure) and the golden tables,
counters, stats and tokens the reference recorded (tests/golden/disaggregation.json).
The same flows run on the GPU through the HIP copier in test_gpu_engine.py."""
from __future__ import annotations

import pytest

from conftest import golden
from helpers import LoggingCopier, direct_oracle_factory, oracle_factory

G = golden("disaggregation")


def model():
    from iekv.engine.toy_model import ModelConfig, ToyTransformer

    return ToyTransformer(ModelConfig(**G["model"]), seed=G["model_seed"], device="cpu")


def engine_config(**over):
    from iekv.engine.engine import EngineConfig

    return EngineConfig(**{**G["engine"], **over})


def colocated(max_new_tokens=10, prompts=None):
    from iekv.engine.engine import Engine

    return Engine(model(), engine_config(), copier_factory=oracle_factory).generate(
        prompts or G["prompts"], max_new_tokens=max_new_tokens, temperature=0.0)


def split(**kw):
    from iekv.serve.disaggregated import DisaggregatedEngine

    kw.setdefault("copier_factory", oracle_factory)
    return DisaggregatedEngine(model(), engine_config(), **kw)


@pytest.mark.parametrize("new_tokens", [1, 5, 10, 12])
def test_disaggregated_serving_decodes_what_one_engine_decodes(new_tokens):
    """Prefill in one pool, hand off, decode in another: the greedy output equals one
    engine doing both, and both equal the tokens the reference produced."""
    out = split().generate(G["prompts"], max_new_tokens=new_tokens, temperature=0.0)
    assert out == colocated(new_tokens)
    if str(new_tokens) in G["disaggregated"]:
        assert out == G["disaggregated"][str(new_tokens)] == G["colocated"][str(new_tokens)]


def test_a_transfer_carries_the_whole_prompt_cache_and_one_token():
    engine = split()
    prompt = G["prompts"][0]
    transfer = engine.prefill.prefill(prompt)
    bs, cfg = G["engine"]["block_size"], G["model"]
    blocks = -(-len(prompt) // bs)
    # tile bytes: bs rows of H x D float32 values, K and V in every layer
    per_block = 2 * cfg["num_layers"] * bs * cfg["num_kv_heads"] * cfg["head_dim"] * 4
    assert (transfer.num_blocks, transfer.num_computed) == (blocks, len(prompt))
    assert transfer.token_ids[:-1] == prompt and len(transfer.token_ids) == len(prompt) + 1
    assert transfer.bytes_moved == blocks * per_block
    prefill_blocks = engine.prefill.engine.blocks
    assert prefill_blocks.num_free == prefill_blocks.num_total     # released after packing


def test_transfer_size_follows_the_prompt_length():
    engine = split()
    sizes = [engine.prefill.prefill(list(range(500, 500 + n))) for n in (1, 16, 17, 80, 100)]
    assert [t.num_blocks for t in sizes] == [1, 1, 2, 5, 7]
    per_block = sizes[0].bytes_moved
    assert [t.bytes_moved for t in sizes] == [n * per_block for n in (1, 1, 2, 5, 7)]


def test_a_request_that_is_done_on_arrival_frees_its_decode_blocks():
    engine = split()
    seq = engine.decode.admit(engine.prefill.prefill(G["prompts"][0]), max_new_tokens=1)
    assert seq.is_finished and seq.num_generated == 1
    decode_blocks = engine.decode.engine.blocks
    assert decode_blocks.num_free == decode_blocks.num_total
    assert seq in engine.decode.engine.scheduler.finished


def test_stats_account_for_every_transfer():
    engine = split()
    engine.generate(G["prompts"], max_new_tokens=10, temperature=0.0)
    st = engine.stats
    assert {k: getattr(st, k) for k in G["stats_10"]} == G["stats_10"]
    assert engine.decode.engine.blocks.stats() == G["decode_block_stats_10"]
    assert list(engine.decode.engine.blocks.free_ids)[:64] == G["decode_free_ids_10"]


def test_an_undersized_decode_pool_raises_and_leaves_what_the_reference_leaves():
    """The reference raises RuntimeError when reserve() runs dry and does not undo
    anything (ie/serve/disaggregated.py:76-79): the partial table and the waiting
    entry stay. The golden fixture recorded that state."""
    from iekv.serve.disaggregated import DecodeWorker

    engine = split()
    engine.decode = DecodeWorker(model(), engine_config(num_blocks=2),
                                 copier_factory=oracle_factory)
    transfer = engine.prefill.prefill(list(range(300, 400)))
    with pytest.raises(RuntimeError, match="no room"):
        engine.decode.admit(transfer, max_new_tokens=4)
    want = G["undersized"]
    waiting = list(engine.decode.engine.scheduler.waiting)
    assert transfer.num_blocks == want["transfer_blocks"]
    assert len(waiting) == want["waiting"]
    assert waiting[0].block_table == want["leaked_table"]
    assert engine.decode.engine.blocks.num_free == want["decode_free"]


def record(engine):
    log: list = []
    engine.prefill.copier = LoggingCopier(engine.prefill.copier, log)
    engine.decode.copier = LoggingCopier(engine.decode.copier, log)
    return log


def test_block_tables_counters_and_trace_match_the_reference():
    engine = split()
    log = record(engine)
    for prompt, want in zip(G["prompts"], G["requests"]):
        before = len(log)
        transfer = engine.prefill.prefill(prompt, 0.0)
        src = [b for op, b in log[before:] if op == "r"]
        seq = engine.decode.admit(transfer, 10, 0.0)
        assert src == want["src_table"]
        assert seq.block_table == want["dst_table"]
        assert transfer.num_blocks == want["num_blocks"]
        assert transfer.num_computed == want["num_computed"]
        assert transfer.token_ids == want["token_ids"]
        assert transfer.bytes_moved == want["bytes_moved"]
        assert engine.prefill.engine.blocks.num_free == want["prefill_free_after"]
    assert log == G["copier_log"]
    for side, copier in (("prefill_copier", engine.prefill.copier),
                         ("decode_copier", engine.decode.copier)):
        got = {k: getattr(copier, k) for k in ("blocks_read", "blocks_written", "bytes_moved")}
        assert got == G[side]
    assert engine.decode.engine.blocks.num_free == G["decode_free_after_admit"]
    assert list(engine.decode.engine.blocks.free_ids)[:64] == G["decode_free_ids_after_admit"]


def test_direct_mode_gives_the_same_tables_and_tokens():
    engine = split(mode="direct", copier_factory=direct_oracle_factory)
    seqs = []
    for prompt, want in zip(G["prompts"], G["requests"]):
        transfer = engine.prefill.prefill(prompt, 0.0)
        assert transfer.block_payloads is None and transfer.source.block_ids == want["src_table"]
        # The prefill blocks stay held until the copy is enqueued.
        assert engine.prefill.engine.blocks.num_free < engine.prefill.engine.blocks.num_total
        seq = engine.decode.admit(transfer, 10, 0.0)
        assert seq.block_table == want["dst_table"]
        assert transfer.bytes_moved == want["bytes_moved"]
        assert engine.prefill.engine.blocks.num_free == engine.prefill.engine.blocks.num_total
        seqs.append(seq)
    out = split(mode="direct", copier_factory=direct_oracle_factory).generate(
        G["prompts"], max_new_tokens=10, temperature=0.0)
    assert out == G["disaggregated"]["10"]


def test_prefix_aware_admit_moves_only_the_unshared_blocks():
    prefix = list(range(1000, 1064))                   # 4 full blocks of 16
    prompts = [prefix + list(range(1200 + 40 * i, 1200 + 40 * i + 20 + 7 * i))
               for i in range(4)]
    plain = split().generate(prompts, max_new_tokens=6, temperature=0.0)
    engine = split(prefix_aware=True)
    out = engine.generate(prompts, max_new_tokens=6, temperature=0.0)
    assert out == plain
    # The first request moves everything; the others find the 4 prefix blocks resident.
    assert engine.stats.blocks_skipped == 4 * (len(prompts) - 1)
    assert engine.stats.blocks_transferred == (
        sum(-(-len(p) // 16) for p in prompts) - engine.stats.blocks_skipped)


def test_prefix_aware_admit_shares_blocks_by_reference_count():
    prefix = list(range(1000, 1064))
    engine = split(prefix_aware=True)
    first = engine.handoff(prefix + [1, 2, 3], max_new_tokens=8)
    second = engine.handoff(prefix + [4, 5, 6, 7], max_new_tokens=8)
    assert second.block_table[:4] == first.block_table[:4]
    blocks = engine.decode.engine.blocks
    assert all(blocks.blocks[b].ref_count == 2 for b in first.block_table[:4])
    assert set(second.block_table[4:]).isdisjoint(first.block_table)


def test_batched_moves_keep_tables_and_tokens():
    sequential = split(mode="direct", copier_factory=direct_oracle_factory)
    expected = sequential.generate(G["prompts"], max_new_tokens=10, temperature=0.0)
    batched = split(mode="direct", copier_factory=direct_oracle_factory)
    pending: list = []
    seqs = [batched.handoff(p, 10, 0.0, pending) for p in G["prompts"]]
    assert [s.block_table for s in seqs] == [r["dst_table"] for r in G["requests"]]
    assert len(pending) == len(G["prompts"])
    # the prefill blocks stay held until the one combined copy
    assert batched.prefill.engine.blocks.num_free < batched.prefill.engine.blocks.num_total
    moved = batched.flush_moves(pending)
    assert moved == sum(r["num_blocks"] for r in G["requests"])
    assert batched.prefill.engine.blocks.num_free == batched.prefill.engine.blocks.num_total
    fresh = split(mode="direct", copier_factory=direct_oracle_factory)
    assert fresh.generate(G["prompts"], max_new_tokens=10, temperature=0.0,
                          batch_moves=True) == expected == G["disaggregated"]["10"]


def test_batched_moves_flush_early_when_the_prefill_pool_is_short():
    from iekv.serve.disaggregated import DisaggregatedEngine

    prompts = [list(range(100 + 40 * i, 100 + 40 * i + 70)) for i in range(6)]   # 5 blocks each
    roomy = split(mode="direct", copier_factory=direct_oracle_factory)
    expected = roomy.generate(prompts, max_new_tokens=4, temperature=0.0)
    tight = DisaggregatedEngine(model(), engine_config(), mode="direct",
                                copier_factory=direct_oracle_factory)
    from iekv.serve.disaggregated import PrefillWorker
    tight.prefill = PrefillWorker(model(), engine_config(num_blocks=12), mode="direct",
                                  copier_factory=direct_oracle_factory)
    assert tight.generate(prompts, max_new_tokens=4, temperature=0.0,
                          batch_moves=True) == expected


def test_a_batched_request_finished_on_arrival_leaves_no_shared_prefix():
    """With batched moves, a request that finishes on arrival is never copied, so its
    blocks must not be offered for prefix sharing: a later request with the same
    prefix moves those blocks itself and decodes as if alone."""
    from iekv.core.sequence import Status

    prefix = list(range(1000, 1064))                   # 4 full blocks of 16
    first, second = prefix + [1, 2, 3], prefix + [4, 5, 6, 7]
    want = split().generate([second], max_new_tokens=6, temperature=0.0)[0]
    engine = split(mode="direct", prefix_aware=True, copier_factory=direct_oracle_factory)
    pending: list = []
    done = engine.handoff(first, 1, 0.0, pending)
    assert done.status == Status.FINISHED and not pending
    seq = engine.handoff(second, 6, 0.0, pending)
    assert engine.stats.blocks_skipped == 0
    engine.flush_moves(pending)
    engine.decode_until_done()
    assert seq.token_ids[seq.num_prompt:] == want


def test_batched_pack_moves_keep_the_reference_reads_and_defer_the_writes():
    """Pack mode with batched moves: every prompt is packed and its prefill blocks
    freed as the reference does (the same source tables and free counts), admission
    reserves the same destination tables, and the writes wait for one flush. The
    trace then holds the reference's calls, its reads in order and all writes after
    them, and the tokens are the reference's."""
    engine = split()
    log = record(engine)
    pending: list = []
    seqs = []
    for prompt, want in zip(G["prompts"], G["requests"]):
        before = len(log)
        seqs.append(engine.handoff(prompt, 10, 0.0, pending))
        assert [b for op, b in log[before:] if op == "r"] == want["src_table"]
        assert all(op == "r" for op, _ in log[before:])
        assert seqs[-1].block_table == want["dst_table"]
        assert engine.prefill.engine.blocks.num_free == want["prefill_free_after"]
    assert len(pending) == len(G["prompts"])
    before = len(log)
    assert engine.flush_moves(pending) == sum(r["num_blocks"] for r in G["requests"])
    assert log[before:] == [["w", b] for r in G["requests"] for b in r["dst_table"]]
    assert sorted(map(tuple, log)) == sorted(map(tuple, G["copier_log"]))
    engine.decode_until_done()
    assert [s.token_ids[s.num_prompt:] for s in seqs] == G["disaggregated"]["10"]
    assert split().generate(G["prompts"], max_new_tokens=10, temperature=0.0,
                            batch_moves=True) == G["disaggregated"]["10"]


def test_the_two_pools_share_one_reservation_with_prefill_first():
    """With a model that can allocate a pool pair, the workers' pools are one
    allocation, prefill's below decode's; tables and tokens are unchanged, and
    separate allocations (paired_pools=False) give the same output."""
    paired = split()
    pk, dk = paired.prefill.engine.k_caches, paired.decode.engine.k_caches
    assert pk[0].untyped_storage().data_ptr() == dk[0].untyped_storage().data_ptr()
    assert pk[0].data_ptr() < dk[0].data_ptr()
    apart = split(paired_pools=False)
    assert apart.prefill.engine.k_caches[0].untyped_storage().data_ptr() != \
        apart.decode.engine.k_caches[0].untyped_storage().data_ptr()
    want = G["disaggregated"]["10"]
    assert paired.generate(G["prompts"], max_new_tokens=10, temperature=0.0) == want
    assert apart.generate(G["prompts"], max_new_tokens=10, temperature=0.0) == want


def test_the_halved_rotary_form_is_the_interleaved_one_on_reordered_pairs():
    """ModelConfig.rope_halved (the reference's option, ie/model/transformer.py:24)
    rotates the pairs (i, i + D/2) of a head instead of (2i, 2i + 1): reordering the
    head so those pairs sit side by side, applying the interleaved form and undoing
    the reordering gives the halved form. A model built with it serves
    disaggregated exactly as it serves colocated."""
    import torch

    from iekv.engine.engine import Engine
    from iekv.engine.toy_model import ModelConfig, ToyTransformer, _rope
    from iekv.serve.disaggregated import DisaggregatedEngine

    gen = torch.Generator().manual_seed(5)
    d, positions = 8, torch.tensor([0, 3, 7, 2])
    x = torch.randn(4, 2, d, generator=gen)
    angles = torch.randn(16, d // 2, generator=gen)
    cos, sin = torch.cos(angles), torch.sin(angles)
    order = torch.stack([torch.arange(d // 2), torch.arange(d // 2) + d // 2], 1).reshape(-1)
    undo = torch.argsort(order)
    halved = _rope(x, positions, cos, sin, True)
    via_pairs = _rope(x[..., order], positions, cos, sin, False)[..., undo]
    assert torch.allclose(halved, via_pairs, atol=1e-6)
    assert not torch.allclose(halved, _rope(x, positions, cos, sin, False), atol=1e-3)
    config = ModelConfig(**{**G["model"], "rope_halved": True})
    make = lambda: ToyTransformer(config, seed=G["model_seed"], device="cpu")
    alone = Engine(make(), engine_config(), copier_factory=oracle_factory).generate(
        G["prompts"], max_new_tokens=6, temperature=0.0)
    apart = DisaggregatedEngine(make(), engine_config(), copier_factory=oracle_factory).generate(
        G["prompts"], max_new_tokens=6, temperature=0.0)
    assert apart == alone
