"""The disaggregated engine on the GPU with the HIP copier (GPU).

The same scenarios as test_disaggregation.py / test_offload.py, now with the
model and both pools in HBM and every KV byte moved by libiekv: block tables,
counters and the protocol trace must equal the reference's golden ones, each
request's moved tiles must equal its source tiles bit for bit, and decode
output must be token-identical between colocated, pack-mode and direct-mode
serving.
"""
from __future__ import annotations

import pytest
import torch

from conftest import golden
from helpers import LoggingCopier

pytestmark = pytest.mark.gpu

G = golden("disaggregation")


def model(device, cache_dtype=torch.float32):
    from iekv.engine.toy_model import ModelConfig, ToyTransformer

    return ToyTransformer(ModelConfig(**G["model"]), seed=G["model_seed"], device=device,
                          cache_dtype=cache_dtype)


def engine_config(**over):
    from iekv.engine.engine import EngineConfig

    return EngineConfig(**{**G["engine"], **over})


def tiles(caches, block_ids, bs):
    return [torch.cat([c[b * bs:(b + 1) * bs] for b in block_ids]).view(torch.uint8)
            for c in caches]


@pytest.mark.parametrize("mode", ["pack", "direct", "queue"])
def test_handoff_tables_and_bytes_match_the_reference(gpu, mode):
    from iekv.engine.copier import HipSlotCopier
    from iekv.serve.disaggregated import DisaggregatedEngine

    engine = DisaggregatedEngine(model(gpu), engine_config(), mode=mode)
    assert isinstance(engine.prefill.copier, HipSlotCopier)
    bs = G["engine"]["block_size"]
    pk, pv = engine.prefill.engine.k_caches, engine.prefill.engine.v_caches
    dk, dv = engine.decode.engine.k_caches, engine.decode.engine.v_caches
    for prompt, want in zip(G["prompts"], G["requests"]):
        transfer = engine.prefill.prefill(prompt, 0.0)
        src_bytes = tiles(pk + pv, want["src_table"], bs)
        if mode == "pack":
            assert len(transfer.block_payloads) == want["num_blocks"]
        else:
            assert transfer.source.block_ids == want["src_table"]
        seq = engine.decode.admit(transfer, 10, 0.0)
        assert seq.block_table == want["dst_table"]
        if mode == "queue":   # the copy went through the request queue, one descriptor each
            (q,) = engine.decode._queues.values()
            q.stop()          # torch reads the pools below
        assert transfer.bytes_moved == want["bytes_moved"]
        assert transfer.token_ids == want["token_ids"]
        dst_bytes = tiles(dk + dv, seq.block_table, bs)
        for a, (s, d) in enumerate(zip(src_bytes, dst_bytes)):
            assert torch.equal(s, d), f"array {a} differs after the handoff"
    assert engine.prefill.copier.blocks_read == G["prefill_copier"]["blocks_read"]
    assert engine.decode.copier.blocks_written == G["decode_copier"]["blocks_written"]
    assert engine.decode.copier.bytes_moved == G["decode_copier"]["bytes_moved"]
    assert engine.decode.engine.blocks.num_free == G["decode_free_after_admit"]
    if mode == "queue":
        (q,) = engine.decode._queues.values()
        assert q.stats()["descriptors"] == len(G["requests"])


@pytest.mark.parametrize("cache_dtype", [torch.float32, torch.bfloat16], ids=str)
def test_decode_is_token_identical_after_the_handoff(gpu, cache_dtype):
    from iekv.engine.engine import Engine
    from iekv.serve.disaggregated import DisaggregatedEngine

    m = model(gpu, cache_dtype)
    colocated = Engine(m, engine_config()).generate(G["prompts"], max_new_tokens=10,
                                                   temperature=0.0)
    packed = DisaggregatedEngine(m, engine_config()).generate(G["prompts"], max_new_tokens=10,
                                                             temperature=0.0)
    direct = DisaggregatedEngine(m, engine_config(), mode="direct").generate(
        G["prompts"], max_new_tokens=10, temperature=0.0)
    queued = DisaggregatedEngine(m, engine_config(), mode="queue").generate(
        G["prompts"], max_new_tokens=10, temperature=0.0)
    queued_batch = DisaggregatedEngine(m, engine_config(), mode="queue").generate(
        G["prompts"], max_new_tokens=10, temperature=0.0, batch_moves=True)
    # Identity is among this build's own paths: the model's float32 products on the
    # GPU need not round like the reference's NumPy ones, so its golden tokens are
    # asserted on the CPU (test_disaggregation.py).
    assert packed == direct == queued == queued_batch == colocated


def test_the_decode_worker_refuses_a_cache_it_cannot_hold_on_gpu(gpu):
    from iekv.serve.disaggregated import DecodeWorker, DisaggregatedEngine

    m = model(gpu)
    engine = DisaggregatedEngine(m, engine_config())
    engine.decode = DecodeWorker(m, engine_config(num_blocks=2))
    transfer = engine.prefill.prefill(list(range(300, 400)))
    with pytest.raises(RuntimeError, match="no room"):
        engine.decode.admit(transfer, max_new_tokens=4)
    assert engine.decode.copier.blocks_written == 0


def test_prefix_aware_handoff_on_gpu(gpu):
    from iekv.serve.disaggregated import DisaggregatedEngine

    m = model(gpu, torch.bfloat16)
    prefix = list(range(1000, 1064))
    prompts = [prefix + list(range(1200 + 40 * i, 1200 + 40 * i + 20 + 7 * i)) for i in range(4)]
    plain = DisaggregatedEngine(m, engine_config()).generate(prompts, max_new_tokens=6)
    shared = DisaggregatedEngine(m, engine_config(), prefix_aware=True, mode="direct")
    assert shared.generate(prompts, max_new_tokens=6) == plain
    assert shared.stats.blocks_skipped == 4 * 3


@pytest.mark.parametrize("capacity", [0, 64])
def test_offload_tier_on_gpu_matches_the_reference_trace(gpu, capacity):
    from iekv.engine.copier import HipSlotCopier
    from iekv.engine.engine import Engine, EngineConfig
    from iekv.engine.toy_model import ModelConfig, ToyTransformer

    g = golden("offload")
    m = ToyTransformer(ModelConfig(**g["model"]), seed=g["model_seed"], device=gpu)
    engine = Engine(m, EngineConfig(block_size=16, num_blocks=12, max_batch_tokens=512,
                                    offload_blocks=capacity))
    log: list = []
    if capacity:
        assert isinstance(engine.blocks.copier, HipSlotCopier)
        assert engine.blocks.copier.payload_location == "host"
        engine.blocks.copier = LoggingCopier(engine.blocks.copier, log)
    for prompt in g["prompts"]:
        engine.generate([prompt], max_new_tokens=2, temperature=0.0)
    revisit = engine.generate([g["prompts"][0]], max_new_tokens=2, temperature=0.0)[0]
    want = g[str(capacity)]
    assert log == want["copier_log"]
    assert engine.blocks.stats() == want["stats"]
    assert list(engine.blocks.free_ids) == want["free_ids"]
    if capacity:
        assert list(engine.blocks.tier.entries) == want["tier_keys"]
        held = next(iter(engine.blocks.tier.entries.values()))[1]
        assert held.packed.on_host
    # Token values come from a GPU model run; their invariance is the next test's job.


def test_offload_does_not_change_tokens_on_gpu(gpu):
    from iekv.engine.engine import Engine, EngineConfig
    from iekv.engine.toy_model import ModelConfig, ToyTransformer

    g = golden("offload")
    results = []
    for capacity in (0, 64):
        m = ToyTransformer(ModelConfig(**g["model"]), seed=g["model_seed"], device=gpu,
                           cache_dtype=torch.bfloat16)
        engine = Engine(m, EngineConfig(block_size=16, num_blocks=12, max_batch_tokens=512,
                                        offload_blocks=capacity))
        for prompt in g["prompts"]:
            engine.generate([prompt], max_new_tokens=2, temperature=0.0)
        results.append((engine.generate([g["prompts"][0]], max_new_tokens=2,
                                        temperature=0.0)[0], engine.blocks.stats()))
    (without, st_off), (with_tier, st_on) = results
    assert without == with_tier
    assert st_on["restored"] > 0 and st_on["computed"] < st_off["computed"]


def test_a_restored_prefix_is_written_with_one_batched_call(gpu):
    """The golden scenario's revisit restores 3 tier blocks. The unwrapped HIP
    copier writes them with one iekv_restore_blocks after the last claim; a
    protocol-only wrapper gets the reference's three interleaved write_block
    calls. Both leave the same block tables, tier and pool bytes."""
    from iekv.engine.engine import Engine, EngineConfig
    from iekv.engine.toy_model import ModelConfig, ToyTransformer

    g = golden("offload")
    runs = []
    for wrap in (False, True):
        m = ToyTransformer(ModelConfig(**g["model"]), seed=g["model_seed"], device=gpu)
        engine = Engine(m, EngineConfig(block_size=16, num_blocks=12, max_batch_tokens=512,
                                        offload_blocks=64))
        hip = engine.blocks.copier
        if wrap:
            engine.blocks.copier = LoggingCopier(hip, [])
        for prompt in g["prompts"]:
            engine.generate([prompt], max_new_tokens=2, temperature=0.0)
        before = hip.restore_launches
        revisit = engine.generate([g["prompts"][0]], max_new_tokens=2, temperature=0.0)[0]
        torch.cuda.synchronize()
        pools = [t.clone() for t in list(hip.k_caches) + list(hip.v_caches)]
        runs.append((revisit, hip.restore_launches - before, engine.blocks.stats(),
                     list(engine.blocks.free_ids), list(engine.blocks.tier.entries), pools))
    (tok_b, launches_b, st_b, free_b, keys_b, pools_b), \
        (tok_p, launches_p, st_p, free_p, keys_p, pools_p) = runs
    assert st_b == st_p == g["64"]["stats"] and st_b["restored"] == 3
    assert launches_b == 1 and launches_p == 3
    assert free_b == free_p == g["64"]["free_ids"]
    assert keys_b == keys_p == g["64"]["tier_keys"]
    assert tok_b == tok_p
    for a, (x, y) in enumerate(zip(pools_b, pools_p)):
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), a


def test_evictions_are_offloaded_in_batches(gpu):
    from iekv.engine.engine import Engine, EngineConfig
    from iekv.engine.toy_model import ModelConfig, ToyTransformer

    g = golden("offload")
    m = ToyTransformer(ModelConfig(**g["model"]), seed=g["model_seed"], device=gpu)
    engine = Engine(m, EngineConfig(block_size=16, num_blocks=12, max_batch_tokens=512,
                                    offload_blocks=64))
    for prompt in g["prompts"]:
        engine.generate([prompt], max_new_tokens=2, temperature=0.0)
    engine.generate([g["prompts"][0]], max_new_tokens=2, temperature=0.0)
    copier = engine.copier
    reads = sum(1 for op, _ in g["64"]["copier_log"] if op == "r")
    assert copier.blocks_read == reads
    assert copier.pending_reads == 0 or copier.offload_launches > 0
    assert 0 < copier.offload_launches < reads
    print(f"{reads} evictions offloaded in {copier.offload_launches} launches "
          f"({copier.blocks_offloaded} blocks copied)")


@pytest.mark.parametrize("mode", ["pack", "direct"])
def test_a_transfer_through_the_wire_format_decodes_identically(gpu, mode):
    from iekv.serve.disaggregated import DisaggregatedEngine
    from iekv.serve.wire import from_wire, to_wire

    m = model(gpu, torch.bfloat16)
    plain = DisaggregatedEngine(m, engine_config()).generate(G["prompts"], max_new_tokens=8)
    engine = DisaggregatedEngine(m, engine_config(), mode=mode)
    seqs = []
    for prompt in G["prompts"]:
        header, payload = to_wire(engine.prefill.prefill(prompt))
        received = from_wire(header, payload.clone())      # what a remote decode GPU rebuilds
        seqs.append(engine.decode.admit(received, max_new_tokens=8))
    dec = engine.decode.engine
    while dec.scheduler.has_work:
        dec.step()
    assert [s.token_ids[s.num_prompt:] for s in seqs] == plain
    assert engine.prefill.engine.blocks.num_free == engine.prefill.engine.blocks.num_total


def test_swap_preemption_on_gpu_keeps_tokens(gpu):
    from iekv.engine.copier import HipSlotCopier
    from iekv.engine.engine import Engine, EngineConfig
    from iekv.engine.toy_model import ModelConfig, ToyTransformer

    small = ModelConfig(vocab_size=64, hidden_size=32, num_layers=2, num_heads=4,
                        num_kv_heads=2, head_dim=8, intermediate_size=64)
    prompts = [list(range(i, i + 12)) for i in range(4)]

    def run(num_blocks, preemption):
        m = ToyTransformer(small, seed=0, device=gpu, cache_dtype=torch.bfloat16)
        e = Engine(m, EngineConfig(block_size=8, num_blocks=num_blocks, max_batch_tokens=256,
                                   preemption=preemption))
        return e.generate(prompts, max_new_tokens=10, temperature=0.0), e

    expected, _ = run(256, "recompute")
    recompute, _ = run(8, "recompute")
    swapped, e = run(8, "swap")
    assert isinstance(e.swapper, HipSlotCopier) and e.swapper.payload_location == "host"
    assert swapped == recompute == expected
    assert e.scheduler.stats.swapped_in == e.scheduler.stats.swapped_out > 0


def test_batched_moves_on_gpu_are_one_launch(gpu):
    from iekv import _native
    from iekv.serve.disaggregated import DisaggregatedEngine

    m = model(gpu, torch.bfloat16)
    expected = DisaggregatedEngine(m, engine_config(), mode="direct").generate(
        G["prompts"], max_new_tokens=8)
    engine = DisaggregatedEngine(m, engine_config(), mode="direct")
    pending: list = []
    seqs = [engine.handoff(p, 8, 0.0, pending) for p in G["prompts"]]
    assert [s.block_table for s in seqs] == [r["dst_table"] for r in G["requests"]]
    with _native.LaunchTimer(64) as timer:
        engine.flush_moves(pending)
        torch.cuda.synchronize()
    assert len(timer.durations_ms) == 1 and timer.durations_ms[0] > 0
    dec = engine.decode.engine
    while dec.scheduler.has_work:
        dec.step()
    assert [s.token_ids[s.num_prompt:] for s in seqs] == expected
    fresh = DisaggregatedEngine(m, engine_config(), mode="direct")
    assert fresh.generate(G["prompts"], max_new_tokens=8, batch_moves=True) == expected


def test_batched_pack_moves_on_gpu_unpack_in_one_launch(gpu, monkeypatch):
    """Pack mode with batched moves: each prompt packs into the next slice of one
    staging buffer and the flush unpacks every request with one launch; the decode
    pool then holds the same bytes as after per-request admission, and decoding
    gives the same tokens. A buffer too small for the batch flushes when full, and a
    request larger than the whole buffer packs into a payload of its own."""
    from iekv import _native
    from iekv.serve import disaggregated
    from iekv.serve.disaggregated import DisaggregatedEngine

    m = model(gpu, torch.bfloat16)
    bs = G["engine"]["block_size"]
    plain = DisaggregatedEngine(m, engine_config())
    plain_seqs = [plain.handoff(p, 8, 0.0) for p in G["prompts"]]
    engine = DisaggregatedEngine(m, engine_config())
    pending: list = []
    total = sum(r["num_blocks"] for r in G["requests"])
    arena = disaggregated._StagingArena(engine, total, pending)
    seqs = [engine.handoff(p, 8, 0.0, pending, arena.take) for p in G["prompts"]]
    assert [s.block_table for s in seqs] == [r["dst_table"] for r in G["requests"]]
    assert arena.used == total and len(pending) == len(G["prompts"])
    with _native.LaunchTimer(64) as timer:
        assert engine.flush_moves(pending) == total
        torch.cuda.synchronize()
    assert len(timer.durations_ms) == 1 and timer.durations_ms[0] > 0
    caches = lambda e: e.decode.engine.k_caches + e.decode.engine.v_caches
    for a, b in zip(tiles(caches(plain), [x for s in plain_seqs for x in s.block_table], bs),
                    tiles(caches(engine), [x for s in seqs for x in s.block_table], bs)):
        assert torch.equal(a, b)
    plain.decode_until_done()
    engine.decode_until_done()
    expected = [s.token_ids[s.num_prompt:] for s in plain_seqs]
    assert [s.token_ids[s.num_prompt:] for s in seqs] == expected
    fresh = DisaggregatedEngine(m, engine_config())
    assert fresh.generate(G["prompts"], max_new_tokens=8, batch_moves=True) == expected
    block = disaggregated._per_block_bytes(fresh.prefill.engine)
    monkeypatch.setattr(disaggregated, "STAGING_ARENA_BYTES", 5 * block)
    small = DisaggregatedEngine(m, engine_config())
    assert small.generate(G["prompts"], max_new_tokens=8, batch_moves=True) == expected
    # A one-block buffer: every request of several blocks packs into a payload of its
    # own, the one-block ones share the buffer; the tokens do not change.
    assert max(r["num_blocks"] for r in G["requests"]) > 1
    monkeypatch.setattr(disaggregated, "STAGING_ARENA_BYTES", block)
    tiny = DisaggregatedEngine(m, engine_config())
    assert tiny.generate(G["prompts"], max_new_tokens=8, batch_moves=True) == expected


def test_batched_prefix_aware_moves_on_gpu(gpu):
    """Batched direct moves with prefix sharing: a prefix whose copy is still pending
    is shared (the one launch fills it before decode), and the blocks of a request
    that finished on arrival, never copied, are not."""
    from iekv.core.sequence import Status
    from iekv.serve.disaggregated import DisaggregatedEngine

    m = model(gpu, torch.bfloat16)
    prefix = list(range(1000, 1064))
    prompts = [prefix + list(range(1200 + 40 * i, 1200 + 40 * i + 20 + 7 * i)) for i in range(4)]
    plain = DisaggregatedEngine(m, engine_config()).generate(prompts, max_new_tokens=6)
    shared = DisaggregatedEngine(m, engine_config(), prefix_aware=True, mode="direct")
    assert shared.generate(prompts, max_new_tokens=6, batch_moves=True) == plain
    assert shared.stats.blocks_skipped == 4 * 3

    engine = DisaggregatedEngine(m, engine_config(), prefix_aware=True, mode="direct")
    pending: list = []
    done = engine.handoff(prompts[0], 1, 0.0, pending)
    assert done.status == Status.FINISHED and not pending
    seq = engine.handoff(prompts[1], 6, 0.0, pending)
    assert engine.stats.blocks_skipped == 0
    engine.flush_moves(pending)
    engine.decode_until_done()
    assert seq.token_ids[seq.num_prompt:] == plain[1]


def _wire_rank(rank: int, port: int, result_path: str) -> None:
    """One side of a two-process handoff: rank 0 prefills and sends, rank 1 admits and decodes."""
    import os
    import sys

    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    sys.path[:0] = [root, os.path.join(root, "inference-engine_amd"), here]
    import torch.distributed as dist

    from iekv.serve.disaggregated import DecodeWorker, DisaggregatedEngine, PrefillWorker
    from iekv.serve.wire import recv_transfer, send_transfer

    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=2)
    try:
        device = torch.device("cuda", 0)
        prompt = G["prompts"][1]
        if rank == 0:
            worker = PrefillWorker(model(device, torch.bfloat16), engine_config())
            transfer = worker.prefill(prompt, 0.0)          # one iekv_pack launch
            send_transfer(transfer, dst=1, device="cpu")    # gloo carries host tensors
        else:
            worker = DecodeWorker(model(device, torch.bfloat16), engine_config())
            transfer = recv_transfer(src=0, device="cpu")
            seq = worker.admit(transfer, max_new_tokens=8, temperature=0.0)  # iekv_restore
            worker.engine.run()
            got = seq.token_ids[seq.num_prompt:]
            want = DisaggregatedEngine(model(device, torch.bfloat16), engine_config()).generate(
                [prompt], max_new_tokens=8, temperature=0.0)[0]
            with open(result_path, "w") as f:
                f.write("ok" if got == want and len(got) == 8 else f"{got} != {want}")
    finally:
        dist.destroy_process_group()


def test_a_transfer_sent_between_processes_decodes_identically(gpu, tmp_path):
    """The wire format end to end: prefill and pack in one process, send the header and
    the block-major payload over torch.distributed, restore and decode in another; the
    tokens equal an in-process handoff's."""
    import socket

    import torch.multiprocessing as mp

    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        port = s.getsockname()[1]
    result = tmp_path / "result.txt"
    mp.spawn(_wire_rank, args=(port, str(result)), nprocs=2, join=True)
    assert result.read_text() == "ok"
