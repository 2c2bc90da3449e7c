"""Write golden fixtures for the handoff by running the reference engine (in the build container only).

Usage:  python tests/golden/make_golden.py /path/to/reference

The reference (kuluruvineeth/inference-engine, pure Python + NumPy) is imported
from the given checkout and driven through three scenarios; only their inputs
and outputs are saved, as JSON next to this script:

* ``disaggregation.json`` — tests/test_disaggregation.py's model, engine config
  and prompts: per-request source and destination block tables (recorded from
  the copier calls), KVTransfer fields, counters, stats, and the greedy tokens
  of the colocated and disaggregated engines; plus the undersized-decode-pool
  failure (tests/test_disaggregation.py:77-84) and the state it leaves behind.
* ``offload.json`` — tests/test_offload.py:103-121's scenario with the tier on
  and off: the exact sequence of copier reads/writes (block ids), tier keys,
  block-manager and tier stats, and the revisit tokens.
* ``cfg1_handoff.json`` — the CPU-runnable benchmark case (4 layers, 4 KV heads,
  head_dim 32, block_size 16, fp32, 4096-block pools, 64 sequences of U[16,512]
  tokens, source ids a random permutation): destination tables from the
  reference BlockManager.reserve, per-array sha256 of the destination pool
  after the reference LayeredSlotCopier moved every block, sha256 of the
  packed payload image, and the copier counters.

The recipes that generate inputs are written out here in plain NumPy and are
restated, independently, by the tests that consume the fixtures.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def sha(array: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(array).tobytes()).hexdigest()


class Recorder:
    """Wraps a copier and logs ("r"|"w", block_id) for every call."""

    def __init__(self, inner, log):
        self.inner = inner
        self.log = log

    def read_block(self, block_id):
        self.log.append(["r", int(block_id)])
        return self.inner.read_block(block_id)

    def write_block(self, block_id, payload):
        self.log.append(["w", int(block_id)])
        return self.inner.write_block(block_id, payload)

    def __getattr__(self, name):
        return getattr(self.inner, name)


def disaggregation() -> dict:
    from ie.engine.engine import EngineConfig, build_engine
    from ie.model.transformer import ModelConfig, Transformer
    from ie.serve.disaggregated import DisaggregatedEngine

    config = dict(vocab_size=2048, hidden_size=64, num_layers=3, num_heads=4, num_kv_heads=2,
                  head_dim=16, intermediate_size=128)
    engine_cfg = dict(block_size=16, num_blocks=512, max_batch_tokens=512)
    prompts = [list(range(100 + i * 80, 100 + i * 80 + 48)) for i in range(4)]
    model_cfg = ModelConfig(**config)
    out: dict = {"model": config, "engine": engine_cfg, "prompts": prompts, "model_seed": 1}

    out["colocated"] = {}
    for n in (1, 5, 10, 12):
        out["colocated"][str(n)] = build_engine(model_cfg, EngineConfig(**engine_cfg),
                                                model_seed=1).generate(
            prompts, max_new_tokens=n, temperature=0.0)

    split = DisaggregatedEngine(Transformer(model_cfg, seed=1), EngineConfig(**engine_cfg))
    log: list = []
    split.prefill.copier = Recorder(split.prefill.copier, log)
    split.decode.copier = Recorder(split.decode.copier, log)
    requests = []
    for prompt in prompts:
        before = len(log)
        transfer = split.prefill.prefill(prompt, 0.0)
        src = [b for op, b in log[before:] if op == "r"]
        seq = split.decode.admit(transfer, 10, 0.0)
        requests.append({
            "src_table": src,
            "dst_table": list(seq.block_table),
            "num_blocks": transfer.num_blocks,
            "num_computed": transfer.num_computed,
            "token_ids": list(transfer.token_ids),
            "bytes_moved": transfer.bytes_moved,
            "prefill_free_after": split.prefill.engine.blocks.num_free,
        })
        split.stats.prefills += 1
        split.stats.transfers += 1
        split.stats.blocks_transferred += transfer.num_blocks
        split.stats.bytes_transferred += transfer.bytes_moved
        split.stats.prefill_tokens += len(prompt)
    out["requests"] = requests
    out["copier_log"] = log
    out["prefill_copier"] = {"blocks_read": split.prefill.copier.blocks_read,
                             "blocks_written": split.prefill.copier.blocks_written,
                             "bytes_moved": split.prefill.copier.bytes_moved}
    out["decode_copier"] = {"blocks_read": split.decode.copier.blocks_read,
                            "blocks_written": split.decode.copier.blocks_written,
                            "bytes_moved": split.decode.copier.bytes_moved}
    out["decode_free_after_admit"] = split.decode.engine.blocks.num_free
    out["decode_free_ids_after_admit"] = list(split.decode.engine.blocks.free_ids)[:64]

    out["disaggregated"] = {}
    for n in (1, 5, 10, 12):
        engine = DisaggregatedEngine(Transformer(model_cfg, seed=1), EngineConfig(**engine_cfg))
        tokens = engine.generate(prompts, max_new_tokens=n, temperature=0.0)
        out["disaggregated"][str(n)] = tokens
        if n == 10:
            st = engine.stats
            out["stats_10"] = {k: getattr(st, k) for k in (
                "prefills", "decodes", "transfers", "blocks_transferred", "bytes_transferred",
                "prefill_tokens", "decode_tokens")}
            out["decode_block_stats_10"] = engine.decode.engine.blocks.stats()
            out["decode_free_ids_10"] = list(engine.decode.engine.blocks.free_ids)[:64]

    # Undersized decode pool (tests/test_disaggregation.py:77-84).
    tiny = DisaggregatedEngine(Transformer(model_cfg, seed=1), EngineConfig(**engine_cfg))
    tiny.decode = type(tiny.decode)(Transformer(model_cfg, seed=1),
                                    EngineConfig(block_size=16, num_blocks=2, max_batch_tokens=512))
    transfer = tiny.prefill.prefill(list(range(300, 400)))
    try:
        tiny.decode.admit(transfer, max_new_tokens=4)
        raised = None
    except RuntimeError as exc:
        raised = str(exc)
    waiting = list(tiny.decode.engine.scheduler.waiting)
    out["undersized"] = {
        "raised": raised,
        "transfer_blocks": transfer.num_blocks,
        "waiting": len(waiting),
        "leaked_table": list(waiting[0].block_table) if waiting else None,
        "decode_free": tiny.decode.engine.blocks.num_free,
    }
    return out


def offload() -> dict:
    from ie.engine.engine import EngineConfig, build_engine
    from ie.model.transformer import ModelConfig

    config = dict(vocab_size=2048, hidden_size=32, num_layers=2, num_heads=4, num_kv_heads=2,
                  head_dim=8, intermediate_size=64)
    prompts = [list(range(100 + i * 64, 100 + i * 64 + 64)) for i in range(6)]
    out: dict = {"model": config, "prompts": prompts, "model_seed": 0}
    for capacity in (0, 64):
        cfg = EngineConfig(block_size=16, num_blocks=12, max_batch_tokens=512,
                           offload_blocks=capacity)
        engine = build_engine(ModelConfig(**config), cfg)
        log: list = []
        if engine.blocks.copier is not None:
            engine.blocks.copier = Recorder(engine.blocks.copier, log)
        steps = []
        for prompt in prompts:
            tokens = engine.generate([prompt], max_new_tokens=2, temperature=0.0)[0]
            steps.append({"tokens": tokens, "free_ids": list(engine.blocks.free_ids),
                          "tier_keys": list(engine.blocks.tier.entries) if engine.blocks.tier
                          else []})
        revisit = engine.generate([prompts[0]], max_new_tokens=2, temperature=0.0)[0]
        tier = engine.blocks.tier
        out[str(capacity)] = {
            "steps": steps,
            "revisit": revisit,
            "stats": engine.blocks.stats(),
            "copier_log": log,
            "tier_keys": list(tier.entries) if tier else [],
            "tier_stats": ({k: getattr(tier.stats, k) for k in
                            ("admitted", "restored", "evicted", "rejected")} if tier else None),
            "free_ids": list(engine.blocks.free_ids),
        }
    return out


def cfg1_handoff() -> dict:
    from ie.core.block_manager import BlockManager
    from ie.core.sequence import Sequence
    from ie.engine.copier import LayeredSlotCopier

    layers, heads, dim, bs, pool_blocks, seqs = 4, 4, 32, 16, 4096, 64
    rng = np.random.default_rng(0)
    lengths = rng.integers(16, 512, size=seqs, endpoint=True)
    counts = [int(-(-int(n) // bs)) for n in lengths]
    perm = rng.permutation(pool_blocks)
    src_tables, at = [], 0
    for c in counts:
        src_tables.append([int(b) for b in perm[at:at + c]])
        at += c

    fill = np.random.default_rng(1)
    shape = (pool_blocks * bs, heads, dim)
    src_k = [fill.standard_normal(shape, dtype=np.float32) for _ in range(layers)]
    src_v = [fill.standard_normal(shape, dtype=np.float32) for _ in range(layers)]
    dst_k = [np.zeros(shape, dtype=np.float32) for _ in range(layers)]
    dst_v = [np.zeros(shape, dtype=np.float32) for _ in range(layers)]

    manager = BlockManager(pool_blocks, bs)
    src = LayeredSlotCopier(src_k, src_v, bs)
    dst = LayeredSlotCopier(dst_k, dst_v, bs)
    dst_tables = []
    image = hashlib.sha256()
    for n, table in zip(lengths, src_tables):
        seq = Sequence(list(range(int(n))), bs)
        assert manager.reserve(seq, len(table))
        dst_tables.append(list(seq.block_table))
        payloads = [src.read_block(b) for b in table]
        for k_tiles, v_tiles in payloads:
            for tile in (*k_tiles, *v_tiles):
                image.update(np.ascontiguousarray(tile).tobytes())
        for block_id, payload in zip(seq.block_table, payloads):
            dst.write_block(block_id, payload)
    return {
        "shape": {"layers": layers, "kv_heads": heads, "head_dim": dim, "block_size": bs,
                  "pool_blocks": pool_blocks, "sequences": seqs, "dtype": "float32"},
        "recipe": "lengths=default_rng(0).integers(16,512,64,endpoint=True); "
                  "perm=same rng.permutation(4096) split in order; "
                  "fill=default_rng(1).standard_normal(float32) for K0..K3 then V0..V3",
        "lengths": [int(n) for n in lengths],
        "src_tables": src_tables,
        "dst_tables": dst_tables,
        "total_blocks": sum(counts),
        "src_sha256": {"k": [sha(a) for a in src_k], "v": [sha(a) for a in src_v]},
        "dst_sha256": {"k": [sha(a) for a in dst_k], "v": [sha(a) for a in dst_v]},
        "packed_sha256": image.hexdigest(),
        "src_counters": {"blocks_read": src.blocks_read, "bytes_moved": src.bytes_moved},
        "dst_counters": {"blocks_written": dst.blocks_written, "bytes_moved": dst.bytes_moved},
    }


def main() -> None:
    reference = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference").resolve()
    sys.path.insert(0, str(reference))
    for name, fn in (("disaggregation", disaggregation), ("offload", offload),
                     ("cfg1_handoff", cfg1_handoff)):
        data = fn()
        path = HERE / f"{name}.json"
        path.write_text(json.dumps(data, separators=(",", ":")) + "\n")
        print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
