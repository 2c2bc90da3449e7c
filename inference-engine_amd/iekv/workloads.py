"""Synthetic handoff workloads: the five configurations the benchmark and tests use.

Each workload is a list of requests; request r moves ``src_tables[r]`` (ids in
the prefill pool) onto ``dst_tables[r]`` (ids in the decode pool). Destination
ids always come from this package's ``BlockManager`` exactly as a decode
worker would obtain them (``reserve`` from the free list, or ``allocate`` with
a resident shared prefix for cfg4), so their order is the reference's
(ie/core/block_manager.py:50, 87-92, 193-198). All draws are from
``numpy.random.default_rng(seed)``.

cfg1  NumPy CPU case: 4L, 4 KV heads, D32, fp32, bs16; 64 seqs U[16,512];
      src = a permutation of a 4096-block pool; dst from a fresh 4096-block pool.
cfg2  Qwen2.5-0.5B shape: 24L, 2 KV heads, D64, fp16, bs256; 64 seqs U[64,400];
      2048-block pools, both free lists randomly fragmented.
cfg3  Llama-3-8B shape: 32L, 8 KV heads, D128, bf16, bs16; 256 seqs, lengths
      log-uniform in [512, 8192]; random non-contiguous src and dst tables.
cfg4  cfg3 shape; a 2048-token prefix (128 blocks) resident in the decode pool
      and shared by refcount; 128 unique suffixes U[256,4096]; only the blocks
      after the prefix move.
cfg5  One GPU's share of a Llama-3-70B-shape handoff: 80L, 8 KV heads, D128,
      fp8 e4m3 stored as raw bytes, bs16; 16 seqs x 16384 tokens; pools of
      exactly 16384 blocks, so the whole pool moves.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from .core.block_manager import BlockManager
from .core.sequence import Sequence

ELEMENT_BYTES = {"float32": 4, "float16": 2, "bfloat16": 2, "fp8_e4m3": 1, "uint8": 1}


@dataclass(frozen=True)
class Shape:
    layers: int
    kv_heads: int
    head_dim: int
    block_size: int
    dtype: str

    @property
    def elem_bytes(self) -> int:
        return ELEMENT_BYTES[self.dtype]

    @property
    def tile_bytes(self) -> int:
        """T = block_size x H x D x element bytes."""
        return self.block_size * self.kv_heads * self.head_dim * self.elem_bytes

    @property
    def n_arrays(self) -> int:
        return 2 * self.layers

    @property
    def block_bytes(self) -> int:
        """Payload of one block, 2L x T."""
        return self.n_arrays * self.tile_bytes


@dataclass
class Workload:
    name: str
    description: str
    shape: Shape
    lengths: list[int]
    src_tables: list[list[int]]
    dst_tables: list[list[int]]
    src_pool_blocks: int
    dst_pool_blocks: int
    skipped_blocks: int = 0            # prefix blocks found resident (cfg4), not moved
    resident_prefix: list[int] = field(default_factory=list)

    @property
    def num_requests(self) -> int:
        return len(self.src_tables)

    @property
    def num_blocks(self) -> int:
        return sum(len(t) for t in self.src_tables)

    @property
    def payload_bytes(self) -> int:
        """P = B x 2L x T, the bytes a handoff reads once and writes once."""
        return self.num_blocks * self.shape.block_bytes

    def subset(self, requests: int) -> "Workload":
        return Workload(self.name, self.description, self.shape, self.lengths[:requests],
                        self.src_tables[:requests], self.dst_tables[:requests],
                        self.src_pool_blocks, self.dst_pool_blocks, self.skipped_blocks,
                        self.resident_prefix)


def _blocks(n_tokens: int, bs: int) -> int:
    return -(-n_tokens // bs)


def _split(ids: np.ndarray, counts: list[int]) -> list[list[int]]:
    out, at = [], 0
    for c in counts:
        out.append([int(b) for b in ids[at:at + c]])
        at += c
    return out


def _reserve_tables(pool_blocks: int, bs: int, lengths: list[int], counts: list[int],
                    free_order: np.ndarray | None = None) -> list[list[int]]:
    """Destination tables as a decode worker gets them: BlockManager.reserve per request."""
    manager = BlockManager(pool_blocks, bs)
    if free_order is not None:
        manager.free_ids = [int(b) for b in free_order]
    tables = []
    for n, c in zip(lengths, counts):
        seq = Sequence(list(range(max(1, n))), bs)
        if not manager.reserve(seq, c):
            raise RuntimeError("destination pool too small for the workload")
        tables.append(seq.block_table)
    return tables


def cfg1(seed: int = 0) -> Workload:
    shape = Shape(4, 4, 32, 16, "float32")
    pool = 4096
    rng = np.random.default_rng(seed)
    lengths = [int(n) for n in rng.integers(16, 512, size=64, endpoint=True)]
    counts = [_blocks(n, shape.block_size) for n in lengths]
    src = _split(rng.permutation(pool), counts)
    dst = _reserve_tables(pool, shape.block_size, lengths, counts)
    return Workload("cfg1", "NumPy CPU case: 4L H4 D32 fp32 bs16, 64 seqs U[16,512]", shape,
                    lengths, src, dst, pool, pool)


def cfg2(seed: int = 0) -> Workload:
    shape = Shape(24, 2, 64, 256, "float16")
    pool = 2048
    rng = np.random.default_rng(seed)
    lengths = [int(n) for n in rng.integers(64, 400, size=64, endpoint=True)]
    counts = [_blocks(n, shape.block_size) for n in lengths]
    src = _split(rng.permutation(pool), counts)
    dst = _reserve_tables(pool, shape.block_size, lengths, counts,
                          free_order=rng.permutation(pool))
    return Workload("cfg2", "Qwen2.5-0.5B shape: 24L H2 D64 fp16 bs256, 64 seqs U[64,400], "
                    "fragmented 2048-block pools", shape, lengths, src, dst, pool, pool)


LLAMA8B_SLACK = 64   # spare blocks of the Llama-3-8B-shape engine's pools beyond cfg3's needs


def _llama8b_lengths(rng: np.random.Generator) -> list[int]:
    """cfg3's 256 prompt lengths, log-uniform in [512, 8192]."""
    return [int(n) for n in np.floor(np.exp(rng.uniform(math.log(512), math.log(8192),
                                                        size=256)))]


def llama8b_engine_blocks(seed: int = 0) -> int:
    """Blocks per pool of the Llama-3-8B-shape engine of these benchmarks: what cfg3's
    256 requests need at ``seed``, plus LLAMA8B_SLACK (49,598 at seed 0, 104 GB)."""
    return sum(_blocks(n, 16) for n in _llama8b_lengths(np.random.default_rng(seed))) + \
        LLAMA8B_SLACK


def cfg3(seed: int = 0, slack: int = LLAMA8B_SLACK) -> Workload:
    shape = Shape(32, 8, 128, 16, "bfloat16")
    rng = np.random.default_rng(seed)
    lengths = _llama8b_lengths(rng)
    counts = [_blocks(n, shape.block_size) for n in lengths]
    pool = sum(counts) + slack
    src = _split(rng.permutation(pool), counts)
    dst = _reserve_tables(pool, shape.block_size, lengths, counts,
                          free_order=rng.permutation(pool))
    return Workload("cfg3", "Llama-3-8B shape: 32L H8 D128 bf16 bs16, 256 seqs log-U[512,8192], "
                    "random src/dst tables", shape, lengths, src, dst, pool, pool)


def cfg4(seed: int = 0, slack: int | None = None) -> Workload:
    """The prefix-sharing workload on the cfg3 model. By default both pools have the
    Llama-3-8B-shape engine's size (llama8b_engine_blocks, as cfg3's pools); ``slack``
    sizes them to this workload's needs plus ``slack`` blocks instead.

    The pool size matters on MI355X: moving the same 17,803 blocks (the pools re-made
    three times in one process, one box), pools sized to the workload (17,867 /
    17,996 blocks, 99.6% moved or resident) ran the per-request direct copy at 5.05,
    5.61 and 5.61 TB/s, depending on the physical pages the driver gave the 37 GB
    pools; 24,403-block pools at 6.04-6.11; the engine's 49,534-block pools at
    6.25 TB/s all three times. Translation counters were the same across those
    placements (UTCL1 misses per MB and UTCL2 busy per cycle).
    """
    shape = Shape(32, 8, 128, 16, "bfloat16")
    bs = shape.block_size
    rng = np.random.default_rng(seed)
    prefix = list(range(2048))
    suffixes = [int(n) for n in rng.integers(256, 4096, size=128, endpoint=True)]
    lengths = [len(prefix) + s for s in suffixes]
    prefix_blocks = len(prefix) // bs
    counts = [_blocks(n, bs) - prefix_blocks for n in lengths]
    need_dst, need_src = prefix_blocks + 1 + sum(counts), sum(counts)
    if slack is None:
        engine = llama8b_engine_blocks(seed)
        dst_pool, src_pool = max(engine, need_dst), max(engine, need_src)
    else:
        dst_pool, src_pool = need_dst + slack, need_src + slack
    src = _split(rng.permutation(src_pool), counts)

    manager = BlockManager(dst_pool, bs)
    manager.free_ids = [int(b) for b in rng.permutation(dst_pool)]
    holder = Sequence(prefix + [0], bs)         # the request that made the prefix resident
    manager.allocate(holder)
    holder.num_computed = len(prefix)
    manager.share_computed_blocks(holder)
    resident = holder.block_table[:prefix_blocks]
    dst = []
    next_token = 1 << 20
    for s in suffixes:
        tokens = prefix + list(range(next_token, next_token + s))
        next_token += s
        seq = Sequence(tokens, bs)
        manager.allocate(seq)
        if seq.block_table[:prefix_blocks] != resident:
            raise RuntimeError("prefix blocks were not shared")
        dst.append(seq.block_table[prefix_blocks:])
    return Workload("cfg4", "prefix sharing: cfg3 shape and pools, 2048-token resident prefix, "
                    "128 suffixes U[256,4096], only unique blocks move", shape, lengths, src, dst,
                    src_pool, dst_pool, skipped_blocks=prefix_blocks * len(suffixes),
                    resident_prefix=resident)


def cfg5(seed: int = 0) -> Workload:
    shape = Shape(80, 8, 128, 16, "fp8_e4m3")
    rng = np.random.default_rng(seed)
    lengths = [16384] * 16
    counts = [_blocks(n, shape.block_size) for n in lengths]
    pool = sum(counts)
    src = _split(rng.permutation(pool), counts)
    dst = _reserve_tables(pool, shape.block_size, lengths, counts)
    return Workload("cfg5", "Llama-3-70B-shape share: 80L H8 D128 fp8 e4m3 bytes bs16, "
                    "16 x 16384 tokens, whole 16384-block pools", shape, lengths, src, dst,
                    pool, pool)


CONFIGS = {"cfg1": cfg1, "cfg2": cfg2, "cfg3": cfg3, "cfg4": cfg4, "cfg5": cfg5}


def tp_share(w: Workload, tp: int) -> Workload:
    """One rank's share of ``w`` under head-sharded tensor parallelism of degree ``tp``.

    Under TP each rank's caches hold ``H / tp`` of the KV heads
    (ie/parallel/tensor_parallel.py:17-18, 76-79) while the block tables are
    shared, so every rank moves the same block ids with tiles of
    ``bs x (H / tp) x D x e`` bytes; the payload per rank is ``P / tp``.
    """
    if tp < 1 or w.shape.kv_heads % tp:
        raise ValueError(f"tp={tp} does not divide the {w.shape.kv_heads} KV heads of {w.name}")
    if tp == 1:
        return w
    s = w.shape
    shape = Shape(s.layers, s.kv_heads // tp, s.head_dim, s.block_size, s.dtype)
    return Workload(f"{w.name}/tp{tp}", f"{w.description}; one rank's share at tp={tp} "
                    f"({shape.kv_heads} of {s.kv_heads} KV heads)", shape, w.lengths,
                    w.src_tables, w.dst_tables, w.src_pool_blocks, w.dst_pool_blocks,
                    w.skipped_blocks, w.resident_prefix)


def make(name: str, seed: int = 0, slack: int | None = None, tp: int = 1) -> Workload:
    """Workload ``name``; ``slack`` (cfg3, cfg4) sets the spare blocks in each pool;
    ``tp`` > 1 gives one rank's share under head-sharded tensor parallelism."""
    if name not in CONFIGS:
        raise ValueError(f"unknown workload {name!r}; choose from {sorted(CONFIGS)}")
    if slack is None:
        w = CONFIGS[name](seed)
    elif name not in ("cfg3", "cfg4"):
        raise ValueError(f"{name} has fixed pool sizes")
    else:
        w = CONFIGS[name](seed, slack=slack)
    return tp_share(w, tp)
