"""A small paged decoder that produces and consumes KV, for token-identity checks.

The handoff is correct iff decode after it reads, through the new block
tables, exactly the bytes prefill wrote. Checking that end to end needs a
model that writes KV by slot (``write_kv``, ie/kernels/torch_backend.py:13-16) and
reads it back through block tables (``gather_context``,
ie/kernels/torch_backend.py:19-24). This is that model, in plain torch,
shaped like the reference's toy transformer (ie/model/transformer.py:12-115:
RMSNorm, GQA attention with interleaved rotary embeddings, SwiGLU MLP; weights
drawn from ``numpy.random.default_rng(seed)`` in the same order). Attention
math runs in float32 whatever the cache dtype. It is support code: the
handoff never calls it. With ``hip_kv=True`` its KV writes and context reads go
through libiekv's slot kernels (``iekv.engine.slots``) instead of torch's
``index_copy_`` / ``index_select``.
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass

import numpy as np
import torch

from ..core.layout import BatchLayout
from .pools import allocate_pool, allocate_pool_pair


@dataclass(slots=True)
class ModelConfig:
    """Shape of the toy model (ie/model/transformer.py:12-34)."""

    vocab_size: int = 256
    hidden_size: int = 64
    num_layers: int = 2
    num_heads: int = 4
    num_kv_heads: int = 2
    head_dim: int = 16
    intermediate_size: int = 128
    max_position: int = 2048
    rope_base: float = 10000.0
    norm_eps: float = 1e-6
    rope_halved: bool = False

    def __post_init__(self) -> None:
        if self.num_heads % self.num_kv_heads:
            raise ValueError("num_heads must be divisible by num_kv_heads")
        if self.head_dim % 2:
            raise ValueError("head_dim must be even for rotary embeddings")

    @property
    def kv_bytes_per_token(self) -> int:
        return 2 * self.num_layers * self.num_kv_heads * self.head_dim * 4


def _rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    scale = torch.sqrt(torch.mean(x * x, dim=-1, keepdim=True) + eps)
    return (x / scale) * weight


def _rope(x: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
          halved: bool) -> torch.Tensor:
    c = cos[positions][:, None, :]
    s = sin[positions][:, None, :]
    out = torch.empty_like(x)
    if halved:
        half = x.shape[-1] // 2
        left, right = x[..., :half], x[..., half:]
        out[..., :half] = left * c - right * s
        out[..., half:] = right * c + left * s
    else:
        even, odd = x[..., 0::2], x[..., 1::2]
        out[..., 0::2] = even * c - odd * s
        out[..., 1::2] = even * s + odd * c
    return out


class _Layer:
    def __init__(self, config: ModelConfig, rng: np.random.Generator, put) -> None:
        scale = 1.0 / np.sqrt(config.hidden_size)
        q_out = config.num_heads * config.head_dim
        kv_out = config.num_kv_heads * config.head_dim

        def normal(*shape):
            return put((rng.standard_normal(shape) * scale).astype(np.float32))

        # Draw order matches the reference block (ie/model/transformer.py:36-60).
        self.attn_norm = put(np.ones(config.hidden_size, dtype=np.float32))
        self.q_proj = normal(config.hidden_size, q_out)
        self.k_proj = normal(config.hidden_size, kv_out)
        self.v_proj = normal(config.hidden_size, kv_out)
        self.o_proj = normal(q_out, config.hidden_size)
        self.mlp_norm = put(np.ones(config.hidden_size, dtype=np.float32))
        self.gate_proj = normal(config.hidden_size, config.intermediate_size)
        self.up_proj = normal(config.hidden_size, config.intermediate_size)
        self.down_proj = normal(config.intermediate_size, config.hidden_size)


class ToyTransformer:
    """Paged toy decoder on ``device`` with KV caches of ``cache_dtype``."""

    def __init__(self, config: ModelConfig, seed: int = 0, device: str | torch.device = "cuda",
                 cache_dtype: torch.dtype = torch.float32, hip_kv: bool = False) -> None:
        self.config = config
        self.device = torch.device(device)
        self.cache_dtype = cache_dtype
        self.hip_kv = hip_kv
        # Registered pools by cache address; an engine holds each one (bind_caches).
        self._pools: weakref.WeakValueDictionary = weakref.WeakValueDictionary()
        rng = np.random.default_rng(seed)
        scale = 1.0 / np.sqrt(config.hidden_size)

        def put(array: np.ndarray) -> torch.Tensor:
            return torch.from_numpy(np.ascontiguousarray(array)).to(self.device)

        self.embedding = put((rng.standard_normal((config.vocab_size, config.hidden_size))
                              * scale).astype(np.float32))
        self.layers = [_Layer(config, rng, put) for _ in range(config.num_layers)]
        self.final_norm = put(np.ones(config.hidden_size, dtype=np.float32))
        self.lm_head = put((rng.standard_normal((config.hidden_size, config.vocab_size))
                            * scale).astype(np.float32))
        exponents = np.arange(0, config.head_dim, 2, dtype=np.float32) / config.head_dim
        angles = np.outer(np.arange(config.max_position, dtype=np.float32),
                          np.power(config.rope_base, -exponents))
        self.cos = put(np.cos(angles))
        self.sin = put(np.sin(angles))

    def allocate_caches(self, num_blocks: int, block_size: int):
        c = self.config
        return allocate_pool(num_blocks, block_size, c.num_layers, c.num_kv_heads, c.head_dim,
                             dtype=self.cache_dtype, device=self.device)

    def allocate_cache_pair(self, first_blocks: int, second_blocks: int, block_size: int):
        """Two pools in one reservation (prefill first); see ``allocate_pool_pair``."""
        c = self.config
        return allocate_pool_pair(first_blocks, second_blocks, block_size, c.num_layers,
                                  c.num_kv_heads, c.head_dim, dtype=self.cache_dtype,
                                  device=self.device)

    def bind_caches(self, k_caches, v_caches, block_size: int):
        """Register a pool for the slot kernels; the caller keeps the returned
        handle for as long as it uses the caches (an Engine holds it for its
        lifetime). The model itself keeps only a weak reference, so a pool is
        released with the engine that owns it. None without ``hip_kv``."""
        if not self.hip_kv:
            return None
        from .pools import KVPool

        key = (k_caches[0].data_ptr(), v_caches[0].data_ptr(), block_size)
        pool = self._pools.get(key)
        if pool is None:
            pool = KVPool(k_caches, v_caches, block_size)
            self._pools[key] = pool
        return pool

    def _pool(self, k_caches, v_caches, block_size: int):
        key = (k_caches[0].data_ptr(), v_caches[0].data_ptr(), block_size)
        pool = self._pools.get(key)
        if pool is None:      # caches nobody bound: a pool for this call only
            from .pools import KVPool

            pool = KVPool(k_caches, v_caches, block_size)
        return pool

    def _cached_rows(self, cache: torch.Tensor, table: list[int], context_len: int,
                     block_size: int) -> torch.Tensor:
        """Rows 0..context_len-1 of a sequence in one cache array (torch's index_select)."""
        needed = -(-context_len // block_size)
        blocks = torch.as_tensor(table[:needed], device=self.device, dtype=torch.long)
        within = torch.arange(block_size, device=self.device)
        slots = (blocks[:, None] * block_size + within[None, :]).reshape(-1)[:context_len]
        return cache.index_select(0, slots)

    def _attend(self, q: torch.Tensor, contexts, layout: BatchLayout) -> torch.Tensor:
        """Causal attention of each sequence's queries over its (K, V) context rows."""
        c = self.config
        group = c.num_heads // c.num_kv_heads
        outputs = []
        start = 0
        for (k, v), context_len, query_len in zip(contexts, layout.context_lens,
                                                  layout.query_lens):
            k = k.float().repeat_interleave(group, dim=1)
            v = v.float().repeat_interleave(group, dim=1)
            # [heads, tokens, dim] operands, made contiguous before the batched products.
            qh = q[start:start + query_len].permute(1, 0, 2).contiguous()
            kt = k.permute(1, 2, 0).contiguous()
            vh = v.permute(1, 0, 2).contiguous()
            scores = torch.matmul(qh, kt) / float(np.sqrt(c.head_dim))
            rows = torch.arange(query_len, device=self.device)[:, None] + (context_len - query_len)
            cols = torch.arange(context_len, device=self.device)[None, :]
            scores = scores.masked_fill(~(cols <= rows), float("-inf"))
            weights = torch.softmax(scores, dim=-1)
            outputs.append(torch.matmul(weights, vh).permute(1, 0, 2))
            start += query_len
        return torch.cat(outputs, dim=0)

    @torch.no_grad()
    def forward(self, layout: BatchLayout, k_caches, v_caches, block_size: int) -> torch.Tensor:
        """One step over the layout's tokens; writes their K/V rows into the caches.

        The torch path writes each layer's rows with index_copy_ and reads each
        sequence's context back with index_select, layer by layer. With ``hip_kv``
        the slot kernels do it in two kinds of launch: before the layers, one
        iekv_gather_rows_arrays per sequence fetches its earlier context (the rows
        before this step) from every layer's K and V cache; each layer then
        attends over that context followed by this step's rows, cast to the cache
        dtype exactly as a cache read returns them; after the layers, one
        iekv_write_slots_layers writes every layer's new rows.
        """
        c = self.config
        tokens = torch.as_tensor(layout.token_ids, device=self.device, dtype=torch.long)
        positions = torch.as_tensor(layout.positions, device=self.device, dtype=torch.long)
        slots = torch.as_tensor(layout.slot_mapping, device=self.device, dtype=torch.long)
        x = self.embedding[tokens]
        pool = self._pool(k_caches, v_caches, block_size) if self.hip_kv else None
        if pool is not None:
            from .slots import gather_rows_arrays, write_slots_layers

            earlier = [gather_rows_arrays(pool, table, ctx - n) if ctx > n else None
                       for table, ctx, n in zip(layout.block_tables, layout.context_lens,
                                                layout.query_lens)]
            new_k, new_v = [], []
        bounds = np.concatenate(([0], np.cumsum(layout.query_lens))).tolist()
        for index, (layer, k_cache, v_cache) in enumerate(zip(self.layers, k_caches, v_caches)):
            normed = _rms_norm(x, layer.attn_norm, c.norm_eps)
            q = (normed @ layer.q_proj).view(-1, c.num_heads, c.head_dim)
            k = (normed @ layer.k_proj).view(-1, c.num_kv_heads, c.head_dim)
            v = (normed @ layer.v_proj).view(-1, c.num_kv_heads, c.head_dim)
            q = _rope(q, positions, self.cos, self.sin, c.rope_halved)
            k = _rope(k, positions, self.cos, self.sin, c.rope_halved)
            kc, vc = k.to(k_cache.dtype), v.to(v_cache.dtype)
            if pool is not None:
                new_k.append(kc)
                new_v.append(vc)
                contexts = []
                for s, prior in enumerate(earlier):
                    ks, vs = kc[bounds[s]:bounds[s + 1]], vc[bounds[s]:bounds[s + 1]]
                    if prior is not None:
                        ks = torch.cat((prior[index], ks))
                        vs = torch.cat((prior[c.num_layers + index], vs))
                    contexts.append((ks, vs))
            else:
                k_cache.index_copy_(0, slots, kc)
                v_cache.index_copy_(0, slots, vc)
                contexts = [(self._cached_rows(k_cache, t, n, block_size),
                             self._cached_rows(v_cache, t, n, block_size))
                            for t, n in zip(layout.block_tables, layout.context_lens)]
            attended = self._attend(q, contexts, layout)
            x = x + attended.reshape(-1, c.num_heads * c.head_dim) @ layer.o_proj
            normed = _rms_norm(x, layer.mlp_norm, c.norm_eps)
            gate = normed @ layer.gate_proj
            x = x + (gate / (1.0 + torch.exp(-gate)) * (normed @ layer.up_proj)) @ layer.down_proj
        if pool is not None and layout.num_tokens:
            write_slots_layers(pool, torch.stack(new_k), torch.stack(new_v), slots)
        return _rms_norm(x, self.final_norm, c.norm_eps)

    @torch.no_grad()
    def logits_for_last_token_of_each(self, hidden: torch.Tensor,
                                      query_lens: list[int]) -> np.ndarray:
        ends = torch.as_tensor(np.cumsum(query_lens) - 1, device=self.device, dtype=torch.long)
        return (hidden[ends] @ self.lm_head).float().cpu().numpy()
