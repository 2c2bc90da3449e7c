"""The engine each disaggregation worker owns: pool, block manager, scheduler, model.

Behaviour follows the reference's ``Engine`` (ie/engine/engine.py:17-127) in
everything the handoff observes: pool allocation per layer, block
management, scheduling, prefill/decode steps and the offload-tier wiring
(engine.py:57-63). The copier is pluggable: by default the HIP copier
(``iekv.engine.copier.copier_for``); any object with the reference's
``read_block``/``write_block`` protocol can be injected via ``copier_factory``
(signature ``factory(k_caches, v_caches, block_size, role)``, ``role`` being
``"transfer"`` or ``"offload"``).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

import numpy as np

from ..core.block_manager import BlockManager
from ..core.layout import build_layout
from ..core.offload import KVTier
from ..core.scheduler import Scheduler
from ..core.sequence import Sequence

CopierFactory = Callable[[Any, Any, int, str], Any]


@dataclass(slots=True)
class EngineConfig:
    """ie/engine/engine.py:17-25. ``capture_graphs`` is accepted and ignored here.

    ``preemption`` is this build's addition: ``"recompute"`` (the reference's
    behaviour) or ``"swap"`` (preempted sequences keep their KV in host memory).
    """

    block_size: int = 16
    num_blocks: int = 1024
    max_batch_sequences: int = 64
    max_batch_tokens: int = 2048
    seed: int = 0
    offload_blocks: int = 0
    capture_graphs: bool = False
    preemption: str = "recompute"


def sample_from_logits(logits: np.ndarray, temperatures: np.ndarray,
                       generator: np.random.Generator) -> np.ndarray:
    """One token per row: the argmax for temperature <= 0, else a draw from
    softmax(logits / temperature).

    The draw is an exponential race: with independent E_i ~ Exp(1), the index
    maximising p_i / E_i is distributed as p. In log space that index maximises
    logits_i / T - log E_i (the softmax normaliser is the same for every i), so
    no probabilities are formed. The race draws one Exp(1) value per logit per
    call, greedy rows included, like the reference's sampler
    (ie/layers/functional.py:64-73), so the two consume the generator alike.
    """
    logits = np.asarray(logits)
    temps = np.asarray(temperatures, dtype=np.float32)
    race = generator.exponential(1.0, size=logits.shape)
    greedy = temps <= 0.0
    scale = np.where(greedy, np.float32(1.0), temps)[:, None]
    keyed = logits.astype(np.float32) / scale - np.log(np.maximum(race, 1e-10))
    return np.where(greedy, logits.argmax(axis=-1), keyed.argmax(axis=-1))


def default_copier_factory(k_caches, v_caches, block_size: int, role: str):
    from .copier import copier_for  # imports torch and the HIP library lazily

    return copier_for(k_caches, v_caches, block_size, role)


class Engine:
    """ie/engine/engine.py:28-127.

    ``caches`` (this build's addition) hands the engine a pool allocated by the
    caller, ``(k_caches, v_caches)`` with ``num_blocks * block_size`` rows per
    array, instead of ``model.allocate_caches``; the disaggregation workers use
    it to share one reservation.
    """

    def __init__(self, model, config: EngineConfig | None = None,
                 copier_factory: CopierFactory | None = None, caches=None) -> None:
        self.model = model
        self.config = config or EngineConfig()
        self.copier_factory = copier_factory or default_copier_factory
        if self.config.preemption not in ("recompute", "swap"):
            raise ValueError("preemption must be 'recompute' or 'swap'")
        self.blocks = BlockManager(self.config.num_blocks, self.config.block_size)
        self.generator = np.random.default_rng(self.config.seed)
        if caches is None:
            caches = model.allocate_caches(self.config.num_blocks, self.config.block_size)
        self.k_caches, self.v_caches = caches
        rows = self.config.num_blocks * self.config.block_size
        if (len(self.k_caches) != len(self.v_caches)
                or any(len(t) != rows for t in list(self.k_caches) + list(self.v_caches))):
            raise ValueError(f"caches must hold {rows} rows per array, K and V per layer")
        # Per-pool state the model keeps for these caches (the toy model's slot-kernel
        # pool registration); held here so it lives exactly as long as the engine.
        bind = getattr(model, "bind_caches", None)
        self.model_state = bind(self.k_caches, self.v_caches, self.config.block_size) \
            if bind is not None else None
        self.swapper = None
        if self.config.preemption == "swap":
            self.swapper = self.copier_factory(self.k_caches, self.v_caches,
                                               self.config.block_size, "swap")
        self.scheduler = Scheduler(self.blocks,
                                   max_batch_sequences=self.config.max_batch_sequences,
                                   max_batch_tokens=self.config.max_batch_tokens,
                                   swapper=self.swapper)
        self.copier = None
        if self.config.offload_blocks > 0:
            self.copier = self.copier_factory(self.k_caches, self.v_caches,
                                              self.config.block_size, "offload")
            self.blocks.tier = KVTier(self.config.offload_blocks)
            self.blocks.copier = self.copier

    def make_copier(self, role: str = "transfer"):
        return self.copier_factory(self.k_caches, self.v_caches, self.config.block_size, role)

    def submit(self, prompt_ids: list[int], max_new_tokens: int = 32,
               temperature: float = 1.0, eos_id: int | None = None) -> Sequence:
        """Queue a request; it starts at the next step the pool has room for it."""
        seq = Sequence(prompt_ids, self.config.block_size, max_new_tokens=max_new_tokens,
                       temperature=temperature, eos_id=eos_id)
        self.scheduler.add(seq)
        return seq

    def flush_offloads(self) -> None:
        """Issue the offload reads queued by this step's evictions (one batched launch).

        Called before anything writes the pool outside the offload copier (the
        model's forward pass, an admitted transfer), so every queued read sees
        the bytes the block held when it was evicted.
        """
        self.blocks.flush_pending()

    def forward(self, batch):
        """Run the model over a scheduled batch; returns (layout, last-token logits)."""
        self.flush_offloads()
        layout = build_layout(batch, self.config.block_size)
        hidden = self.model.forward(layout, self.k_caches, self.v_caches, self.config.block_size)
        return layout, self.model.logits_for_last_token_of_each(hidden, layout.query_lens)

    def _advance(self):
        """One scheduled step: forward, sample one token per sequence, commit.
        Returns (batch, sequences that finished), or (None, []) when nothing ran."""
        batch = self.scheduler.schedule()
        if not batch:
            return None, []
        _, logits = self.forward(batch)
        temps = np.fromiter((s.temperature for s in batch.sequences), dtype=np.float32,
                            count=len(batch))
        tokens = sample_from_logits(logits, temps, self.generator)
        return batch, self.scheduler.finish_step(batch, [int(t) for t in tokens])

    def step(self) -> list[Sequence]:
        """Run one step; returns the sequences it finished."""
        return self._advance()[1]

    def run(self, max_steps: int = 100_000) -> list[Sequence]:
        """Step until every queued request finished (or ``max_steps``)."""
        finished: list[Sequence] = []
        steps = 0
        while steps < max_steps and self.scheduler.has_work:
            finished += self.step()
            steps += 1
        return finished

    def generate(self, prompts: list[list[int]], max_new_tokens: int = 32,
                 temperature: float = 1.0) -> list[list[int]]:
        """Serve ``prompts`` to completion; the generated tokens of each, in order."""
        seqs = [self.submit(p, max_new_tokens=max_new_tokens, temperature=temperature)
                for p in prompts]
        self.run()
        return [s.token_ids[s.num_prompt:] for s in seqs]
