"""Engine-side pieces of the handoff: pools, the HIP copier, the engine and a toy model.

Modules that need torch or the HIP library (``pools``, ``copier``,
``toy_model``) are imported on use, so the host logic stays importable
without them.
"""
from .engine import Engine, EngineConfig, sample_from_logits

__all__ = ["Engine", "EngineConfig", "sample_from_logits"]
