"""iekv — MI355X-native (gfx950 HIP) paged KV-cache handoff with the reference engine's API.

Layers:
  iekv.core      host bookkeeping (Sequence, BlockManager, KVTier, Scheduler, layout)
  iekv.engine    device pools, the HIP SlotCopier, the Engine, a toy paged model
  iekv.serve     PrefillWorker / DecodeWorker / DisaggregatedEngine
  iekv._native   ctypes binding of libiekv.so (include/iekv.h)
"""
__version__ = "0.1.0"
