"""Host-side block bookkeeping of the handoff: sequences, block manager, offload tier, scheduler."""
from .block_manager import BlockManager, BlockView, FreeList, PrefixPlan, chain_hash
from .layout import BatchLayout, build_layout, slot_for_position
from .offload import KVTier, SlotCopier, TierEntry, TierStats
from .scheduler import Batch, Scheduler, SchedulerStats
from .sequence import BlockGeometry, Sequence, Status

__all__ = ["Batch", "BatchLayout", "BlockGeometry", "BlockManager", "BlockView", "FreeList",
           "KVTier", "PrefixPlan", "Scheduler", "SchedulerStats", "Sequence", "SlotCopier",
           "Status", "TierEntry", "TierStats", "build_layout", "chain_hash",
           "slot_for_position"]
