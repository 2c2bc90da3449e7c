"""Host-side block bookkeeping of the handoff: sequences, block manager, offload tier, scheduler."""
from .block_manager import Block, BlockManager, chain_hash
from .layout import BatchLayout, build_layout, slot_for_position
from .offload import KVTier, SlotCopier, TierStats
from .scheduler import Batch, Scheduler, SchedulerStats
from .sequence import Sequence, Status

__all__ = ["Batch", "BatchLayout", "Block", "BlockManager", "KVTier", "Scheduler",
           "SchedulerStats", "Sequence", "SlotCopier", "Status", "TierStats", "build_layout",
           "chain_hash", "slot_for_position"]
