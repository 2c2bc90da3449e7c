"""Disaggregated prefill -> decode serving."""
from .disaggregated import (DecodeWorker, DirectSource, DisaggregatedEngine, DisaggregationStats,
                            KVTransfer, PrefillWorker)

__all__ = ["DecodeWorker", "DirectSource", "DisaggregatedEngine", "DisaggregationStats",
           "KVTransfer", "PrefillWorker"]
