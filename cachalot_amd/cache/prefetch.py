"""ResidentExpertPrefetcher: the prefill call sites' prefetcher handle.

Same interface as ``src/cachalot/io/resident_prefetch.py:12-120``
(``prefetch``, ``get``, ``depth``, ``workers``, ``pending_count``,
``discard_pending``, ``pending_keys``).  The reference hides SSD latency by
keeping ``depth`` expert reads in flight on worker threads.  Here a load is a
read plus copies enqueued on the caller's HIP stream, so a load "in flight" is
one already enqueued: ``prefetch`` issues it at once through the store's
prefill path (a transient slot, or admitted resident capacity) and nothing
stays pending.  ``moe_prefill_grouped`` takes the prefetcher's presence as the
signal to plan the layer's resident set (``prepare_prefill_layer``), as the
reference does.
"""
from __future__ import annotations

import os

from ..storage.index import ExpertEntry
from .resident import ResidentExpert


class ResidentExpertPrefetcher:
    def __init__(self, store, workers: int = 2, depth: int | None = None) -> None:
        if workers <= 0:
            raise ValueError(f"workers must be > 0, got {workers}")
        self.store = store
        self.workers = int(workers)
        env = os.environ.get("CACHALOT_PREFETCH_DEPTH")
        self.depth = int(depth) if depth else (int(env) if env else self.workers)
        self.issued = 0

    def prefetch(self, entry: ExpertEntry) -> bool:
        """Load the expert unless it is resident (or already held in a transient
        slot).  True when a load was issued, False when nothing was needed."""
        key = (entry.layer, entry.expert)
        if self.store.is_resident(key):
            return False
        self.store.get_many_prefill([entry])
        self.issued += 1
        return True

    def get(self, entry: ExpertEntry) -> ResidentExpert:
        return self.store.get_many_prefill([entry])[0]

    def pending_count(self) -> int:
        return 0

    def discard_pending(self, layer: int, keep: set[tuple[int, int]]) -> int:
        return 0

    def pending_keys(self) -> list[tuple[int, int]]:
        return []
