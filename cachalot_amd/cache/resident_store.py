"""ResidentExpertStore over an HBM slot pool.

The reference store (``src/cachalot/cache/resident_store.py:157-1421``) keeps a
budgeted LRU of experts in wired memory and reads misses from SSD on loader
threads.  On MI355X the full bank is resident in HBM (``north_star``), so the
store's job shrinks to:

* placing every (layer, expert) in a slot once (``preload``), bulk-laid out
  as ``slot = layer * n_experts + expert`` when the pool holds the whole bank;
* keeping the ``(layer, expert) -> slot`` table (``track_slots``,
  ``resident_store.py:637-646``) as a device int32 tensor, so decode kernels
  address experts from GPU-computed router ids with no host round trip;
* answering ``get`` / ``get_many`` (``resident_store.py:789-943``) for callers
  that still address experts from the host, with LRU replacement through an
  optional ``loader(entry, slot)`` when the pool is smaller than the bank.

Slot reuse is stream-ordered: a refill is enqueued on the current stream after
every kernel that read the slot, which is the reference's "never overwrite a
slot before the ops that read it are evaluated" rule (``slots.py:15-18``)
expressed on one HIP stream.
"""
from __future__ import annotations

import os
from collections import OrderedDict
from dataclasses import dataclass
from typing import Callable

import numpy as np
import torch

from ..storage.index import ExpertEntry, ExpertFormat
from .resident import ResidentExpert
from .slots import ExpertSlot, HBMSlotPool


# Free slots a prediction leaves for the demand path (resident_store.py:52 of the reference).
PREDICT_SLOT_RESERVE = 16
# At most this many non-resident predicted experts per layer and call, in the
# caller's (ranked) order; 0 = no limit (resident_store.py:58).
DECODE_PREFETCH_LIMIT = int(os.environ.get("CACHALOT_DECODE_PREFETCH_LIMIT", "0"))


@dataclass
class ResidentStoreStats:
    hits: int = 0
    misses: int = 0
    bytes_loaded: int = 0
    evictions: int = 0


class ResidentExpertStore:
    def __init__(self, budget_bytes: int | None = None, reader=None, *, fmt: ExpertFormat, n_slots: int | None = None,
                 n_layers: int = 40, n_experts: int = 384, device="cuda",
                 loader: Callable[[ExpertEntry, ExpertSlot], None] | None = None) -> None:
        if n_slots is None:
            if budget_bytes is None or budget_bytes <= 0:
                raise ValueError("budget_bytes must be positive")
            n_slots = budget_bytes // fmt.expert_bytes
            if n_slots <= 0:
                raise ValueError(f"budget {budget_bytes} smaller than one expert ({fmt.expert_bytes})")
        self.format = fmt
        self.pool = HBMSlotPool(fmt, int(n_slots), device=device)
        self.capacity = self.pool.capacity
        self.expert_bytes = fmt.expert_bytes
        self.n_layers = n_layers
        self.n_experts = n_experts
        self.loader = loader
        self.reader = reader
        self.stats = ResidentStoreStats()
        self._items: OrderedDict[tuple[int, int], ExpertSlot] = OrderedDict()
        self._table = np.full((n_layers, n_experts), -1, np.int32)
        self._table_dev: torch.Tensor | None = None
        self.slot_table_version = 0
        # opt-in partial-residency approximations read by moe_layer_forward
        # (resident_store.py:272-276 of the reference; None = exact inference)
        self.decode_miss_budget: int | None = None
        self.decode_substitute_tau: float | None = None
        self.decode_substitute_ranks = 4
        self.substituted_experts = 0
        self.skipped_experts = 0
        # one-layer-early routing prediction (resident_store.py:230-262 of the
        # reference): layer -> (gate weight, gate bias), set by the runtime; a
        # predicted expert is loaded into a free slot ahead of its layer and becomes
        # resident only when that layer requests it
        self.decode_gates: dict[int, tuple] = {}
        self.predict_slot_reserve = PREDICT_SLOT_RESERVE
        self.predicted_loads = 0
        self.predicted_used = 0
        self.predicted_expired = 0
        self.predicted_wasted_bytes = 0
        self._inflight: dict[tuple[int, int], tuple[ExpertSlot, ExpertEntry]] = {}
        self._inflight_deadline: dict[tuple[int, int], tuple[int, int]] = {}
        self._decode_pass = 0
        self._decode_layer = -1

    # the reference's counters (resident_store.py:270-271), over this store's stats
    @property
    def cache_hits(self) -> int:
        return self.stats.hits

    @property
    def cache_misses(self) -> int:
        return self.stats.misses

    # ----------------------------------------------------------- slot table
    def track_slots(self, n_layers: int | None = None, n_experts: int | None = None) -> torch.Tensor:
        """Device int32 [layers, experts] table, -1 for a non-resident expert."""
        if n_layers is not None and n_experts is not None and (n_layers, n_experts) != self._table.shape:
            raise ValueError(f"table shape {(n_layers, n_experts)} != store shape {self._table.shape}")
        if self._table_dev is None:
            self._table_dev = torch.from_numpy(self._table).to(self.pool.device)
        return self._table_dev

    def layer_table(self, layer: int) -> torch.Tensor:
        return self.track_slots()[layer]

    def _set_table(self, key, slot: int) -> None:
        layer, expert = key
        self._table[layer, expert] = slot
        if self._table_dev is not None:
            self._table_dev[layer, expert] = slot
        self.slot_table_version += 1

    # ------------------------------------------------------------- residency
    def is_resident(self, key: tuple[int, int]) -> bool:
        return key in self._items

    is_cached = is_resident

    def layer_fully_resident(self, layer: int) -> bool:
        return bool((self._table[layer] >= 0).all())

    def preload(self, keys, fill: Callable[[tuple[int, int], ExpertSlot], None]) -> None:
        """Place `keys` in slots (slot = layer * n_experts + expert when the pool holds every expert)."""
        bulk = self.capacity >= self.n_layers * self.n_experts
        for key in keys:
            if key in self._items:
                continue
            if bulk:
                slot = self.pool.acquire_index(key[0] * self.n_experts + key[1])
            else:
                slot = self._take_slot(protect=())
            fill(key, slot)
            self._items[key] = slot
            self._set_table(key, slot.index)
            self.stats.bytes_loaded += self.expert_bytes

    def _take_slot(self, protect) -> ExpertSlot:
        slot = self.pool.try_acquire()
        if slot is not None:
            return slot
        for key in self._items:  # least recently used first
            if key not in protect:
                slot = self._items.pop(key)
                self._set_table(key, -1)
                self.stats.evictions += 1
                return slot
        for key in list(self._inflight):  # then a prediction nobody has asked for yet
            if key not in protect:
                return self._drop_prediction(key)
        raise TimeoutError("every slot holds an expert of the current request")

    # ------------------------------------------------------ routing prediction
    def prefetch_decode(self, entries: list[ExpertEntry], limit: int | None = None) -> int:
        """Load experts predicted for an upcoming decode layer into free slots,
        never evicting a resident and leaving ``predict_slot_reserve`` slots free
        (``resident_store.py:291-320`` of the reference).  Entries are taken in
        the caller's order, at most ``limit`` (default DECODE_PREFETCH_LIMIT, 0 =
        no limit) per layer.  Returns how many loads were started."""
        if self.loader is None:
            return 0
        cap = DECODE_PREFETCH_LIMIT if limit is None else limit
        per_layer: dict[int, int] = {}
        submitted = 0
        for entry in entries:
            if cap and per_layer.get(entry.layer, 0) >= cap:
                continue
            key = (entry.layer, entry.expert)
            if key in self._items or key in self._inflight:
                continue
            if self.pool.free_count() <= self.predict_slot_reserve:
                break
            slot = self.pool.try_acquire()
            if slot is None:
                break
            self.loader(entry, slot)
            self._inflight[key] = (slot, entry)
            self._inflight_deadline[key] = (self._decode_pass, entry.layer)
            self.predicted_loads += 1
            submitted += 1
            per_layer[entry.layer] = per_layer.get(entry.layer, 0) + 1
        return submitted

    def _advance_decode_pass(self, layer: int) -> None:
        """Decode requests layers in ascending order, once per token: a layer that
        does not advance starts a new walk (``resident_store.py:420-430``)."""
        if layer <= self._decode_layer:
            self._decode_pass += 1
        self._decode_layer = layer

    def _drop_prediction(self, key) -> ExpertSlot:
        slot, _ = self._inflight.pop(key)
        self._inflight_deadline.pop(key, None)
        self.predicted_expired += 1
        self.predicted_wasted_bytes += self.expert_bytes
        self.stats.bytes_loaded += self.expert_bytes
        return slot

    def _sweep_inflight(self, keep) -> None:
        """Give back the slots of predictions whose walk is over or whose target
        layer has already been requested (``resident_store.py:432-476``); a
        prediction for a layer this walk has not reached yet is kept."""
        for key in list(self._inflight):
            if key in keep:
                continue
            pass_id, target = self._inflight_deadline.get(key, (self._decode_pass, self._decode_layer))
            if pass_id == self._decode_pass and target > self._decode_layer:
                continue
            self.pool.release(self._drop_prediction(key))

    def _wrap(self, key, slot) -> ResidentExpert:
        return ResidentExpert(layer=key[0], expert=key[1], slot=slot)

    def get(self, entry: ExpertEntry) -> ResidentExpert:
        return self.get_many([entry])[0]

    def get_many(self, entries: list[ExpertEntry], *, max_misses: int | None = None,
                 priorities: list[float] | None = None, prefetch: list[ExpertEntry] | None = None,
                 prefetch_limit: int | None = None, prefetch_after: bool | None = None,
                 on_hits=None) -> list[ResidentExpert | None]:
        """Resident experts for `entries`, in order; misses are loaded (strongest
        priority first) up to `max_misses`, the rest returned as None.  Without a
        loader a miss raises KeyError, as ``moe_layer_forward`` does for a missing
        expert (``moe_layer_metal.py:279-283``).

        An entry predicted earlier (``prefetch_decode``) is admitted from its slot
        without a load.  ``prefetch`` (a list, or a callable returning one) names
        experts predicted for a later layer; they are loaded into free slots after
        this layer's misses (``resident_store.py:789-943``), ``prefetch_limit``
        capping them per layer.  Loads here are enqueued on the stream as they are
        issued, so ``prefetch_after`` (the reference's choice between issuing the
        prediction beside or after the demand reads) changes nothing and is only
        accepted."""
        keys = [(e.layer, e.expert) for e in entries]
        out: list[ResidentExpert | None] = [None] * len(keys)
        if keys:
            # decode asks for one layer at a time, so the first entry names it
            self._advance_decode_pass(keys[0][0])
        self._sweep_inflight(keep=set(keys))
        misses = []
        for i, key in enumerate(keys):
            slot = self._items.get(key)
            if slot is None and key in self._inflight:
                # predicted earlier: its data already sits in a slot, so it becomes
                # resident without a load (counted as the miss it was)
                slot, _ = self._inflight.pop(key)
                self._inflight_deadline.pop(key, None)
                self._items[key] = slot
                self._set_table(key, slot.index)
                self.predicted_used += 1
                self.stats.misses += 1
                self.stats.bytes_loaded += self.expert_bytes
                out[i] = self._wrap(key, slot)
                continue
            if slot is not None:
                self._items.move_to_end(key)
                self.stats.hits += 1
                out[i] = self._wrap(key, slot)
            else:
                misses.append(i)
        if on_hits is not None:
            on_hits([out[i] for i in range(len(keys)) if out[i] is not None])
        if misses:
            if priorities is not None:
                misses.sort(key=lambda i: -priorities[i])
            budget = len(misses) if max_misses is None else max(0, int(max_misses))
            unique_misses = len({keys[i] for i in misses})
            self.skipped_experts += max(0, unique_misses - budget)
            protect = set(keys)
            loaded = 0
            for i in misses:
                slot = self._items.get(keys[i])
                if slot is not None:        # a repeated key, loaded earlier in this call
                    out[i] = self._wrap(keys[i], slot)
                    continue
                if loaded >= budget:
                    continue
                loaded += 1
                if self.loader is None:
                    raise KeyError(f"Missing routed expert layer={keys[i][0]}, expert={keys[i][1]}")
                slot = self._take_slot(protect)
                self.loader(entries[i], slot)
                self._items[keys[i]] = slot
                self._set_table(keys[i], slot.index)
                self.stats.misses += 1
                self.stats.bytes_loaded += self.expert_bytes
                out[i] = self._wrap(keys[i], slot)
        if prefetch:
            # predicted experts of a later layer, after this layer's own loads have
            # their slots (a callable is evaluated only here)
            ents = prefetch() if callable(prefetch) else prefetch
            if ents:
                self.prefetch_decode(list(ents), prefetch_limit)
        return out


class SyntheticLoader:
    """loader(entry, slot) that writes the seeded synthetic expert (GPU fill)."""

    def __init__(self, fmt: ExpertFormat, seed: int, **spec_kw) -> None:
        self.fmt = fmt
        self.seed = seed
        self.spec_kw = spec_kw

    def __call__(self, entry, slot: ExpertSlot) -> None:
        from ..synth import fill_expert

        layer, expert = (entry.layer, entry.expert) if hasattr(entry, "layer") else entry
        fill_expert(slot.arrays, self.fmt, self.seed, layer, expert, **self.spec_kw)

    def fill_key(self, key, slot: ExpertSlot) -> None:
        self(ExpertEntry(key[0], key[1]), slot)
