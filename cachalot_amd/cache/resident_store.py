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

from ..storage.index import ExpertEntry, ExpertFormat, tensor_sizes_from_format
from .resident import ResidentExpert
from .slots import ExpertSlot, HBMSlotPool


# Transient slots a decode prediction leaves free for prefill's bypass loads
# (resident_store.py:50 of the reference).
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
    """Budgeted expert residency over one HBM slot pool.

    The constructor takes the reference's arguments (``resident_store.py:157-167``):
    ``budget_bytes`` sizes the resident set (``capacity = budget // expert bytes``);
    ``tensor_sizes`` ({short name: bytes}, ``tensor_sizes_from_entry``) lays out the
    slot record; ``transient_slots`` more slots (at least one) hold decode
    predictions and prefill bypass loads, which never count as residents;
    ``slot_pool`` brings a pool instead.  The runtime assigns ``.format`` after
    construction (``text_decode_runtime.py:442-453``); the setter checks it
    against the slot layout.  ``reader`` (an ``ExpertReader``) loads misses whose
    entry carries its byte ranges, unless a ``loader(entry, slot)`` is given.
    ``load_workers`` is accepted for the call site: loads here are single reads
    followed by copies enqueued on the caller's stream, not thread-pool jobs.

    Extensions for this build: ``fmt`` (the format up front), ``n_slots`` (the
    resident capacity in experts instead of a byte budget), ``n_layers`` /
    ``n_experts`` (the device slot table's shape) and ``device``."""

    def __init__(self, budget_bytes: int | None = None, reader=None, *,
                 tensor_sizes: dict[str, int] | None = None, slot_pool: HBMSlotPool | None = None,
                 transient_slots: int = 128, load_workers: int = 8, verbose: bool = False,
                 fmt: ExpertFormat | None = None, n_slots: int | None = None,
                 n_layers: int = 40, n_experts: int = 384, device="cuda",
                 loader: Callable[[ExpertEntry, ExpertSlot], None] | None = None) -> None:
        if slot_pool is None:
            if tensor_sizes is None:
                if fmt is None:
                    raise ValueError("tensor_sizes or slot_pool is required")
                tensor_sizes = tensor_sizes_from_format(fmt)
            expert_bytes = sum(tensor_sizes.values())
            if n_slots is None:
                if budget_bytes is None or budget_bytes <= 0:
                    raise ValueError("budget_bytes must be positive")
                n_slots = budget_bytes // expert_bytes
                if n_slots <= 0:
                    raise ValueError(f"budget {budget_bytes} smaller than one expert ({expert_bytes})")
            capacity = int(n_slots)
            if capacity <= 0:
                raise ValueError(f"n_slots must be positive, got {n_slots}")
            total = capacity + max(1, int(transient_slots))
            if verbose:
                print(f"Allocating {total} expert slots ({total * expert_bytes / 1024 ** 3:.1f} GiB) in HBM...",
                      flush=True)
            slot_pool = HBMSlotPool(fmt if fmt is not None else dict(tensor_sizes), total, device=device)
        else:
            expert_bytes = slot_pool.slot_bytes
            if n_slots is not None:
                capacity = min(int(n_slots), slot_pool.capacity - 1)
            elif budget_bytes is not None and budget_bytes > 0:
                capacity = min(budget_bytes // expert_bytes, slot_pool.capacity - 1)
            else:
                raise ValueError("budget_bytes must be positive")
            if capacity <= 0:
                raise ValueError(f"budget {budget_bytes} smaller than one expert ({expert_bytes})")
        self.pool = slot_pool
        self.capacity = int(capacity)
        self.transient_slots = self.pool.capacity - self.capacity
        self.expert_bytes = expert_bytes
        self.budget_bytes = self.capacity * expert_bytes
        self.load_workers = load_workers
        self.verbose = verbose
        if fmt is not None:
            self.format = fmt
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
        # predicted expert is loaded into a transient slot ahead of its layer and
        # becomes resident only when that layer requests it
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
        # transient slots in use: predictions in flight plus prefill bypass loads
        self._transient_count = 0
        # prefill: bypass loads held until release_prefill_layer, the layer plans
        # of prepare_prefill_layer, and the keys the current plan admits
        self._transients: dict[tuple[int, int], ExpertSlot] = {}
        self._prefill_layer_keys: dict[int, list[tuple[int, int]]] = {}
        self._prefill_admit: set[tuple[int, int]] = set()
        self.use_counts: dict[tuple[int, int], int] = {}

    # ---------------------------------------------------------------- format
    @property
    def format(self) -> ExpertFormat | None:
        return self.pool.format

    @format.setter
    def format(self, fmt: ExpertFormat) -> None:
        self.pool.set_format(fmt)

    def _load(self, entry: ExpertEntry, slot: ExpertSlot) -> None:
        """Fill ``slot`` with ``entry``'s bytes: the loader, else the reader for an
        indexed entry; an expert neither can produce is missing (KeyError, as
        ``moe_layer_metal.py:279-283``)."""
        if self.loader is not None:
            self.loader(entry, slot)
        elif self.reader is not None and entry.tensors:
            self.reader.read_expert_into(entry, slot.arrays)
        else:
            raise KeyError(f"Missing routed expert layer={entry.layer}, expert={entry.expert}")

    def _can_load(self, entry: ExpertEntry) -> bool:
        return self.loader is not None or (self.reader is not None and bool(entry.tensors))

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
        return key in self._items or key in self._transients

    def is_cached(self, key: tuple[int, int]) -> bool:
        return key in self._items

    def resident_keys(self) -> list[tuple[int, int]]:
        """Resident experts, least recently used first (transients excluded)."""
        return list(self._items)

    def layer_fully_resident(self, layer: int) -> bool:
        return bool((self._table[layer] >= 0).all())

    def preload(self, keys, fill: Callable[[tuple[int, int], ExpertSlot], None]) -> None:
        """Place `keys` in slots (slot = layer * n_experts + expert when the store holds every expert)."""
        bulk = self.capacity >= self.n_layers * self.n_experts
        for key in keys:
            if key in self._items:
                continue
            if bulk:
                slot = self.pool.acquire_index(key[0] * self.n_experts + key[1])
            else:
                slot = self._take_slot(protect=())
            fill(key, slot)
            self._admit(key, slot)
            self.stats.bytes_loaded += self.expert_bytes

    def _admit(self, key, slot: ExpertSlot) -> None:
        self._items[key] = slot
        self._set_table(key, slot.index)

    def _evict_lru(self, protect=(), avoid_layer: int | None = None) -> ExpertSlot | None:
        """Take the least recently used resident out of the table; its slot is
        returned to the caller (still marked in use)."""
        for pass_avoid in ((avoid_layer,) if avoid_layer is not None else ()) + (None,):
            for key in self._items:
                if key in protect or (pass_avoid is not None and key[0] == pass_avoid):
                    continue
                slot = self._items.pop(key)
                self._set_table(key, -1)
                self.stats.evictions += 1
                return slot
        return None

    def _take_slot(self, protect) -> ExpertSlot:
        """A slot for one more resident.  Residents never grow past ``capacity``:
        below it a free slot is taken (one always exists, since transients stay
        within their own count), at it the least recently used resident outside
        ``protect`` is evicted."""
        if len(self._items) < self.capacity:
            slot = self.pool.try_acquire()
            if slot is not None:
                return slot
        slot = self._evict_lru(protect)
        if slot is not None:
            return slot
        raise TimeoutError("every resident slot holds an expert of the current request")

    # ------------------------------------------------------ routing prediction
    def prefetch_decode(self, entries: list[ExpertEntry], limit: int | None = None) -> int:
        """Load experts predicted for an upcoming decode layer into transient
        slots, never evicting a resident and leaving ``predict_slot_reserve``
        transient slots to prefill (``resident_store.py:291-320`` of the
        reference).  Entries are taken in the caller's order, at most ``limit``
        (default DECODE_PREFETCH_LIMIT, 0 = no limit) per layer.  Returns how many
        loads were started."""
        cap = DECODE_PREFETCH_LIMIT if limit is None else limit
        per_layer: dict[int, int] = {}
        submitted = 0
        for entry in entries:
            if cap and per_layer.get(entry.layer, 0) >= cap:
                continue
            key = (entry.layer, entry.expert)
            if key in self._items or key in self._inflight or key in self._transients:
                continue
            if not self._can_load(entry):
                continue
            if self._transient_count >= self.transient_slots - self.predict_slot_reserve:
                break
            slot = self.pool.try_acquire()
            if slot is None:
                break
            self._transient_count += 1
            self._load(entry, slot)
            self._inflight[key] = (slot, entry)
            self._inflight_deadline[key] = (self._decode_pass, entry.layer)
            self.predicted_loads += 1
            submitted += 1
            per_layer[entry.layer] = per_layer.get(entry.layer, 0) + 1
        return submitted

    def note_decode_layer(self, layer: int) -> None:
        """A decode layer ran without asking the store for experts (a fully
        resident layer on the device path): the walk still advances, so the
        deadlines of predictions issued from it are counted from this layer."""
        self._advance_decode_pass(layer)

    def _advance_decode_pass(self, layer: int) -> None:
        """Decode requests layers in ascending order, once per token: a layer that
        does not advance starts a new walk (``resident_store.py:420-430``)."""
        if layer <= self._decode_layer:
            self._decode_pass += 1
        self._decode_layer = layer

    def _drop_prediction(self, key) -> ExpertSlot:
        slot, _ = self._inflight.pop(key)
        self._inflight_deadline.pop(key, None)
        self._transient_count -= 1
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

    def _wrap(self, key, slot, transient: bool = False) -> ResidentExpert:
        return ResidentExpert(layer=key[0], expert=key[1], slot=slot, transient=transient)

    def get(self, entry: ExpertEntry) -> ResidentExpert:
        return self.get_many([entry])[0]

    def get_many(self, entries: list[ExpertEntry], *, max_misses: int | None = None,
                 priorities: list[float] | None = None, prefetch: list[ExpertEntry] | None = None,
                 prefetch_limit: int | None = None, prefetch_after: bool | None = None,
                 on_hits=None) -> list[ResidentExpert | None]:
        """Resident experts for `entries`, in order; misses are loaded (strongest
        priority first) up to `max_misses`, the rest returned as None.  A miss
        that neither the loader nor the reader can fill raises KeyError, as
        ``moe_layer_forward`` does for a missing expert (``moe_layer_metal.py:279-283``).

        An entry predicted earlier (``prefetch_decode``) is admitted from its slot
        without a load.  ``prefetch`` (a list, or a callable returning one) names
        experts predicted for a later layer; they are loaded into transient slots
        after this layer's misses (``resident_store.py:789-943``), ``prefetch_limit``
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
        protect = set(keys)
        misses = []
        for i, key in enumerate(keys):
            self.use_counts[key] = self.use_counts.get(key, 0) + 1
            slot = self._items.get(key)
            if slot is None and key in self._inflight:
                # predicted earlier: its data already sits in a transient slot; the
                # slot turns resident (making room under capacity first), counted
                # as the miss it was
                slot, _ = self._inflight.pop(key)
                self._inflight_deadline.pop(key, None)
                self._transient_count -= 1
                if len(self._items) >= self.capacity:
                    victim = self._evict_lru(protect)
                    if victim is None:
                        raise TimeoutError("every resident slot holds an expert of the current request")
                    self.pool.release(victim)
                self._admit(key, slot)
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
            loaded = 0
            for i in misses:
                slot = self._items.get(keys[i])
                if slot is not None:        # a repeated key, loaded earlier in this call
                    out[i] = self._wrap(keys[i], slot)
                    continue
                if loaded >= budget:
                    continue
                loaded += 1
                if not self._can_load(entries[i]):
                    raise KeyError(f"Missing routed expert layer={keys[i][0]}, expert={keys[i][1]}")
                slot = self._take_slot(protect)
                self._load(entries[i], slot)
                self._admit(keys[i], slot)
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

    # ------------------------------------------------------------ prefill path
    def prepare_prefill_layer(self, layer_id: int, entries: list[ExpertEntry], *, num_layers: int = 40) -> None:
        """Fix this layer's resident set before its loads (``resident_store.py:954-1084``).

        The resident capacity is split evenly over ``num_layers`` (the first
        ``capacity % num_layers`` layers one more).  Of the experts the layer
        routes to, residents are kept first (the previous plan's, then the rest in
        request order), then misses are planned for admission in request order
        until the layer's share is full; the layer's other residents are evicted
        when this prompt's misses need their room, least recently used first.
        If admission would push the store past ``capacity``, other layers above
        their share give residents back (those their own plan does not name
        first).  Everything else the layer needs goes to transient slots in
        ``get_many_prefill``."""
        if num_layers <= 0:
            raise ValueError(f"num_layers must be > 0, got {num_layers}")
        order: list[tuple[int, int]] = []
        for e in entries:
            if e.layer != layer_id:
                raise ValueError(f"prepare_prefill_layer received entry layer={e.layer} for layer_id={layer_id}")
            if (e.layer, e.expert) not in order:
                order.append((e.layer, e.expert))
        share = lambda la: self.capacity // num_layers + (1 if la < self.capacity % num_layers else 0)  # noqa: E731
        quota = share(layer_id)
        needed = set(order)
        # earlier bypass loads that this layer does not need go back now
        self._release_transients(lambda k: k[0] != layer_id or k not in needed)
        if not order:
            self._prefill_layer_keys[layer_id] = []
            self._prefill_admit = set()
            return
        prev = [k for k in self._prefill_layer_keys.get(layer_id, []) if k in needed and k in self._items]
        kept = prev[:quota]
        kept += [k for k in order if k in self._items and k not in kept][:max(0, quota - len(kept))]
        # bypass loads this layer needs become residents while the share has room
        for k in order:
            if len(kept) >= quota or len(self._items) >= self.capacity:
                break
            if k in self._transients and k not in kept:
                self._admit(k, self._transients.pop(k))
                self._transient_count -= 1
                kept.append(k)
        missing = sum(1 for k in order if k not in kept)
        room = quota - len(kept) - missing      # share the prompt's misses leave to older residents
        if room > 0:
            for k in reversed(list(self._items)):
                if room <= 0:
                    break
                if k[0] == layer_id and k not in kept:
                    kept.append(k)
                    room -= 1
        keep = set(kept)
        for k in [k for k in self._items if k[0] == layer_id and k not in keep]:
            self.pool.release(self._items.pop(k))
            self._set_table(k, -1)
            self.stats.evictions += 1
        plan = list(kept)
        admit = set()
        for k in order:
            if len(plan) >= quota:
                break
            if k not in keep:
                plan.append(k)
                admit.add(k)
        over = len(self._items) + len(admit) - self.capacity
        for other in range(num_layers):
            if over <= 0:
                break
            if other == layer_id:
                continue
            theirs = [k for k in self._items if k[0] == other]
            extra = len(theirs) - share(other)
            if extra <= 0:
                continue
            named = set(self._prefill_layer_keys.get(other, []))
            for k in (sorted(k for k in theirs if k not in named) + sorted(k for k in theirs if k in named))[:extra]:
                if over <= 0:
                    break
                self.pool.release(self._items.pop(k))
                self._set_table(k, -1)
                self.stats.evictions += 1
                over -= 1
        if over > 0:
            raise RuntimeError(f"Unable to reclaim enough resident capacity for prepared prefill layer "
                               f"{layer_id}: short by {over} slots")
        self._prefill_layer_keys[layer_id] = plan
        self._prefill_admit = admit

    def get_many_prefill(self, entries: list[ExpertEntry], *,
                         speculate: list[ExpertEntry] | None = None) -> list[ResidentExpert]:
        """One prefill layer's experts without evicting a resident
        (``resident_store.py:1123-1210``): residents are returned as they are (LRU
        order untouched); a miss takes free resident capacity (admitted; with a
        prepared plan only the keys it admits), else a transient slot, held until
        ``release_prefill_layer``.  ``speculate`` (the next layer's likely experts)
        is loaded behind this layer's misses into whatever slots remain, never
        blocking.  Slot reuse is stream-ordered, so a released transient is
        refilled only after the kernels that read it."""
        out: list[ResidentExpert | None] = [None] * len(entries)
        requested = {(e.layer, e.expert) for e in entries}
        for i, e in enumerate(entries):
            key = (e.layer, e.expert)
            self.use_counts[key] = self.use_counts.get(key, 0) + 1
            slot = self._items.get(key)
            if slot is not None:
                self.stats.hits += 1
                out[i] = self._wrap(key, slot)
                continue
            slot = self._transients.get(key)
            if slot is not None:
                self.stats.hits += 1
                out[i] = self._wrap(key, slot, transient=True)
                continue
            if not self._can_load(e):
                raise KeyError(f"Missing routed expert layer={key[0]}, expert={key[1]}")
            slot, admit = self._prefill_slot(key, block=True, protect=requested)
            self._load(e, slot)
            self.stats.misses += 1
            self.stats.bytes_loaded += self.expert_bytes
            if admit:
                self._admit(key, slot)
            else:
                self._transients[key] = slot
            out[i] = self._wrap(key, slot, transient=not admit)
        for e in speculate or ():
            key = (e.layer, e.expert)
            if key in self._items or key in self._transients or not self._can_load(e):
                continue
            got = self._prefill_slot(key, block=False, protect=requested)
            if got is None:
                break
            slot, admit = got
            self._load(e, slot)
            self.stats.bytes_loaded += self.expert_bytes
            if admit:
                self._admit(key, slot)
            else:
                self._transients[key] = slot
        return out

    def _prefill_slot(self, key, *, block: bool, protect=()):
        """(slot, admit) for a prefill load: resident capacity when the plan allows
        it, else a transient slot; when both are exhausted, a blocking request
        makes room by evicting a resident outside ``protect`` (this call's experts),
        another layer's first (the one way to free a slot here, since releases are
        this thread's own)."""
        may_admit = not self._prefill_admit or key in self._prefill_admit
        if may_admit and len(self._items) < self.capacity:
            slot = self.pool.try_acquire()
            if slot is not None:
                return slot, True
        if self._transient_count < self.transient_slots:
            slot = self.pool.try_acquire()
            if slot is not None:
                self._transient_count += 1
                return slot, False
        if not block:
            return None
        slot = self._evict_lru(protect, avoid_layer=key[0])
        if slot is None:
            raise TimeoutError(f"no slot for prefill expert {key}: {self.capacity} resident and "
                               f"{self.transient_slots} transient slots are all in use")
        return slot, True

    def _release_transients(self, pred) -> None:
        for key in [k for k in self._transients if pred(k)]:
            self.pool.release(self._transients.pop(key))
            self._transient_count -= 1

    def release_prefill_layer(self, layer: int) -> None:
        """After a prefill layer's kernels are enqueued: free its transient slots
        (``resident_store.py:1212-1224``).  A later load into one is enqueued on the
        same stream, behind the kernels that read it."""
        self._release_transients(lambda k: k[0] == layer)

    def release_prefill(self) -> None:
        """End of a prefill (or an aborted one): nothing stays transient."""
        self._release_transients(lambda k: True)
        self._prefill_admit = set()

    def prefill_slot_table(self, layer: int, experts: list[ResidentExpert | None]) -> torch.Tensor:
        """The layer's device slot table with this call's transient experts added:
        what the prefill kernels address (residents through the store's table,
        bypass loads through their transient slots)."""
        row = self._table[layer].copy()
        for r in experts:
            if r is not None:
                row[r.expert] = r.slot.index
        return torch.from_numpy(row).to(self.pool.device, non_blocking=False)


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
