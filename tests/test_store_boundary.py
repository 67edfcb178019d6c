"""The store's reference-facing contract on host-memory pools (no GPU needed):
the runtime's constructor call, transient slots for predictions, the decode walk
on device-path layers, and the prefill path for partial residency."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import oracle_tensors
from cachalot_amd.cache.prefetch import ResidentExpertPrefetcher
from cachalot_amd.cache.resident_store import ResidentExpertStore
from cachalot_amd.storage import index as I
from cachalot_amd.storage.reader import ExpertReader
from cachalot_amd.storage.writer import StackedShardWriter, write_stacked_config

L, E = 2, 6


def _bank(root, d=256, f=160):
    fmt = I.affine_format(d, f)
    for la in range(L):
        w = StackedShardWriter(root, la, L, E, fmt)
        for e in range(E):
            w.put(e, oracle_tensors(fmt, la, e))
        w.close()
    write_stacked_config(root, fmt, L, E)
    return fmt


def test_store_built_as_the_runtime_builds_it(tmp_path):
    """text_decode_runtime.py:442-453: budget, tensor sizes from an index entry,
    load workers and verbosity; the format is assigned afterwards; misses are read
    through the reader from the entry's byte ranges."""
    _bank(tmp_path)
    fmt, index = I.detect_expert_bank(tmp_path)
    sizes = I.tensor_sizes_from_entry(next(iter(index.values())))
    assert sizes == dict(sorted((n, fmt.tensor_bytes(n)) for n in fmt.tensor_names))
    store = ResidentExpertStore(budget_bytes=3 * fmt.expert_bytes, reader=ExpertReader(), tensor_sizes=sizes,
                                load_workers=4, verbose=False, n_layers=L, n_experts=E, device="cpu")
    assert store.capacity == 3 and store.transient_slots == 128 and store.format is None
    with pytest.raises(ValueError, match="no expert format"):
        store.pool.layout()
    store.format = fmt
    assert store.format is fmt and store.pool.layout().record_bytes == store.pool.record_bytes
    got = store.get_many([index[(1, 4)], index[(0, 2)]])
    for r in got:
        want = oracle_tensors(fmt, r.layer, r.expert)
        for name, arr in want.items():
            assert np.array_equal(r.slot.arrays[name].numpy(), arr.view(np.uint8).reshape(-1)), (r.key, name)
    # an index entry without byte ranges and no loader: missing
    with pytest.raises(KeyError):
        store.get_many([I.ExpertEntry(0, 5)])
    # a format whose tensors do not match the record is refused
    with pytest.raises(ValueError, match="do not match"):
        store.format = I.affine_format(512, 160)


def test_tensor_sizes_from_entry_needs_the_weights():
    r = I.TensorRange("layers.0.ffn.experts.1.w1.scales", None, 0, 10)
    with pytest.raises(ValueError, match="w1.weight"):
        I.tensor_sizes_from_entry(I.ExpertEntry(0, 1, (r,)))


def _loader_store(capacity, *, transient=128, n_layers=3, n_experts=8):
    loads = []
    store = ResidentExpertStore(fmt=I.affine_format(256, 128), n_slots=capacity, transient_slots=transient,
                                n_layers=n_layers, n_experts=n_experts, device="cpu",
                                loader=lambda entry, slot: loads.append((entry.layer, entry.expert, slot.index)))
    return store, loads


def test_predictions_still_load_when_the_residents_are_full():
    """Residents never grow into the transient slots, so a store filled to capacity
    still takes predictions (resident_store.py:291-320)."""
    store, loads = _loader_store(4, transient=20)
    store.get_many([I.ExpertEntry(0, e) for e in range(4)])
    store.get_many([I.ExpertEntry(0, e) for e in range(4, 8)])          # evicts: residents stay at 4
    assert len(store.resident_keys()) == 4 == store.capacity
    assert store.pool.free_count() == 20
    assert store.prefetch_decode([I.ExpertEntry(1, e) for e in range(8)]) == 4   # 20 - reserve 16
    assert store.pool.free_count() == 16 and len(store.resident_keys()) == 4
    # admitting a prediction keeps the resident count at capacity
    store.get_many([I.ExpertEntry(1, 0)])
    assert len(store.resident_keys()) == 4 and store.predicted_used == 1
    assert store.is_cached((1, 0)) and not store.is_cached((0, 4))


def test_device_path_layers_advance_the_walk():
    """Lead 2 with fully resident and partly resident layers alternating: a
    prediction issued on a device-path layer for two layers ahead survives the
    layer in between and is used by its target."""
    store, loads = _loader_store(6)
    store.predict_slot_reserve = 0
    for token in range(3):
        store.note_decode_layer(0)                                       # device path, layer 0
        assert store.prefetch_decode([I.ExpertEntry(2, token)]) == 1     # predicted for layer 2
        store.get_many([I.ExpertEntry(1, 7)])                            # host path, layer 1
        n = len(loads)
        got = store.get_many([I.ExpertEntry(2, token)])                  # host path, layer 2
        assert got[0].expert == token and len(loads) == n                # admitted without a load
    assert store.predicted_used == 3 and store.predicted_expired == 0


def test_prefill_without_a_plan_uses_free_capacity_then_transients():
    store, loads = _loader_store(4, transient=3, n_layers=2)
    got = store.get_many_prefill([I.ExpertEntry(0, e) for e in range(6)])
    assert [g.transient for g in got] == [False] * 4 + [True] * 2
    assert len(store.resident_keys()) == 4 and store._transient_count == 2
    table = store.prefill_slot_table(0, got)
    assert [int(v) for v in table[:6]] == [g.slot.index for g in got]
    assert int(store.layer_table(0)[5]) == -1                          # transients stay out of the store's table
    store.release_prefill_layer(0)
    assert store._transient_count == 0 and store.pool.free_count() == 3
    # residents are returned as hits without a load; misses past both pools evict
    # another layer's resident
    n = len(loads)
    again = store.get_many_prefill([I.ExpertEntry(0, e) for e in range(4)])
    assert len(loads) == n and all(not g.transient for g in again)
    store.get_many_prefill([I.ExpertEntry(1, e) for e in range(3)])      # fills the transients
    extra = store.get_many_prefill([I.ExpertEntry(1, 7)])                # no slot left: evicts a layer-0 resident
    assert not extra[0].transient and store.stats.evictions == 1
    store.release_prefill()
    assert store._transient_count == 0


def test_prepare_prefill_layer_plans_the_share():
    """resident_store.py:954-1084: each layer gets capacity / num_layers residents;
    needed residents stay, the plan admits misses in request order up to the
    share, the layer's unneeded residents go, the rest is transient."""
    store, loads = _loader_store(4, transient=8, n_layers=2)
    store.get_many([I.ExpertEntry(0, e) for e in (0, 1)])               # two residents of layer 0
    store.get_many([I.ExpertEntry(1, e) for e in (0, 1)])               # two of layer 1
    req = [I.ExpertEntry(0, e) for e in (1, 5, 6)]
    store.prepare_prefill_layer(0, req, num_layers=2)
    assert (0, 0) not in store.resident_keys()                          # not needed, room went to misses
    assert store._prefill_admit == {(0, 5)}                              # share 2: (0, 1) kept, (0, 5) admitted
    got = store.get_many_prefill(req)
    assert [g.transient for g in got] == [False, False, True]
    assert sorted(store.resident_keys()) == [(0, 1), (0, 5), (1, 0), (1, 1)]
    store.release_prefill_layer(0)
    assert store._transient_count == 0
    with pytest.raises(ValueError, match="layer=1"):
        store.prepare_prefill_layer(0, [I.ExpertEntry(1, 0)])


def test_prefetcher_interface():
    store, loads = _loader_store(2, transient=4, n_layers=2)
    pf = ResidentExpertPrefetcher(store, workers=3)
    assert pf.depth == 3 and pf.pending_count() == 0 and pf.pending_keys() == []
    assert pf.prefetch(I.ExpertEntry(0, 1)) is True
    assert pf.prefetch(I.ExpertEntry(0, 1)) is False                    # now resident
    assert pf.get(I.ExpertEntry(0, 1)).key == (0, 1)
    with pytest.raises(ValueError):
        ResidentExpertPrefetcher(store, workers=0)
