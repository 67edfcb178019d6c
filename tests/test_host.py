"""Host-side checks that need no GPU: bank formats, record layout, the C-ABI
library's exports, argument validation, and the synthetic-data definitions
shared by the GPU generator and the oracle."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_expert_bytes_match_reference_counts():
    from cachalot_amd.storage.index import affine_format, fp4_format

    q2 = affine_format(4096, 2880)
    assert q2.algorithmic_bytes == 9_953_280            # build_affine_bank.py:12-15
    assert q2.expert_bytes == 10_027_008                # w2 padded to 23 groups
    assert q2.shapes["w2.weight"] == (4096, 184) and q2.shapes["w2.scales"] == (4096, 23)
    assert q2.shapes["w1.weight"] == (2880, 256) and q2.shapes["w1.scales"] == (2880, 32)
    fp4 = fp4_format(4096, 2880)
    assert fp4.expert_bytes == fp4.algorithmic_bytes == 18_800_640   # text_decode_runtime.py:347
    # the reference-true DeepSeek shape is group-aligned: no padding at all
    ds = affine_format(5120, 2304)
    assert ds.expert_bytes == ds.algorithmic_bytes == 9_953_280


def test_kernel_order_and_layout_offsets():
    from cachalot_amd.storage.index import KERNEL_ORDER, affine_format, fp4_format, kernel_tensor_name

    assert KERNEL_ORDER[0] == "w1.weight" and KERNEL_ORDER[4] == "w2.scales" and KERNEL_ORDER[8] == "w3.biases"
    fmt = fp4_format(64, 64)
    assert kernel_tensor_name(fmt, "w2.scales") == "w2.scale" and kernel_tensor_name(fmt, "w1.biases") is None
    q2 = affine_format(4096, 2880)
    # offsets the pool would use: page-aligned, in tensor order
    pos, offs = 0, {}
    for n in q2.tensor_names:
        offs[n] = pos
        pos += -(-q2.tensor_bytes(n) // 4096) * 4096
    assert all(o % 4096 == 0 for o in offs.values())
    assert pos == 10_027_008   # every tensor is already a whole number of pages


def _header_functions():
    text = (ROOT / "include/cachalot_amd.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int|size_t)\s+(cachalot_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from cachalot_amd import _lib

    declared = _header_functions()
    assert declared and set(declared) == set(_lib.exported_symbols())
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared:
        assert hasattr(handle, name), name


def test_library_validates_without_a_gpu():
    """Argument checks run on the host before any HIP call."""
    from cachalot_amd import _lib

    L = _lib.lib()
    assert L.cachalot_version() == 1
    rc = L.cachalot_router_topk(1, 1, 1, None, None, 0, 4096, 384, 6, 0, 1.0, 1.5, 1, 0, 1, 1, 1, None)
    assert rc == _lib.EINVAL and "at least one token" in _lib.last_error()
    rc = L.cachalot_router_topk(1, 1, 1, None, None, 1, 4096, 384, 400, 0, 1.0, 1.5, 1, 0, 1, 1, 1, None)
    assert rc == _lib.EINVAL and "topk" in _lib.last_error()
    rc = L.cachalot_router_topk(1, 1, 1, 1, None, 1, 4096, 384, 6, 0, 1.0, 1.5, 1, 0, 1, 1, 1, None)
    assert rc == _lib.EINVAL and "together" in _lib.last_error()
    with pytest.raises(ValueError):
        _lib.check(rc)
    lay = _lib.ExpertLayout()
    lay.record_bytes = 4096
    rc = L.cachalot_moe_decode_q2(1, 1, ctypes.byref(lay), 1, 1, 1, 4096, 2880, 384, 9, 128, 10.0, None, 1, None,
                                  1, 1 << 20, None)
    assert rc == _lib.EINVAL and "k=9" in _lib.last_error()
    need = L.cachalot_moe_decode_q2_workspace_bytes(4096, 2880, 6)
    assert need >= 6 * 2880 * 2   # at least the hidden activations
    rc = L.cachalot_moe_decode_q2(1, 1, ctypes.byref(lay), 1, 1, 1, 4096, 2880, 384, 6, 128, 10.0, None, 1, None,
                                  1, need - 1, None)
    assert rc == _lib.ESPACE
    with pytest.raises(MemoryError):
        _lib.check(rc)
    assert L.cachalot_dequant_fp4(1, 1, 4, 48, 0, 1, None) == _lib.EINVAL


def test_synth_keys_and_specs_agree_with_oracle():
    from cachalot_amd import synth
    from cachalot_amd.storage.index import affine_format, fp4_format
    from oracle import synth as osynth

    for args in [(0, 0, 0, 0), (20260917, 39, 383, 8), (1, 2, 1 << 20, 5), (2**63 + 5, 7, 11, 3)]:
        assert synth.stream_key(*args) == osynth.stream_key(*args)
    assert synth.TENSOR_IDS == osynth.TENSOR_IDS
    assert synth.IRWIN_HALL_STD == osynth.IRWIN_HALL_STD
    # the product's tensor specs equal the oracle's (name, kind, params, padding)
    for fmt, ospecs in ((affine_format(4096, 2880), osynth.q2_tensor_specs(4096, 2880)),
                        (fp4_format(4096, 2880), osynth.fp4_tensor_specs(4096, 2880))):
        prod = {s[0]: s[1:] for s in synth.tensor_specs(fmt)}
        for name, shape, dtype, kind, p0, p1, rt, rv in ospecs:
            assert prod[name] == (kind, p0, p1, rt, rv), name
            assert fmt.shapes[name] == shape


def test_oracle_synth_distributions():
    from oracle import synth as osynth
    from oracle.bf16 import bf16_bits_to_f32

    x = bf16_bits_to_f32(osynth.activations(1, 0, 8, 4096))
    assert abs(float(x.mean())) < 0.02 and abs(float(x.std()) - 1.0) < 0.02 and np.abs(x).max() < 3.47
    ex = osynth.expert_tensors(3, 1, 2, osynth.q2_tensor_specs(4096, 2880))
    s = bf16_bits_to_f32(ex["w1.scales"])
    assert s.min() >= 0.0049 and s.max() <= 0.0502
    assert np.all(ex["w2.weight"][:, 180:] == 0) and np.any(ex["w2.weight"][:, :180] != 0)
    f = osynth.expert_tensors(3, 1, 2, osynth.fp4_tensor_specs(4096, 2880))
    assert f["w1.scale"].min() == 119 and f["w1.scale"].max() == 127


def test_zipf_bias_is_a_permutation_of_ranks():
    from cachalot_amd.synth import zipf_bias

    b = zipf_bias(384, seed=5)
    ranks = sorted(b, reverse=True)
    assert ranks[0] == pytest.approx(0.5) and ranks[-1] == pytest.approx(0.5 * 384 ** -1.1)
    assert zipf_bias(384, seed=5) == b and zipf_bias(384, seed=6) != b


def test_get_many_loads_a_repeated_key_once():
    """A key named twice in one request is loaded once and both entries share its slot
    (a host-memory pool: the store's bookkeeping needs no GPU)."""
    from cachalot_amd.cache.resident_store import ResidentExpertStore
    from cachalot_amd.storage.index import ExpertEntry, affine_format

    loads = []
    store = ResidentExpertStore(fmt=affine_format(256, 128), n_slots=3, n_layers=1, n_experts=8, device="cpu",
                                loader=lambda entry, slot: loads.append((entry.layer, entry.expert, slot.index)))
    got = store.get_many([ExpertEntry(0, 2), ExpertEntry(0, 5), ExpertEntry(0, 2)])
    assert [g.expert for g in got] == [2, 5, 2] and got[0].slot is got[2].slot
    assert len(loads) == 2 and store.stats.misses == 2
    store.get_many([ExpertEntry(0, 6), ExpertEntry(0, 7)])        # both earlier slots can be reused now
    assert store.stats.misses == 4 and store.stats.evictions >= 1
    budget = store.get_many([ExpertEntry(0, 1), ExpertEntry(0, 1), ExpertEntry(0, 3)], max_misses=1)
    assert budget[0] is not None and budget[1].slot is budget[0].slot
    assert budget[2] is None


def test_predicted_experts_load_ahead_and_expire():
    """prefetch_decode loads predicted experts into free slots without making them
    resident; the layer that asks for one admits it without a load, and the rest expire
    once their layer has been requested or a new walk begins
    (resident_store.py:291-320,432-476,871-940 of the reference)."""
    from cachalot_amd.cache.resident_store import ResidentExpertStore
    from cachalot_amd.storage.index import ExpertEntry, affine_format

    loads = []
    store = ResidentExpertStore(fmt=affine_format(256, 128), n_slots=8, n_layers=3, n_experts=8, device="cpu",
                                loader=lambda entry, slot: loads.append((entry.layer, entry.expert)))
    store.predict_slot_reserve = 0
    assert store.prefetch_decode([ExpertEntry(1, 3), ExpertEntry(1, 4), ExpertEntry(1, 3)]) == 2
    assert loads == [(1, 3), (1, 4)] and not store.is_resident((1, 3)) and store.layer_table(1)[3] == -1
    store.get_many([ExpertEntry(0, 1)])                       # layer 0: layer-1 predictions are kept
    assert store.predicted_expired == 0 and len(loads) == 3
    got = store.get_many([ExpertEntry(1, 3), ExpertEntry(1, 5)])
    assert [g.expert for g in got] == [3, 5] and loads[3:] == [(1, 5)]   # (1, 3) admitted without a load
    assert store.is_resident((1, 3)) and store.layer_table(1)[3] == got[0].slot.index
    assert store.predicted_used == 1 and store.predicted_expired == 1   # (1, 4): its layer came and went
    assert store.predicted_wasted_bytes == store.expert_bytes and store.stats.misses == 3 == store.cache_misses
    # a layer that does not advance begins a new walk: older predictions expire
    store.prefetch_decode([ExpertEntry(2, 0), ExpertEntry(2, 1), ExpertEntry(2, 2)], limit=2)
    assert loads[-2:] == [(2, 0), (2, 1)] and store.predicted_loads == 4
    store.get_many([ExpertEntry(0, 1)])
    assert store.predicted_expired == 3
    # the prediction is issued after the demand loads, a callable only then
    order = []
    store.loader = lambda entry, slot: order.append((entry.layer, entry.expert))
    store.get_many([ExpertEntry(1, 6)], prefetch=lambda: [ExpertEntry(2, 7)])
    assert order == [(1, 6), (2, 7)]
    # the reserve: no prediction takes the last free slots
    store.predict_slot_reserve = store.pool.free_count()
    assert store.prefetch_decode([ExpertEntry(2, 5)]) == 0


def test_bench_cpu_dequant_equals_oracle():
    """The CPU baseline's table-driven dequant gives the oracle's values exactly."""
    import bench
    from cachalot_amd.storage.index import affine_format, fp4_format  # noqa: F401
    from oracle import synth as osynth
    from oracle.affine2 import dequantize_affine
    from oracle.fp4 import dequantize_fp4_weight

    t = osynth.expert_tensors(3, 0, 5, osynth.q2_tensor_specs(512, 320))
    for p, k in (("w1", 512), ("w2", 320)):
        got = bench._deq_q2_f32(t[f"{p}.weight"], t[f"{p}.scales"], t[f"{p}.biases"], k)
        want = dequantize_affine(t[f"{p}.weight"], t[f"{p}.scales"], t[f"{p}.biases"], k=k, group=128)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), p
    t = osynth.expert_tensors(3, 0, 5, osynth.fp4_tensor_specs(512, 320))
    got = bench._deq_fp4_f32(t["w2.weight"], t["w2.scale"])
    assert np.array_equal(got, dequantize_fp4_weight(t["w2.weight"], t["w2.scale"]))


def test_substitution_plan_follows_the_reference_rule():
    """Weakest non-resident experts under tau * total are replaced first, each by the best
    unused resident candidate; strong or resident experts stay; weights stay aligned."""
    from cachalot_amd.decode_substitution import plan_substitution, ranked_candidates, rescale_kept

    sel = np.array([0.9, 0.1, 0.8, 0.7, 0.2, 0.6, 0.5, 0.3], np.float32)
    assert ranked_candidates(sel, [0, 2, 3], 3) == [5, 6, 7]
    assert ranked_candidates(sel, [0, 2, 3], 0) == []
    tie = np.array([0.5, 0.5, 0.5, 0.1], np.float32)
    assert ranked_candidates(tie, [1], 2) == [0, 2]               # ties: lower id first
    resident = {0, 5, 7}
    ids, n = plan_substitution([0, 2, 3], [0.6, 0.1, 0.3], [5, 6, 7], lambda e: e in resident, tau=0.35)
    # expert 2 (share 0.1) is replaced by 5 (best resident); expert 3 (0.3 < 0.35) by 7; 0 is resident
    assert ids == [0, 5, 7] and n == 2
    ids, n = plan_substitution([0, 2, 3], [0.6, 0.1, 0.3], [5, 6, 7], lambda e: e in resident, tau=0.2)
    assert ids == [0, 5, 3] and n == 1                           # 3 holds 0.3 of the mass >= 0.2
    ids, n = plan_substitution([0, 2, 3], [0.6, 0.1, 0.3], [6], lambda e: e in resident, tau=0.5)
    assert ids == [0, 2, 3] and n == 0                           # no resident candidate
    ids, n = plan_substitution([1, 2], [0.0, 0.0], [5], lambda e: True, tau=0.5)
    assert ids == [1, 2] and n == 0                              # no routing mass
    w = rescale_kept([0.5, 0.25, 0.25], [0, 2])
    assert np.isclose(sum(w), 1.0) and np.isclose(w[0], 2 / 3) and np.isclose(w[1], 1 / 3)


def test_prediction_entries_strongest_first():
    """moe_layer_metal.py:236-244: predicted ids go to the store strongest first (route_topk's
    ascending order lists them weakest first; rank order strongest first), each layer's in turn,
    and an id the expert index does not hold is skipped."""
    import torch

    from cachalot_amd.moe_layer import prediction_entries
    from cachalot_amd.storage.index import ExpertEntry

    pred = [(3, torch.tensor([5, 9, 2])), (4, torch.tensor([7, 1, 8]))]
    got = prediction_entries(pred, None, "ascending")
    assert [(e.layer, e.expert) for e in got] == [(3, 2), (3, 9), (3, 5), (4, 8), (4, 1), (4, 7)]
    got = prediction_entries(pred, None, "rank")
    assert [(e.layer, e.expert) for e in got] == [(3, 5), (3, 9), (3, 2), (4, 7), (4, 1), (4, 8)]
    index = {(3, 5): ExpertEntry(3, 5), (3, 2): ExpertEntry(3, 2)}
    assert [(e.layer, e.expert) for e in prediction_entries(pred[:1], index, "ascending")] == [(3, 2), (3, 5)]


def test_layout_carries_the_scale_dtype():
    """The record descriptor tells the kernels how a 2-bit bank stores its scales;
    FP4 banks (E8M0 scales) send 0; other storage types are refused."""
    from cachalot_amd import _lib
    from cachalot_amd.cache.slots import HBMSlotPool
    from cachalot_amd.storage.index import affine_format, fp4_format

    for fmt, code in ((affine_format(256, 128), 0), (affine_format(256, 128, scale_dtype="float16"), 1),
                      (fp4_format(256, 128), 0)):
        assert HBMSlotPool(fmt, 1, device="cpu").layout().scale_dtype == code
    with pytest.raises(ValueError, match="bfloat16 or float16"):
        _lib.scale_dtype_code("float32")
