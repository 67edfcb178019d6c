"""Bank loader on the GPU: safetensors shards -> HBM slot pool.

A bank written from the seeded synthetic experts is loaded with preload_bank
(stacked runs scattered by one 2-D copy each) and with BankLoader under a
small pool (misses loaded by get_many); slot bytes must equal the source, and
a decode over the loaded bank must equal, bit for bit, the decode over the
same experts filled by the synthetic generator.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import SEED, make_store, oracle_tensors
from cachalot_amd.storage import index as I
from cachalot_amd.storage.writer import StackedShardWriter, write_fp4_shard, write_stacked_config

pytestmark = pytest.mark.gpu

L, E = 2, 8


def _write(root, fmt):
    if fmt.kind == "affine":
        for la in range(L):
            w = StackedShardWriter(root, la, L, E, fmt)
            for e in range(E):
                w.put(e, oracle_tensors(fmt, la, e))
            w.close()
        write_stacked_config(root, fmt, L, E)
    else:
        write_fp4_shard(root / "model-00001-of-00001.safetensors",
                        {(la, e): oracle_tensors(fmt, la, e) for la in range(L) for e in range(E)})


@pytest.mark.parametrize("kind", ["affine", "fp4"])
def test_preload_bank_bytes_and_decode(cuda, tmp_path, kind):
    from cachalot_amd.cache.resident_store import ResidentExpertStore
    from cachalot_amd.moe_decode import decode_experts
    from cachalot_amd.storage.reader import preload_bank

    fmt0 = I.affine_format(4096, 2880) if kind == "affine" else I.fp4_format(4096, 2880)
    _write(tmp_path, fmt0)
    fmt, index = I.detect_expert_bank(tmp_path)
    store = ResidentExpertStore(fmt=fmt, n_slots=L * E, n_layers=L, n_experts=E, device=cuda)
    nbytes = preload_bank(store, index, run_bytes=8 << 20)
    assert nbytes == L * E * fmt.expert_bytes
    for la, e in [(0, 0), (1, 5), (1, 7)]:
        slot = store.pool.slot(store.layer_table(la)[e].item())
        for name, arr in oracle_tensors(fmt0, la, e).items():
            assert np.array_equal(slot.arrays[name].cpu().numpy(), arr.view(np.uint8).reshape(-1)), (la, e, name)
    ref = make_store(fmt0, n_layers=L, n_experts=E)
    x = torch.randn(4096, device=cuda).to(torch.bfloat16)
    idx = torch.tensor([3, 0, 7, 5, 1, 6], dtype=torch.int32, device=cuda)
    w = torch.rand(6, device=cuda)
    for la in range(L):
        _, a = decode_experts(x, store.pool, store.layer_table(la), idx, w, want_routed=False, want_out=True)
        _, b = decode_experts(x, ref.pool, ref.layer_table(la), idx, w, want_routed=False, want_out=True)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), la


def test_bank_loader_fills_misses(cuda, tmp_path):
    from cachalot_amd.cache.resident_store import ResidentExpertStore
    from cachalot_amd.storage.reader import BankLoader

    fmt0 = I.affine_format(1024, 640)
    _write(tmp_path, fmt0)
    fmt, index = I.detect_expert_bank(tmp_path)
    store = ResidentExpertStore(fmt=fmt, n_slots=4, n_layers=L, n_experts=E, device=cuda, loader=BankLoader(index))
    keys = [(1, 2), (0, 7), (1, 6)]
    got = store.get_many([I.ExpertEntry(*k) for k in keys])
    torch.cuda.synchronize()
    assert store.stats.misses == 3
    for (la, e), res in zip(keys, got):
        for name, arr in oracle_tensors(fmt0, la, e).items():
            assert np.array_equal(res.slot.arrays[name].cpu().numpy(), arr.view(np.uint8).reshape(-1)), (la, e, name)
    # a fourth and fifth miss evict the least recently used
    store.get_many([I.ExpertEntry(0, 1), I.ExpertEntry(0, 3)])
    torch.cuda.synchronize()
    assert store.stats.evictions == 1 and not store.is_resident((1, 2))


def test_runtime_constructed_store_decodes(cuda, tmp_path):
    """The store built exactly as text_decode_runtime.py:442-453 builds it (budget,
    tensor sizes from an index entry, load workers, verbosity, then `.format =`)
    serves moe_layer_forward over a partly resident bank read through the reader;
    the output equals, bit for bit, the same layer over a fully resident store."""
    from cachalot_amd import synth
    from cachalot_amd.cache.resident_store import ResidentExpertStore
    from cachalot_amd.moe_layer import moe_layer_forward
    from cachalot_amd.storage.reader import ExpertReader

    fmt0 = I.affine_format(4096, 2880)
    _write(tmp_path, fmt0)
    fmt, index = I.detect_expert_bank(tmp_path)
    store = ResidentExpertStore(budget_bytes=6 * fmt.expert_bytes, reader=ExpertReader(),
                                tensor_sizes=I.tensor_sizes_from_entry(next(iter(index.values()))),
                                load_workers=8, verbose=False, n_layers=L, n_experts=E)
    store.format = fmt
    ref = make_store(fmt0, n_layers=L, n_experts=E)
    for step in range(3):
        la = step % L
        w, b = synth.router_weights(SEED, la, E, 4096, cuda)
        x = synth.activations(SEED, 90 + step, 1, 4096, cuda)[0]
        out, route = moe_layer_forward(x, layer_id=la, gate_weight=w, gate_bias=b, expert_index=index,
                                       expert_store=store, topk=6, route_scale=1.0, score_fn="sigmoid")
        want, route_ref = moe_layer_forward(x, layer_id=la, gate_weight=w, gate_bias=b, expert_index=None,
                                            expert_store=ref, topk=6, route_scale=1.0, score_fn="sigmoid")
        assert torch.equal(route.indices, route_ref.indices)
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), step
    assert store.stats.misses >= 6 and len(store.resident_keys()) <= 6


@pytest.mark.parametrize("planned", [False, True])
def test_prefill_partial_residency_matches_full(cuda, planned):
    """moe_prefill_grouped over a store that holds 8 of a layer's 32 experts: the
    rest go to transient slots (with a prefetcher, after prepare_prefill_layer
    plans the layer's share) and are released after the launches; the output
    equals the fully resident store's bit for bit, on two layers in a row."""
    from cachalot_amd.cache.prefetch import ResidentExpertPrefetcher
    from cachalot_amd.cache.resident_store import ResidentExpertStore, SyntheticLoader
    from cachalot_amd.moe_prefill import moe_prefill_grouped
    from oracle import synth as osynth

    d, f, nE, t = 512, 256, 32, 150
    fmt = I.affine_format(d, f)
    full = make_store(fmt, n_layers=2, n_experts=nE)
    part = ResidentExpertStore(fmt=fmt, n_slots=8, transient_slots=32, n_layers=2, n_experts=nE, device=cuda,
                               loader=SyntheticLoader(fmt, SEED))
    pf = ResidentExpertPrefetcher(part) if planned else None
    for la in (0, 1, 0):
        wb, bias = osynth.router_tensors(SEED, la, nE, d)
        xb = osynth.activations(SEED, 700 + la, t, d)
        kw = dict(layer_id=la, gate_weight=torch.from_numpy(wb.view(np.int16)).view(torch.bfloat16).to(cuda),
                  gate_bias=torch.from_numpy(bias).to(cuda), expert_index=None, topk=6, route_scale=1.0,
                  score_fn="sigmoid")
        x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(cuda)
        a, ra = moe_prefill_grouped(x, expert_store=part, expert_prefetcher=pf, **kw)
        b, rb = moe_prefill_grouped(x, expert_store=full, **kw)
        assert torch.equal(ra.indices, rb.indices)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), la
        assert part._transient_count == 0 and len(part.resident_keys()) <= 8
