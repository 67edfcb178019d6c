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
