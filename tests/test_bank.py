"""Bank loader, host side: safetensors index, format detection, contiguous reads.

Banks are written by cachalot_amd.storage.writer from the seeded synthetic
experts (oracle/synth.py) in the reference's two on-disk layouts (stacked
affine, build_affine_bank.py:72-160; per-expert FP4, storage/index.py:9-11) and
read back through the index, so every byte is checked against its source.
"""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from helpers import oracle_tensors
from cachalot_amd.storage import index as I
from cachalot_amd.storage.reader import ExpertReader, check_kernel_format, short_name
from cachalot_amd.storage.writer import StackedShardWriter, write_fp4_shard, write_stacked_config

L, E = 2, 5


def _stacked_bank(root, d=256, f=160):
    fmt = I.affine_format(d, f)
    for la in range(L):
        w = StackedShardWriter(root, la, L, E, fmt)
        for e in range(E):
            w.put(e, oracle_tensors(fmt, la, e))
        w.close()
    write_stacked_config(root, fmt, L, E)
    return fmt


def test_stacked_bank_index_and_bytes(tmp_path):
    fmt = _stacked_bank(tmp_path)
    got_fmt, index = I.detect_expert_bank(tmp_path)
    assert (got_fmt.kind, got_fmt.bits, got_fmt.group_size, got_fmt.d_model, got_fmt.d_ff) == ("affine", 2, 128, 256, 160)
    assert got_fmt.shapes == fmt.shapes and got_fmt.dtypes == fmt.dtypes
    assert got_fmt.expert_bytes == fmt.expert_bytes
    check_kernel_format(got_fmt)
    assert sorted(index) == [(la, e) for la in range(L) for e in range(E)]
    with ExpertReader() as rd:
        for key, entry in index.items():
            want = oracle_tensors(fmt, *key)
            assert len(entry.tensors) == 9
            assert len(I.merge_contiguous_ranges(entry)) == 9          # one run per stacked tensor
            chunks = rd.read_expert(entry)
            by = {short_name(t.name): c.data for t, c in zip(entry.tensors, chunks)}
            for name, arr in want.items():
                assert by[name] == arr.tobytes(), (key, name)
            views = {n: torch.empty(fmt.tensor_bytes(n), dtype=torch.uint8) for n in fmt.tensor_names}
            assert rd.read_expert_into(entry, views) == fmt.expert_bytes
            for name, arr in want.items():
                assert np.array_equal(views[name].numpy(), arr.view(np.uint8).reshape(-1)), (key, name)


def test_fp4_bank_index_and_contiguous_read(tmp_path):
    fmt = I.fp4_format(256, 160)
    experts = {(la, e): oracle_tensors(fmt, la, e) for la in range(L) for e in range(E)}
    write_fp4_shard(tmp_path / "model-00001-of-00001.safetensors", experts)
    got_fmt, index = I.detect_expert_bank(tmp_path)
    assert got_fmt.kind == "fp4" and (got_fmt.d_model, got_fmt.d_ff) == (256, 160)
    check_kernel_format(got_fmt)
    entry = index[(1, 3)]
    assert len(I.merge_contiguous_ranges(entry)) == 1                  # six adjacent tensors, one read
    with ExpertReader() as rd:
        views = {n: torch.empty(fmt.tensor_bytes(n), dtype=torch.uint8) for n in fmt.tensor_names}
        rd.read_expert_into(entry, views)
    for name, arr in experts[(1, 3)].items():
        assert np.array_equal(views[name].numpy(), arr.reshape(-1)), name


def test_index_rejects_mixed_or_non_affine(tmp_path):
    _stacked_bank(tmp_path)
    cfg = json.loads((tmp_path / "config.json").read_text())
    mods = cfg["omlx_deepseek_v41"]["quantized_modules"]
    mods["language_model.layers.1.ffn.experts.w2"]["group_size"] = 64
    with pytest.raises(ValueError, match="mixed"):
        I.build_stacked_expert_index(tmp_path, mods)
    mods["language_model.layers.1.ffn.experts.w2"] = {"mode": "mxfp4", "bits": 4}
    with pytest.raises(ValueError, match="affine"):
        I.build_stacked_expert_index(tmp_path, mods)
    with pytest.raises(ValueError, match="no stacked"):
        I.build_stacked_expert_index(tmp_path / "nothing-here", {})


def test_unreadable_shard_is_skipped_and_short_layouts_rejected(tmp_path):
    fmt = _stacked_bank(tmp_path)
    (tmp_path / "model-00009-of-00009.safetensors").write_bytes(b"\x03")   # a shard still downloading
    _, index = I.detect_expert_bank(tmp_path)
    assert len(index) == L * E
    # a last group truncated instead of padded (cols // group at K = 2880) is not what the kernels read
    bad = I.ExpertFormat("affine", 2, 128, fmt.tensor_names, dict(fmt.shapes), dict(fmt.dtypes), 4096, 2880)
    bad.shapes.update({n: s for n, s in I.affine_format(4096, 2880).shapes.items()})
    bad.shapes["w2.scales"] = (4096, 22)
    with pytest.raises(ValueError, match="w2.scales"):
        check_kernel_format(bad)
