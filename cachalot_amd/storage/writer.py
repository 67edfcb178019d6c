"""Bank writer: expert tensors -> safetensors shards the index and loader read.

The two on-disk layouts of ``storage/index.py``:

* stacked affine (``benchmarks/build_affine_bank.py:72-160,195-224``): one shard
  per layer, ``model-{layer+1:05d}-of-{n_layers:05d}.safetensors``, nine tensors
  ``language_model.layers.L.ffn.experts.wP.{weight,scales,biases}`` of shape
  ``[n_experts, rows, cols]`` (U32 codes, BF16 scales and biases) in the order
  w1, w2, w3 x weight, scales, biases; ``config.json`` carries
  ``omlx_deepseek_v41.quantized_modules`` with mode / bits / group_size per
  projection, which is what ``detect_expert_bank`` keys on;
* per-expert FP4 (the shipped checkpoint's naming, ``storage/index.py:9-11``):
  ``layers.L.ffn.experts.E.wP.{weight,scale}``, U8 packed E2M1 ``[N, K/2]`` and
  U8 E8M0 ``[N, K/32]``.

The header is JSON padded with spaces to a multiple of 8 bytes, data offsets
relative to the end of the header, as the safetensors format defines.  Experts
are written one at a time (``os.pwrite`` at their computed offsets), so a
writer never holds more than one expert.
"""
from __future__ import annotations

import json
import os
import struct
from pathlib import Path

import numpy as np

from .index import ExpertFormat

_ST = {"uint32": "U32", "bfloat16": "BF16", "float16": "F16", "uint8": "U8", "float32": "F32"}
_ITEM = {"U32": 4, "BF16": 2, "F16": 2, "U8": 1, "F32": 4}
PROJS = ("w1", "w2", "w3")


def shard_name(layer: int, n_layers: int) -> str:
    return f"model-{layer + 1:05d}-of-{n_layers:05d}.safetensors"


def _write_header(path: Path, header: dict) -> int:
    blob = json.dumps(header, separators=(",", ":")).encode()
    blob += b" " * ((-len(blob)) % 8)
    total = 8 + len(blob) + max((m["data_offsets"][1] for m in header.values()), default=0)
    with path.open("wb") as fh:
        fh.write(struct.pack("<Q", len(blob)))
        fh.write(blob)
        fh.truncate(total)
    return 8 + len(blob)


class StackedShardWriter:
    """One layer's stacked affine shard; ``put(expert, tensors)`` writes an expert's nine tensors."""

    def __init__(self, root: str | Path, layer: int, n_layers: int, n_experts: int, fmt: ExpertFormat) -> None:
        if fmt.kind != "affine":
            raise ValueError("stacked shards hold affine banks")
        self.fmt, self.layer, self.n_experts = fmt, layer, n_experts
        self.path = Path(root) / shard_name(layer, n_layers)
        header, self.offsets, off = {}, {}, 0
        for proj in PROJS:
            for fld in ("weight", "scales", "biases"):
                short = f"{proj}.{fld}"
                rows, cols = fmt.shapes[short]
                dt = _ST[fmt.dtypes[short]]
                size = n_experts * rows * cols * _ITEM[dt]
                name = f"language_model.layers.{layer}.ffn.experts.{short}"
                header[name] = {"dtype": dt, "shape": [n_experts, rows, cols], "data_offsets": [off, off + size]}
                self.offsets[short] = off
                off += size
        self.data_start = _write_header(self.path, header)
        self._fd = os.open(self.path, os.O_WRONLY)

    def put(self, expert: int, tensors: dict[str, np.ndarray]) -> None:
        for short, base in self.offsets.items():
            arr = np.ascontiguousarray(tensors[short])
            per = self.fmt.tensor_bytes(short)
            if arr.nbytes != per:
                raise ValueError(f"{short}: {arr.nbytes} bytes, the format has {per}")
            os.pwrite(self._fd, arr.view(np.uint8).tobytes(), self.data_start + base + expert * per)

    def close(self) -> None:
        os.close(self._fd)


def write_stacked_config(root: str | Path, fmt: ExpertFormat, n_layers: int, n_experts: int) -> None:
    modules = {f"language_model.layers.{la}.ffn.experts.{p}": {"bits": fmt.bits, "group_size": fmt.group_size,
                                                               "mode": "affine", "quantize_input": True}
               for la in range(n_layers) for p in PROJS}
    Path(root, "config.json").write_text(json.dumps({
        "omlx_deepseek_v41": {"version": 1, "quantized_modules": modules},
        "cachalot_bank": {"bits": fmt.bits, "group_size": fmt.group_size, "bytes_per_expert": fmt.expert_bytes,
                          "n_layers": n_layers, "n_experts": n_experts},
    }, indent=1))


def write_fp4_shard(path: str | Path, experts: dict[tuple[int, int], dict[str, np.ndarray]]) -> None:
    """Per-expert FP4 tensors ``{(layer, expert): {"w1.weight": u8 [N, K/2], "w1.scale": u8 [N, K/32], ...}}``."""
    header, blobs, off = {}, [], 0
    for (layer, expert), tensors in sorted(experts.items()):
        for proj in PROJS:
            for fld in ("weight", "scale"):
                arr = np.ascontiguousarray(tensors[f"{proj}.{fld}"], dtype=np.uint8)
                name = f"layers.{layer}.ffn.experts.{expert}.{proj}.{fld}"
                header[name] = {"dtype": "U8", "shape": list(arr.shape), "data_offsets": [off, off + arr.nbytes]}
                blobs.append(arr)
                off += arr.nbytes
    path = Path(path)
    start = _write_header(path, header)
    with path.open("r+b") as fh:
        fh.seek(start)
        for arr in blobs:
            fh.write(arr.tobytes())
