"""Expert-bank formats: how a routed expert's bytes are laid out.

Mirrors ``src/cachalot/storage/index.py:21-67``: ``ExpertEntry`` /
``TensorRange`` name a (layer, expert) and its tensors, ``ExpertFormat``
describes the slot views per short tensor name.  Two kinds:

* ``fp4``    -- the shipped checkpoint layout: ``w{1,2,3}.weight`` packed E2M1
  ``[N, K/2]`` u8 and ``w{1,2,3}.scale`` E8M0 ``[N, K/32]`` u8
  (``FP4_FORMAT``, ``storage/index.py:60-67``; per-layer checkpoint names
  ``layers.L.ffn.experts.E.wP.{weight,scale}``, ``:9-11``);
* ``affine`` -- MLX affine quantisation, stacked per layer in the bank:
  ``w{1,2,3}.weight`` u32 ``[N, Kp*bits/32]``, ``.scales`` / ``.biases``
  ``[N, Kp/group]`` bf16 (``storage/index.py:120-179``,
  ``benchmarks/build_affine_bank.py:72-97``).

Kp is K rounded up to a whole group.  At d_ff = 2880 with group 128 the down
projection's K is 22.5 groups; it is stored as 23 groups with zero codes past
K (the reference only ever ran K = 2304 = 18 groups, so this is this build's
extension of the layout, needed for the configured shapes).
"""
from __future__ import annotations

import json
import re
import struct
from dataclasses import dataclass, field
from pathlib import Path

PROJ_SHAPES = ("w1", "w2", "w3")


@dataclass(frozen=True)
class TensorRange:
    name: str
    shard: Path | None
    start: int
    end: int
    dtype: str | None = None                 # safetensors dtype of the source tensor, when indexed from a header
    shape: tuple[int, ...] | None = None     # this expert's slice shape

    @property
    def size(self) -> int:
        return self.end - self.start


@dataclass(frozen=True)
class ExpertEntry:
    layer: int
    expert: int
    tensors: tuple[TensorRange, ...] = field(default=())


@dataclass(frozen=True)
class ExpertFormat:
    kind: str
    bits: int
    group_size: int
    tensor_names: tuple[str, ...]
    shapes: dict[str, tuple[int, int]]
    dtypes: dict[str, str]
    d_model: int = 0
    d_ff: int = 0

    def tensor_bytes(self, name: str) -> int:
        rows, cols = self.shapes[name]
        return rows * cols * _ITEM_BYTES[self.dtypes[name]]

    @property
    def expert_bytes(self) -> int:
        """Stored bytes of one expert (padding included)."""
        return sum(self.tensor_bytes(n) for n in self.tensor_names)

    @property
    def algorithmic_bytes(self) -> int:
        """Bytes one expert pass must read at the unpadded shape: 3 * (D*F*bits/8
        + scale/bias bytes at D*F/group each).  9,953,280 B for the 2-bit g128
        expert at 4096 x 2880; 18,800,640 B for FP4 (``build_affine_bank.py:12-15``)."""
        d, f = self.d_model, self.d_ff
        if self.kind == "fp4":
            return 3 * (d * f // 2 + d * f // 32)
        per = d * f * self.bits // 8 + 2 * (d * f * _ITEM_BYTES[self.dtypes["w1.scales"]] // self.group_size)
        return 3 * per


_ITEM_BYTES = {"uint32": 4, "float32": 4, "float16": 2, "bfloat16": 2, "uint8": 1}

FP4_FORMAT = ExpertFormat(
    kind="fp4",
    bits=4,
    group_size=32,
    tensor_names=("w1.weight", "w1.scale", "w2.weight", "w2.scale", "w3.weight", "w3.scale"),
    shapes={},
    dtypes={},
)


def fp4_format(d_model: int, d_ff: int) -> ExpertFormat:
    """FP4_FORMAT with the slot shapes filled in for one model shape."""
    if d_model % 32 or d_ff % 32:
        raise ValueError(f"FP4 needs K divisible by 32 (d_model={d_model}, d_ff={d_ff})")
    shapes, dtypes = {}, {}
    for proj, (n, k) in (("w1", (d_ff, d_model)), ("w2", (d_model, d_ff)), ("w3", (d_ff, d_model))):
        shapes[f"{proj}.weight"] = (n, k // 2)
        shapes[f"{proj}.scale"] = (n, k // 32)
        dtypes[f"{proj}.weight"] = "uint8"
        dtypes[f"{proj}.scale"] = "uint8"
    return ExpertFormat("fp4", 4, 32, FP4_FORMAT.tensor_names, shapes, dtypes, d_model, d_ff)


def affine_format(d_model: int, d_ff: int, *, bits: int = 2, group_size: int = 128,
                  scale_dtype: str = "bfloat16") -> ExpertFormat:
    """Stacked-affine bank format (``storage/index.py:167-174``) for one model shape."""
    if bits != 2:
        raise ValueError(f"only the 2-bit affine bank is implemented (bits={bits})")
    if scale_dtype not in ("bfloat16", "float16"):
        raise ValueError(f"scale dtype {scale_dtype}")
    shapes, dtypes = {}, {}
    for proj, (n, k) in (("w1", (d_ff, d_model)), ("w2", (d_model, d_ff)), ("w3", (d_ff, d_model))):
        groups = -(-k // group_size)
        shapes[f"{proj}.weight"] = (n, groups * group_size * bits // 32)
        shapes[f"{proj}.scales"] = (n, groups)
        shapes[f"{proj}.biases"] = (n, groups)
        dtypes[f"{proj}.weight"] = "uint32"
        dtypes[f"{proj}.scales"] = scale_dtype
        dtypes[f"{proj}.biases"] = scale_dtype
    names = tuple(f"{p}.{f}" for p in PROJ_SHAPES for f in ("weight", "scales", "biases"))
    return ExpertFormat("affine", bits, group_size, names, shapes, dtypes, d_model, d_ff)


def tensor_sizes_from_format(fmt: ExpertFormat) -> dict[str, int]:
    return {n: fmt.tensor_bytes(n) for n in fmt.tensor_names}


# canonical kernel order of the nine record tensors (include/cachalot_amd.h)
KERNEL_ORDER = ("w1.weight", "w1.scales", "w1.biases", "w2.weight", "w2.scales", "w2.biases",
                "w3.weight", "w3.scales", "w3.biases")


def kernel_tensor_name(fmt: ExpertFormat, canonical: str) -> str | None:
    """Map a canonical name to the format's own (``.scale`` for FP4; no biases)."""
    if fmt.kind == "fp4":
        if canonical.endswith(".biases"):
            return None
        return canonical.replace(".scales", ".scale")
    return canonical


# ------------------------------------------------------------------ banks on disk
# Checkpoint tensor names (``storage/index.py:9-16``): the shipped FP4 checkpoint
# names every expert's tensors; oMLX-converted banks stack a layer's experts in
# one tensor per projection field, [n_experts, rows, cols].
_EXPERT_RE = re.compile(r"^layers\.(\d+)\.ffn\.experts\.(\d+)\.(w[123])\.(weight|scale)$")
_STACKED_RE = re.compile(r"^language_model\.layers\.(\d+)\.ffn\.experts\.(w[123])\.(weight|scales|biases)$")
_ST_ITEM_BYTES = {"U32": 4, "F32": 4, "F16": 2, "BF16": 2, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E8M0": 1}
_ST_DTYPE = {"U32": "uint32", "F32": "float32", "F16": "float16", "BF16": "bfloat16", "U8": "uint8"}


def read_safetensors_header(path: Path) -> tuple[dict, int]:
    """(header dict, byte offset of the data section) of a safetensors file (``storage/index.py:70-76``)."""
    with Path(path).open("rb") as f:
        header_len = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(header_len))
    return header, 8 + header_len


def build_expert_index(model_path: str | Path) -> dict[tuple[int, int], ExpertEntry]:
    """Per-expert tensors of the shipped FP4 checkpoint -> {(layer, expert): entry}, tensors in file
    order; unreadable shards are skipped (``storage/index.py:79-117``)."""
    root = Path(model_path)
    entries: dict[tuple[int, int], list[TensorRange]] = {}
    for shard in sorted(root.glob("model-*.safetensors")):
        try:
            header, data_start = read_safetensors_header(shard)
        except (OSError, json.JSONDecodeError, struct.error):
            continue
        for name, meta in header.items():
            m = _EXPERT_RE.match(name)
            if not m:
                continue
            a, b = meta["data_offsets"]
            entries.setdefault((int(m.group(1)), int(m.group(2))), []).append(
                TensorRange(name, shard, data_start + a, data_start + b, meta.get("dtype"),
                            tuple(meta.get("shape", ()))))
    return {k: ExpertEntry(k[0], k[1], tuple(sorted(v, key=lambda t: t.start))) for k, v in entries.items()}


def build_stacked_expert_index(model_path: str | Path, quantized_modules: dict) -> tuple[ExpertFormat, dict]:
    """oMLX-converted stacked affine bank -> (format, index); every expert's nine tensors are rows of
    the layer's stacked tensors (``storage/index.py:120-179``).  Mixed quantization, non-affine
    modules and inconsistent shapes raise ValueError."""
    root = Path(model_path)
    entries: dict[tuple[int, int], list[TensorRange]] = {}
    shapes: dict[str, tuple[int, int]] = {}
    dtypes: dict[str, str] = {}
    bits = group = None
    for shard in sorted(root.glob("model-*.safetensors")):
        try:
            header, data_start = read_safetensors_header(shard)
        except (OSError, json.JSONDecodeError, struct.error):
            continue
        for name, meta in header.items():
            m = _STACKED_RE.match(name)
            if not m:
                continue
            layer, proj, fld = int(m.group(1)), m.group(2), m.group(3)
            spec = quantized_modules.get(f"language_model.layers.{layer}.ffn.experts.{proj}")
            if spec is None or spec.get("mode") != "affine":
                raise ValueError(f"{name}: routed experts must be affine-quantized, got {spec}")
            this = (int(spec["bits"]), int(spec.get("group_size", 64)))
            if bits is None:
                bits, group = this
            elif this != (bits, group):
                raise ValueError(f"{name}: mixed expert quantization ({spec} vs {bits}-bit/{group})")
            n_exp, rows, cols = (int(v) for v in meta["shape"])
            short = f"{proj}.{fld}"
            if shapes.setdefault(short, (rows, cols)) != (rows, cols):
                raise ValueError(f"{name}: shape {(rows, cols)} differs from {shapes[short]}")
            dtypes[short] = _ST_DTYPE[meta["dtype"]]
            per = rows * cols * _ST_ITEM_BYTES[meta["dtype"]]
            base = data_start + meta["data_offsets"][0]
            for e in range(n_exp):
                entries.setdefault((layer, e), []).append(
                    TensorRange(f"layers.{layer}.ffn.experts.{e}.{short}", shard, base + e * per,
                                base + (e + 1) * per, meta["dtype"], (rows, cols)))
    if bits is None:
        raise ValueError(f"no stacked routed-expert tensors under {root}")
    rows1, cols1 = shapes["w1.weight"]
    d_model, d_ff = cols1 * 32 // bits, rows1
    fmt = ExpertFormat("affine", bits, group, tuple(sorted(shapes)), shapes, dtypes, d_model, d_ff)
    index = {k: ExpertEntry(k[0], k[1], tuple(sorted(v, key=lambda t: t.start))) for k, v in entries.items()}
    return fmt, index


def detect_expert_bank(model_path: str | Path) -> tuple[ExpertFormat, dict[tuple[int, int], ExpertEntry]]:
    """(format, index) of the routed experts under `model_path`: a stacked affine bank when
    config.json carries ``omlx_deepseek_v41``, else the shipped FP4 layout (``storage/index.py:182-194``).
    The FP4 format's shapes come from the first expert's w1 / w2 headers."""
    root = Path(model_path)
    config = root / "config.json"
    if config.exists():
        try:
            spec = json.loads(config.read_text()).get("omlx_deepseek_v41")
        except (OSError, json.JSONDecodeError):
            spec = None
        if spec:
            return build_stacked_expert_index(root, spec.get("quantized_modules", {}))
    index = build_expert_index(root)
    if not index:
        return FP4_FORMAT, index
    first = index[min(index)]
    by = {".".join(t.name.rsplit(".", 2)[-2:]): t for t in first.tensors}
    if "w1.weight" not in by or by["w1.weight"].shape is None or len(by["w1.weight"].shape) != 2:
        return FP4_FORMAT, index
    d_ff, half_d = by["w1.weight"].shape
    return fp4_format(half_d * 2, d_ff), index


@dataclass(frozen=True)
class ReadRange:
    shard: Path
    start: int
    end: int
    tensors: tuple[TensorRange, ...]

    @property
    def size(self) -> int:
        return self.end - self.start


def merge_contiguous_ranges(entry: ExpertEntry) -> tuple[ReadRange, ...]:
    """Runs of an entry's tensors that are adjacent in one shard, one read each (``storage/index.py:208-233``)."""
    groups: list[list[TensorRange]] = []
    for t in entry.tensors:
        if groups and groups[-1][-1].shard == t.shard and groups[-1][-1].end == t.start:
            groups[-1].append(t)
        else:
            groups.append([t])
    return tuple(ReadRange(g[0].shard, g[0].start, g[-1].end, tuple(g)) for g in groups)
