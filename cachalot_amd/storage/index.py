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
    """Stacked-affine bank format (``storage/index.py:167-174``) for one model shape: 2, 3 or
    4 bits per code in groups of 32, 64 or 128 (the widths ``build_affine_bank.py:266-267``
    writes; oQ3e is 3-bit g64 with fp16 scales, ``expert_affine.py:1-4``)."""
    if bits not in (2, 3, 4) or group_size not in (32, 64, 128):
        raise ValueError(f"affine banks have 2, 3 or 4 bits in groups of 32, 64 or 128 "
                         f"(bits={bits}, group_size={group_size})")
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
# A bank on disk is a set of ``model-*.safetensors`` shards.  Two layouts name
# the routed experts (the names are the reference's, ``storage/index.py:9-16``):
#
#   per-expert  ``layers.L.ffn.experts.E.wP.{weight,scale}``: one tensor per
#               expert and field (the shipped FP4 checkpoint);
#   stacked     ``language_model.layers.L.ffn.experts.wP.{weight,scales,biases}``:
#               one ``[n_experts, rows, cols]`` tensor per layer and field (an
#               oMLX-converted affine bank), each expert a contiguous row block.
#
# Both are read the same way here: the shards are walked once, every tensor
# name is classified by one table (``_LAYOUTS``), and each match is cut into
# (layer, expert, short name) byte ranges: one range for a per-expert tensor,
# n_experts equal ranges for a stacked one.  The format (shapes, dtypes,
# quantization) is then inferred from the ranges, not from a second walk.


@dataclass(frozen=True)
class _Layout:
    """How one on-disk layout spells its expert tensors."""
    kind: str
    pattern: re.Pattern
    stacked: bool


_LAYOUTS = {
    "fp4": _Layout("fp4", re.compile(
        r"layers\.(?P<layer>\d+)\.ffn\.experts\.(?P<expert>\d+)\.(?P<proj>w[123])\.(?P<field>weight|scale)"), False),
    "affine": _Layout("affine", re.compile(
        r"language_model\.layers\.(?P<layer>\d+)\.ffn\.experts\.(?P<proj>w[123])\.(?P<field>weight|scales|biases)"), True),
}

# safetensors dtype tag -> (element bytes, slot dtype name); None = not a slot dtype
_ST_TYPES = {"U32": (4, "uint32"), "F32": (4, "float32"), "F16": (2, "float16"), "BF16": (2, "bfloat16"),
             "U8": (1, "uint8"), "I8": (1, None), "F8_E4M3": (1, None), "F8_E8M0": (1, None)}


def read_safetensors_header(path: Path) -> tuple[dict, int]:
    """(header dict, byte offset of the data section) of a safetensors file.  The file
    starts with a little-endian u64 header length, then that many bytes of JSON
    (the interface of ``storage/index.py:70-76``)."""
    with open(path, "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
        body = f.read(n)
    if len(body) != n:
        raise struct.error(f"{path}: header truncated ({len(body)} of {n} bytes)")
    return json.loads(body), 8 + n


def _readable_shards(root: Path):
    """(shard, header, data base) for every shard whose header parses.  A shard that
    is still being written (a partial download) is passed over, as the reference's
    indexer does, so a bank can be indexed while it is being fetched."""
    for shard in sorted(root.glob("model-*.safetensors")):
        try:
            header, base = read_safetensors_header(shard)
        except (OSError, ValueError, struct.error):
            continue
        yield shard, header, base


@dataclass
class _Piece:
    layer: int
    expert: int
    short: str
    rng: TensorRange


def _pieces(root: Path, layout: _Layout):
    """Every expert byte range the layout names under ``root``, with the tensor's
    metadata: yields (piece, header meta)."""
    for shard, header, base in _readable_shards(root):
        for name, meta in header.items():
            m = layout.pattern.fullmatch(name)
            if m is None:
                continue
            layer, short = int(m["layer"]), f"{m['proj']}.{m['field']}"
            start, end = (base + o for o in meta["data_offsets"])
            shape = tuple(int(v) for v in meta.get("shape", ()))
            if not layout.stacked:
                yield _Piece(layer, int(m["expert"]), short,
                             TensorRange(name, shard, start, end, meta.get("dtype"), shape)), meta
                continue
            n_exp, per_shape = shape[0], shape[1:]
            step = (end - start) // max(n_exp, 1)
            for e in range(n_exp):
                lo = start + e * step
                yield _Piece(layer, e, short,
                             TensorRange(f"layers.{layer}.ffn.experts.{e}.{short}", shard, lo, lo + step,
                                         meta.get("dtype"), per_shape)), meta


def _collect(pieces) -> dict[tuple[int, int], ExpertEntry]:
    """Group ranges by (layer, expert); each entry lists its tensors in file order."""
    by_key: dict[tuple[int, int], list[TensorRange]] = {}
    for p in pieces:
        by_key.setdefault((p.layer, p.expert), []).append(p.rng)
    return {key: ExpertEntry(key[0], key[1], tuple(sorted(rs, key=lambda r: (str(r.shard), r.start))))
            for key, rs in by_key.items()}


def build_expert_index(model_path: str | Path) -> dict[tuple[int, int], ExpertEntry]:
    """Per-expert tensors of the shipped FP4 checkpoint -> {(layer, expert): entry}
    (the interface of ``storage/index.py:79-117``)."""
    return _collect(p for p, _ in _pieces(Path(model_path), _LAYOUTS["fp4"]))


def _affine_spec(quantized_modules: dict, layer: int, proj: str) -> tuple[int, int]:
    """(bits, group size) the converter recorded for one stacked projection; MLX's
    default group size is 64.  Anything but affine quantization is refused."""
    spec = quantized_modules.get(f"language_model.layers.{layer}.ffn.experts.{proj}") or {}
    if spec.get("mode") != "affine":
        raise ValueError(f"layer {layer} {proj}: the routed experts are {spec or 'unquantized'}, "
                         "not affine-quantized")
    return int(spec["bits"]), int(spec.get("group_size", 64))


def build_stacked_expert_index(model_path: str | Path, quantized_modules: dict) -> tuple[ExpertFormat, dict]:
    """oMLX-converted stacked affine bank -> (format, index) (the interface of
    ``storage/index.py:120-179``).  Every projection must carry one affine
    (bits, group) and every field one slice shape and dtype across layers;
    otherwise ValueError."""
    root = Path(model_path)
    pieces, quant, shapes, dtypes = [], set(), {}, {}
    seen_tensor: set[tuple[Path, str, int]] = set()
    for piece, meta in _pieces(root, _LAYOUTS["affine"]):
        proj = piece.short.split(".")[0]
        tag = (piece.rng.shard, piece.short, piece.layer)
        if tag not in seen_tensor:      # per stacked tensor, not per expert slice
            seen_tensor.add(tag)
            quant.add(_affine_spec(quantized_modules, piece.layer, proj))
            if len(quant) > 1:
                raise ValueError(f"layer {piece.layer} {proj}: mixed expert quantization {sorted(quant)}")
            item, slot_dtype = _ST_TYPES.get(meta["dtype"], (None, None))
            if slot_dtype is None:
                raise ValueError(f"layer {piece.layer} {piece.short}: dtype {meta['dtype']} is not a bank dtype")
            if shapes.setdefault(piece.short, piece.rng.shape) != piece.rng.shape:
                raise ValueError(f"layer {piece.layer} {piece.short}: slice shape {piece.rng.shape}, "
                                 f"other layers have {shapes[piece.short]}")
            dtypes[piece.short] = slot_dtype
        pieces.append(piece)
    if not quant:
        raise ValueError(f"no stacked routed-expert tensors under {root}")
    (bits, group), = quant
    n_w1, words_w1 = shapes["w1.weight"]
    fmt = ExpertFormat("affine", bits, group, tuple(sorted(shapes)), shapes, dtypes,
                       d_model=words_w1 * 32 // bits, d_ff=n_w1)
    return fmt, _collect(pieces)


def detect_expert_bank(model_path: str | Path) -> tuple[ExpertFormat, dict[tuple[int, int], ExpertEntry]]:
    """(format, index) of the routed experts under ``model_path`` (the interface of
    ``storage/index.py:182-194``).  ``config.json`` with an ``omlx_deepseek_v41``
    block marks a stacked affine bank; anything else is read as the FP4 layout,
    whose shapes come from the first expert's ``w1.weight`` header."""
    root = Path(model_path)
    spec = None
    try:
        spec = json.loads((root / "config.json").read_text()).get("omlx_deepseek_v41")
    except (OSError, ValueError, AttributeError):
        pass
    if spec:
        return build_stacked_expert_index(root, spec.get("quantized_modules", {}))
    index = build_expert_index(root)
    w1 = next((t for t in index[min(index)].tensors if t.name.endswith(".w1.weight")), None) if index else None
    if w1 is None or w1.shape is None or len(w1.shape) != 2:
        return FP4_FORMAT, index
    d_ff, half_d = w1.shape
    return fp4_format(2 * half_d, d_ff), index


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
    """An entry's tensors as the fewest single reads: a new read starts wherever
    a tensor does not begin, in the same shard, at the byte the previous one ended
    (the interface of ``storage/index.py:208-233``)."""
    ts = entry.tensors
    cuts = [0] + [i for i in range(1, len(ts))
                  if (ts[i].shard, ts[i].start) != (ts[i - 1].shard, ts[i - 1].end)] + [len(ts)]
    return tuple(ReadRange(ts[a].shard, ts[a].start, ts[b - 1].end, ts[a:b])
                 for a, b in zip(cuts, cuts[1:]) if b > a)


def tensor_sizes_from_entry(entry: ExpertEntry) -> dict[str, int]:
    """{short name: bytes} of one indexed expert, sorted by name: what the runtime
    hands the store to size its slots (the interface of
    ``cache/resident_store.py:103-111``)."""
    sizes = {".".join(t.name.split(".")[-2:]): t.size for t in entry.tensors}
    lacking = sorted({"w1.weight", "w2.weight", "w3.weight"}.difference(sizes))
    if lacking:
        raise ValueError(f"expert ({entry.layer}, {entry.expert}) has no {', '.join(lacking)}")
    return dict(sorted(sizes.items()))
