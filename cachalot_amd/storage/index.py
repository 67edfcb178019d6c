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

from dataclasses import dataclass, field
from pathlib import Path

PROJ_SHAPES = ("w1", "w2", "w3")


@dataclass(frozen=True)
class TensorRange:
    name: str
    shard: Path | None
    start: int
    end: int

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
