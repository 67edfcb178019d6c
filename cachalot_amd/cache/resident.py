"""ResidentExpert: a routed expert living in a pool slot.

Same accessors as ``src/cachalot/cache/resident.py:10-52``; the tensors are
uint8 device views that alias the slot record in HBM.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .slots import ExpertSlot


@dataclass(eq=False)
class ResidentExpert:
    layer: int
    expert: int
    slot: ExpertSlot
    transient: bool = False

    def _get(self, name: str) -> torch.Tensor:
        arrays = self.slot.arrays
        return arrays[name] if name in arrays else arrays[name.replace(".scale", ".scales")]

    @property
    def w1_weight(self) -> torch.Tensor:
        return self._get("w1.weight")

    @property
    def w1_scale(self) -> torch.Tensor:
        return self._get("w1.scale")

    @property
    def w2_weight(self) -> torch.Tensor:
        return self._get("w2.weight")

    @property
    def w2_scale(self) -> torch.Tensor:
        return self._get("w2.scale")

    @property
    def w3_weight(self) -> torch.Tensor:
        return self._get("w3.weight")

    @property
    def w3_scale(self) -> torch.Tensor:
        return self._get("w3.scale")

    @property
    def size(self) -> int:
        return self.slot.size

    @property
    def key(self) -> tuple[int, int]:
        return (self.layer, self.expert)

    def as_model_dict(self) -> dict[str, torch.Tensor]:
        return self.slot.arrays
