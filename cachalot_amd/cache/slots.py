"""HBM-resident expert slot pool.

Mirrors ``SlabSlotPool`` (``src/cachalot/cache/slots.py:185-302``): every slot
is one contiguous record with each tensor at a fixed, page-aligned offset, so a
kernel reaches any resident expert from a slot index computed on the GPU
(``pool + slot * record_bytes + offset[t]``).  On MI355X the whole pool is one
device allocation (288 GB of HBM holds the full 2-bit bank: 15,360 x
10,027,008 B = 154 GB), so there are no slabs to juggle, no parking and no
per-slab buffer-binding limit.  ``ExpertSlot.arrays`` are zero-copy uint8 views
of the record, as the reference's ``slot.arrays`` alias slab memory
(``slots.py:240-251``).
"""
from __future__ import annotations

import threading
from collections import deque
from dataclasses import dataclass, field

import torch

from .. import _lib
from ..storage.index import KERNEL_ORDER, ExpertFormat, kernel_tensor_name

PAGE = 4096


@dataclass(eq=False)
class ExpertSlot:
    index: int
    arrays: dict[str, torch.Tensor]
    pool: "HBMSlotPool | None" = None
    typed: dict[str, tuple] = field(default_factory=dict)

    @property
    def size(self) -> int:
        return sum(a.numel() for a in self.arrays.values())


class HBMSlotPool:
    """``fmt`` is an ``ExpertFormat`` or, as the reference's ``ExpertSlotPool``
    takes it (``slots.py:68-108``), a {short name: bytes} dict; then the format
    (needed by the kernels' record descriptor and typed views) is set later with
    ``set_format``, which checks it against the record."""

    def __init__(self, fmt: ExpertFormat | dict[str, int], n_slots: int, *, device="cuda", page: int = PAGE) -> None:
        if n_slots <= 0:
            raise ValueError(f"n_slots must be positive, got {n_slots}")
        if isinstance(fmt, ExpertFormat):
            self.format: ExpertFormat | None = fmt
            self.tensor_sizes = {n: fmt.tensor_bytes(n) for n in fmt.tensor_names}
        else:
            self.format = None
            self.tensor_sizes = {str(n): int(b) for n, b in fmt.items()}
            if not self.tensor_sizes or min(self.tensor_sizes.values()) <= 0:
                raise ValueError(f"tensor sizes must be positive: {fmt}")
        self.tensor_names = tuple(self.tensor_sizes)
        self.slot_bytes = sum(self.tensor_sizes.values())
        self.offsets: dict[str, int] = {}
        pos = 0
        for name in self.tensor_names:
            self.offsets[name] = pos
            pos += -(-self.tensor_sizes[name] // page) * page
        self.record_bytes = pos
        self.device = torch.device(device)
        self.storage = torch.empty(n_slots * self.record_bytes, dtype=torch.uint8, device=self.device)
        self.n_slots = n_slots
        self._slots: dict[int, ExpertSlot] = {}   # views built on first use
        self._used = bytearray(n_slots)
        self._free: deque[int] = deque(range(n_slots))
        self._cond = threading.Condition()

    # ---------------------------------------------------------------- layout
    def set_format(self, fmt: ExpertFormat) -> None:
        """Attach the format to a pool laid out from tensor sizes; every tensor the
        format names must have a record slice of exactly its size."""
        got = {n: fmt.tensor_bytes(n) for n in fmt.tensor_names}
        if got != self.tensor_sizes:
            raise ValueError(f"format {fmt.kind} ({fmt.bits}-bit) tensors {got} do not match the slot "
                             f"record {self.tensor_sizes}")
        self.format = fmt

    def expert_format(self) -> ExpertFormat:
        if self.format is None:
            raise ValueError("the pool has no expert format yet (assign store.format first)")
        return self.format

    def _make_slot(self, i: int) -> ExpertSlot:
        base = i * self.record_bytes
        arrays = {n: self.storage[base + o: base + o + self.tensor_sizes[n]] for n, o in self.offsets.items()}
        return ExpertSlot(i, arrays, self)

    def layout(self) -> _lib.ExpertLayout:
        """The C-ABI record descriptor (tensor offsets in kernel order)."""
        fmt = self.expert_format()
        lay = _lib.ExpertLayout()
        lay.record_bytes = self.record_bytes
        lay.scale_dtype = _lib.scale_dtype_code(fmt.dtypes["w1.scales"]) if fmt.kind == "affine" else _lib.SCALE_BF16
        for i, canonical in enumerate(KERNEL_ORDER):
            name = kernel_tensor_name(fmt, canonical)
            lay.offset[i] = self.offsets[name] if name is not None else 0
        return lay

    @property
    def capacity(self) -> int:
        return self.n_slots

    def slot(self, index: int) -> ExpertSlot:
        s = self._slots.get(index)
        if s is None:
            if not 0 <= index < self.n_slots:
                raise IndexError(f"slot {index} outside 0..{self.n_slots - 1}")
            s = self._slots[index] = self._make_slot(index)
        return s

    def typed_view(self, slot: ExpertSlot, name: str) -> torch.Tensor:
        """A shaped, typed zero-copy view of one tensor of a slot."""
        dt = {"uint32": torch.int32, "uint8": torch.uint8, "bfloat16": torch.bfloat16,
              "float16": torch.float16, "float32": torch.float32}[self.expert_format().dtypes[name]]
        return slot.arrays[name].view(dt).view(self.format.shapes[name])

    # ------------------------------------------------------------ free list
    def _pop_free(self) -> int | None:
        while self._free:
            i = self._free.popleft()
            if not self._used[i]:
                self._used[i] = 1
                return i
        return None

    def try_acquire(self) -> ExpertSlot | None:
        with self._cond:
            i = self._pop_free()
        return None if i is None else self.slot(i)

    def acquire(self, timeout: float | None = None) -> ExpertSlot:
        with self._cond:
            if not self._cond.wait_for(lambda: self.free_count() > 0, timeout=timeout):
                raise TimeoutError("no free expert slot")
            i = self._pop_free()
        return self.slot(i)

    def free_count(self) -> int:
        return self.n_slots - sum(self._used)

    def release(self, slot: ExpertSlot) -> None:
        with self._cond:
            if self._used[slot.index]:
                self._used[slot.index] = 0
                self._free.append(slot.index)
            self._cond.notify()

    def acquire_index(self, index: int) -> ExpertSlot:
        """Take a specific free slot (bulk loading lays slots out as layer * E + expert)."""
        with self._cond:
            if self._used[index]:
                raise RuntimeError(f"slot {index} is in use")
            self._used[index] = 1
        return self.slot(index)
