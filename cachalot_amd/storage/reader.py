"""Bank loader: expert bytes from safetensors shards into the HBM slot pool.

Mirrors the reference's reader (``src/cachalot/storage/reader.py:50-250``):
``ExpertReader.read_expert`` / ``read_expert_into(entry, views)`` read an
expert's tensor ranges with ``os.preadv`` (contiguous tensors of one shard in
one call) into caller buffers named by short tensor name.  Here the buffers
are slot views in HBM, so the bytes land in a pinned staging buffer first and
go to the device with an asynchronous copy on the current stream.

``preload_bank`` is the MI355X addition: the whole bank is resident (288 GB of
HBM holds all 15,360 2-bit experts), so a stacked shard tensor
``[n_experts, rows, cols]`` is read in large runs and scattered into the slot
records with one 2-D copy per run (``cachalot_copy_records``: width = the
tensor's bytes per expert, destination pitch = the slot record), double
buffered so that the next run's reads overlap the previous run's copy.
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from pathlib import Path

import torch

from .. import _lib
from .index import ExpertEntry, ExpertFormat, affine_format, fp4_format, merge_contiguous_ranges


def short_name(tensor_name: str) -> str:
    """``layers.3.ffn.experts.7.w1.weight`` -> ``w1.weight`` (``reader.py:217``)."""
    return ".".join(tensor_name.rsplit(".", 2)[-2:])


def check_kernel_format(fmt: ExpertFormat) -> None:
    """The kernels read the layouts of ``affine_format`` / ``fp4_format``; a bank whose tensors differ
    (another group count, fp32 scales, a truncated last group) is rejected before any byte moves."""
    if fmt.kind == "affine":
        want = affine_format(fmt.d_model, fmt.d_ff, bits=fmt.bits, group_size=fmt.group_size,
                             scale_dtype=fmt.dtypes.get("w1.scales", "bfloat16"))
    elif fmt.kind == "fp4":
        want = fp4_format(fmt.d_model, fmt.d_ff)
    else:
        raise ValueError(f"unknown expert format {fmt.kind!r}")
    for name in want.tensor_names:
        if fmt.shapes.get(name) != want.shapes[name] or fmt.dtypes.get(name) != want.dtypes[name]:
            raise ValueError(f"bank tensor {name}: {fmt.dtypes.get(name)} {fmt.shapes.get(name)}, the kernels need "
                             f"{want.dtypes[name]} {want.shapes[name]} (d_model={fmt.d_model}, d_ff={fmt.d_ff})")


@dataclass(frozen=True)
class ReadChunk:
    shard: Path
    start: int
    data: bytes


class ExpertReader:
    """pread/preadv reader of expert byte ranges, one cached descriptor per shard."""

    def __init__(self) -> None:
        self._fds: dict[Path, int] = {}
        self._staging: torch.Tensor | None = None
        self._staging_done: torch.cuda.Event | None = None

    def _fd(self, path: Path) -> int:
        fd = self._fds.get(path)
        if fd is None:
            fd = self._fds[path] = os.open(path, os.O_RDONLY)
        return fd

    def close(self) -> None:
        for fd in self._fds.values():
            os.close(fd)
        self._fds.clear()

    def __enter__(self):
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def read_expert(self, entry: ExpertEntry) -> tuple[ReadChunk, ...]:
        chunks = []
        for rr in merge_contiguous_ranges(entry):
            data = os.pread(self._fd(rr.shard), rr.size, rr.start)
            if len(data) != rr.size:
                raise OSError(f"Short read from {rr.shard}: expected {rr.size}, got {len(data)}")
            chunks.append(ReadChunk(rr.shard, rr.start, data))
        return tuple(chunks)

    def _stage(self, nbytes: int) -> torch.Tensor:
        if self._staging_done is not None:
            self._staging_done.synchronize()          # the previous copy out of the staging buffer is done
        if self._staging is None or self._staging.numel() < nbytes:
            self._staging = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
        return self._staging[:nbytes]

    def read_expert_into(self, entry: ExpertEntry, views: dict[str, torch.Tensor]) -> int:
        """Read an expert into `views` (short name -> uint8 tensor of the tensor's size, host or device).
        Device views are filled from pinned staging by an async copy on the current stream.  Returns bytes read."""
        ranges = merge_contiguous_ranges(entry)
        targets = []
        for rr in ranges:
            for t in rr.tensors:
                name = short_name(t.name)
                if name not in views:
                    raise KeyError(f"no slot buffer for {name} ({t.name})")
                v = views[name]
                if v.numel() * v.element_size() != t.size:
                    raise ValueError(f"slot buffer for {name} has {v.numel() * v.element_size()} bytes, "
                                     f"tensor {t.name} has {t.size}")
                targets.append((t, v))
        on_device = any(v.is_cuda for _, v in targets)
        total = sum(rr.size for rr in ranges)
        stage = self._stage(total) if on_device else None
        pos = 0
        done = 0
        for rr in ranges:
            if on_device:
                bufs = [memoryview(stage[pos:pos + rr.size].numpy())]
            else:
                bufs = [memoryview(views[short_name(t.name)].view(torch.uint8).numpy()) for t in rr.tensors]
            got = os.preadv(self._fd(rr.shard), bufs, rr.start)
            if got != rr.size:
                raise OSError(f"Short read from {rr.shard}: expected {rr.size}, got {got}")
            pos += rr.size
            done += got
        if on_device:
            pos = 0
            for rr in ranges:
                off = 0
                for t in rr.tensors:
                    views[short_name(t.name)].view(torch.uint8).copy_(stage[pos + off: pos + off + t.size],
                                                                      non_blocking=True)
                    off += t.size
                pos += rr.size
            self._staging_done = torch.cuda.Event()
            self._staging_done.record()
        return done


class BankLoader:
    """``loader(entry, slot)`` for ``ResidentExpertStore``: reads the expert's bytes into the slot
    (the reference's ``reader.read_expert_into(entry, slot.views)``, ``resident_store.py:567``)."""

    def __init__(self, index: dict[tuple[int, int], ExpertEntry], reader: ExpertReader | None = None) -> None:
        self.index = index
        self.reader = reader or ExpertReader()

    def __call__(self, entry, slot) -> None:
        key = (entry.layer, entry.expert)
        full = entry if entry.tensors else self.index.get(key)
        if full is None:
            raise KeyError(f"Missing routed expert layer={key[0]}, expert={key[1]}")
        self.reader.read_expert_into(full, slot.arrays)

    def fill_key(self, key, slot) -> None:
        self(ExpertEntry(key[0], key[1]), slot)


def copy_records(pool, first_slot: int, name: str, src: torch.Tensor, n: int, stream=None) -> None:
    """Scatter n experts' bytes of one tensor (src: [n, tensor_bytes] contiguous, pinned host or device)
    into slots first_slot .. first_slot + n - 1 of an HBMSlotPool, one 2-D copy."""
    tb = pool.tensor_sizes[name]
    if src.numel() != n * tb:
        raise ValueError(f"{name}: {src.numel()} source bytes for {n} x {tb}")
    if first_slot < 0 or first_slot + n > pool.n_slots:
        raise IndexError(f"slots {first_slot}..{first_slot + n - 1} outside the pool")
    stream = stream if stream is not None else _lib.stream_handle(pool.device)
    rc = _lib.lib().cachalot_copy_records(pool.storage.data_ptr(), pool.record_bytes, pool.offsets[name], first_slot,
                                          src.data_ptr(), tb, n, stream)
    _lib.check(rc, "copy_records")


def preload_bank(store, index: dict[tuple[int, int], ExpertEntry], fmt: ExpertFormat | None = None, *,
                 layers=None, run_bytes: int = 256 << 20) -> int:
    """Load every indexed expert of `layers` into `store` (which must hold the whole bank: slot =
    layer * n_experts + expert).  Tensors whose per-expert ranges are consecutive in a shard (stacked
    banks) are read in runs of up to `run_bytes` and scattered with one 2-D copy per run; other
    tensors go expert by expert.  Returns bytes read."""
    fmt = fmt or store.format
    check_kernel_format(fmt)
    if store.capacity < store.n_layers * store.n_experts:
        raise ValueError("preload_bank needs a store that holds every expert; use BankLoader for partial residency")
    pool = store.pool
    keys = sorted(k for k in index if layers is None or k[0] in set(layers))
    # (layer, name) -> [(expert, TensorRange)]
    by_tensor: dict[tuple[int, str], list] = {}
    for key in keys:
        for t in index[key].tensors:
            by_tensor.setdefault((key[0], short_name(t.name)), []).append((key[1], t))
    stages = [torch.empty(run_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    events: list[torch.cuda.Event | None] = [None, None]
    reader = ExpertReader()
    total = 0
    turn = 0
    try:
        for (layer, name), items in sorted(by_tensor.items()):
            if name not in pool.tensor_sizes:
                raise KeyError(f"bank tensor {name} is not part of the slot format")
            tb = pool.tensor_sizes[name]
            if tb > run_bytes:
                raise ValueError(f"run_bytes {run_bytes} below one tensor ({tb})")
            items.sort()
            i = 0
            while i < len(items):
                # a run: consecutive experts whose ranges follow each other in one shard
                j = i + 1
                while (j < len(items) and (j - i + 1) * tb <= run_bytes and items[j][0] == items[j - 1][0] + 1
                       and items[j][1].shard == items[i][1].shard and items[j][1].start == items[j - 1][1].end):
                    j += 1
                n = j - i
                if events[turn] is not None:
                    events[turn].synchronize()
                buf = stages[turn][: n * tb]
                first = items[i][1]
                if first.size != tb:
                    raise ValueError(f"{first.name}: {first.size} bytes, the slot tensor has {tb}")
                got = os.preadv(reader._fd(first.shard), [memoryview(buf.numpy())], first.start)
                if got != n * tb:
                    raise OSError(f"Short read from {first.shard}: expected {n * tb}, got {got}")
                copy_records(pool, layer * store.n_experts + items[i][0], name, buf, n)
                ev = torch.cuda.Event()
                ev.record()
                events[turn] = ev
                turn ^= 1
                total += got
                i = j
        for key in keys:
            if key not in store._items:
                slot = pool.acquire_index(key[0] * store.n_experts + key[1])
                store._items[key] = slot
                store._set_table(key, slot.index)
                store.stats.bytes_loaded += store.expert_bytes
        torch.cuda.current_stream(pool.device).synchronize()
    finally:
        reader.close()
    return total
