"""One expert over many rows: the reference's per-expert prefill entry points.

``routed_expert_forward_batched`` (``src/cachalot/model/moe_prefill_batched.py:31-61``),
``routed_expert_forward_sgmm`` (``fp4_sgmm_metal.py:318-333``, the same contract) and
``affine_expert_forward_batched`` (``expert_affine.py:84-99``) all return fp32
``[M, HIDDEN] = bf16(W2 bf16(silu(min(bf16 W1 x, L)) * clip(bf16 W3 x, -L, L) * w))``
for M rows of one expert, ``w`` the row's router weight.

They run the grouped expert kernels of ``moe_prefill.grouped_experts`` with one
route per row (k = 1), so the output is that path's, row for row: the combine of
one route is ``0 + y`` in fp32, the bf16 value of y as fp32, which is what the
reference's final ``.astype(mx.float32)`` of a bf16 product gives.

The kernels read an expert from a slot record of an ``HBMSlotPool``.  A
``ResidentExpert`` (``expert=``) is used in place.  The reference's keyword form
(``w1_packed=`` ...) passes bare tensors: they are copied into a one-slot pool
kept per device and shape (one expert's bytes per call) before the same
launch.
"""
from __future__ import annotations

import torch

from .cache.slots import HBMSlotPool
from .moe_prefill import grouped_experts
from .storage.index import ExpertFormat, fp4_format

_SCRATCH: dict[tuple, HBMSlotPool] = {}


def _rows(x: torch.Tensor, pool: HBMSlotPool, slot: int, weights: torch.Tensor, swiglu_limit: float) -> torch.Tensor:
    if x.ndim != 2 or x.shape[1] != pool.expert_format().d_model:
        raise ValueError(f"x must be [rows, {pool.expert_format().d_model}], got {tuple(x.shape)}")
    m = x.shape[0]
    w = torch.as_tensor(weights, dtype=torch.float32).reshape(-1)
    if w.numel() != m:
        raise ValueError(f"{w.numel()} weights for {m} rows")
    dev = pool.device
    table = torch.tensor([slot], dtype=torch.int32).to(dev)
    idx = torch.zeros((m, 1), dtype=torch.int32, device=dev)
    routed, _ = grouped_experts(x.to(device=dev, dtype=torch.bfloat16), idx, w.to(dev).reshape(m, 1), pool, table,
                               swiglu_limit=swiglu_limit, want_routed=True, want_out=False)
    return routed


def affine_expert_forward_batched(x: torch.Tensor, expert, fmt: ExpertFormat, weights: torch.Tensor,
                                  swiglu_limit: float = 10.0) -> torch.Tensor:
    """x [M, D], one resident 2-bit expert, weights [M] -> fp32 [M, D] (``expert_affine.py:84-99``)."""
    pool = expert.slot.pool
    if pool is None or pool.expert_format().kind != "affine" or fmt.kind != "affine":
        raise ValueError("affine_expert_forward_batched needs an expert of an affine bank")
    return _rows(x, pool, expert.slot.index, weights, swiglu_limit)


def _fp4_scratch(d_model: int, w1_packed: torch.Tensor, device) -> tuple[HBMSlotPool, ExpertFormat]:
    # D from x; F from W1's packed bytes (F rows of D / 2 bytes), so flat views work too
    w1_bytes = w1_packed.numel() * w1_packed.element_size()
    if d_model <= 0 or (2 * w1_bytes) % d_model:
        raise ValueError(f"w1_packed ({w1_bytes} bytes) is not F rows of {d_model // 2} bytes")
    fmt = fp4_format(d_model, 2 * w1_bytes // d_model)
    dev = torch.device(device)
    key = (dev.type, dev.index, fmt.d_model, fmt.d_ff)
    pool = _SCRATCH.get(key)
    if pool is None:
        pool = _SCRATCH[key] = HBMSlotPool(fmt, 1, device=dev)
    return pool, fmt


def routed_expert_forward_batched(x: torch.Tensor, *, w1_packed=None, w1_scales=None, w2_packed=None,
                                  w2_scales=None, w3_packed=None, w3_scales=None, weights=None,
                                  swiglu_limit: float = 10.0, expert=None) -> torch.Tensor:
    """x [M, HIDDEN], weights [M] -> fp32 [M, HIDDEN] for one FP4 expert
    (``moe_prefill_batched.py:31-61``).  The expert is either ``expert`` (a
    ResidentExpert of an FP4 pool, used in place) or the six packed tensors and
    their E8M0 scales in the checkpoint's layout (``w1_packed`` [F, D/2] uint8,
    ``w1_scales`` [F, D/32] uint8, ...), which are copied into a one-slot pool."""
    if weights is None:
        raise ValueError("weights (one router weight per row) are required")
    if expert is not None:
        pool = expert.slot.pool
        if pool is None or pool.expert_format().kind != "fp4":
            raise ValueError("expert must belong to an FP4 slot pool")
        return _rows(x, pool, expert.slot.index, weights, swiglu_limit)
    parts = {"w1.weight": w1_packed, "w1.scale": w1_scales, "w2.weight": w2_packed, "w2.scale": w2_scales,
             "w3.weight": w3_packed, "w3.scale": w3_scales}
    missing = [n for n, t in parts.items() if t is None]
    if missing:
        raise ValueError(f"missing expert tensors: {missing}")
    pool, fmt = _fp4_scratch(int(x.shape[-1]), w1_packed, x.device if x.is_cuda else "cuda")
    slot = pool.slot(0)
    for name, t in parts.items():
        src = t.contiguous().view(torch.uint8).reshape(-1)
        dst = slot.arrays[name]
        if src.numel() != dst.numel():
            raise ValueError(f"{name}: {src.numel()} bytes, the format of D {fmt.d_model} x F {fmt.d_ff} "
                             f"holds {dst.numel()}")
        dst.copy_(src.to(dst.device), non_blocking=True)
    return _rows(x, pool, 0, weights, swiglu_limit)


# fp4_sgmm_metal.py:318-333: "Same contract as moe_prefill_batched.routed_expert_forward_batched"
routed_expert_forward_sgmm = routed_expert_forward_batched
