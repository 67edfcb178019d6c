"""Device-addressed decode of the top-k routed experts (one token).

``decode_experts`` is the single entry the reference-shaped wrappers below and
``moe_layer_forward`` share: experts are named by router ids on the device and
resolved through the store's slot table inside the kernels, so nothing crosses
to the host between routing and the expert GEMVs.

* ``fused_routed_experts``  -- ``src/cachalot/model/moe_fused_metal.py:189-233`` (FP4 bank)
* ``affine_routed_experts`` -- ``src/cachalot/model/expert_affine.py:186-206`` (2-bit bank)
* ``affine_expert_forward`` -- ``expert_affine.py:65-81`` (one expert)
"""
from __future__ import annotations

import torch

from . import _lib
from .cache.slots import HBMSlotPool
from .router import RouterResult
from .storage.index import ExpertFormat

_WORKSPACES: dict[tuple, torch.Tensor] = {}


def is_q2_g128(fmt: ExpertFormat) -> bool:
    """The 2-bit g128 bank, which has matrix-core kernels; other affine widths (3 / 4 bits,
    groups of 32 / 64) take the generic affine kernels (csrc/affine.hip)."""
    return fmt.kind == "affine" and fmt.bits == 2 and fmt.group_size == 128


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """The decode scratch workspace, cached per device (grown on demand).

    Decode calls on one device share it and must therefore be ordered (one
    stream, or streams that wait on each other); a HIP-graph capture must be
    preceded by an eager call of the same shape so that the workspace exists
    before capture.  A new workspace is zero-filled: the bf16-MFMA layer decode keeps
    a completion counter in its first bytes that must start at zero (every call
    leaves it zero)."""
    key = (device.index,)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def decode_experts(x: torch.Tensor, pool: HBMSlotPool, slot_table: torch.Tensor, idx: torch.Tensor,
                   weights: torch.Tensor, *, swiglu_limit: float = 10.0, addend: torch.Tensor | None = None,
                   want_routed: bool = True, want_out: bool = True):
    """x [D] bf16; slot_table [E] int32 (device); idx [k] int32; weights [k] fp32.

    Returns (routed fp32 [D] or None, out bf16 [D] or None)."""
    fmt: ExpertFormat = pool.expert_format()
    if x.ndim != 1:
        raise ValueError(f"x must be 1D for decode, got {tuple(x.shape)}")
    if x.dtype != torch.bfloat16:
        raise TypeError("decode expects bf16 activations")
    d, f = fmt.d_model, fmt.d_ff
    if x.shape[0] != d:
        raise ValueError(f"x has {x.shape[0]} elements, experts expect {d}")
    k = int(idx.numel())
    if weights.numel() != k:
        raise ValueError(f"{weights.numel()} router weights for {k} experts")
    _lib.require_cuda(x, slot_table, idx, weights, addend)
    dev = x.device
    idx = idx.to(torch.int32).contiguous()
    weights = weights.to(torch.float32).contiguous()
    slot_table = slot_table.to(torch.int32).contiguous()
    x = x.contiguous()
    if addend is not None:
        if addend.dtype != torch.bfloat16 or addend.shape != x.shape:
            raise ValueError("addend must be a bf16 vector shaped like x")
        addend = addend.contiguous()
    routed = torch.empty((d,), dtype=torch.float32, device=dev) if want_routed else None
    out = torch.empty((d,), dtype=torch.bfloat16, device=dev) if want_out else None
    L = _lib.lib()
    layout = pool.layout()
    stream = _lib.stream_handle(dev)
    e = int(slot_table.numel())
    if fmt.kind == "affine" and not is_q2_g128(fmt):
        nbytes = L.cachalot_moe_decode_affine_workspace_bytes(d, f, k)
        ws = workspace(dev, nbytes)
        rc = L.cachalot_moe_decode_affine(x.data_ptr(), pool.storage.data_ptr(), layout, slot_table.data_ptr(),
                                          idx.data_ptr(), weights.data_ptr(), d, f, e, k, fmt.bits, fmt.group_size,
                                          float(swiglu_limit), _lib.ptr(addend), _lib.ptr(routed), _lib.ptr(out),
                                          ws.data_ptr(), nbytes, stream)
        _lib.check(rc, "moe_decode_affine")
    elif fmt.kind == "affine":
        nbytes = L.cachalot_moe_decode_q2_workspace_bytes(d, f, k)
        ws = workspace(dev, nbytes)
        rc = L.cachalot_moe_decode_q2(x.data_ptr(), pool.storage.data_ptr(), layout, slot_table.data_ptr(),
                                      idx.data_ptr(), weights.data_ptr(), d, f, e, k, fmt.group_size,
                                      float(swiglu_limit), _lib.ptr(addend), _lib.ptr(routed), _lib.ptr(out),
                                      ws.data_ptr(), nbytes, stream)
        _lib.check(rc, "moe_decode_q2")
    elif fmt.kind == "fp4":
        nbytes = L.cachalot_moe_decode_fp4_workspace_bytes(d, f, k)
        ws = workspace(dev, nbytes)
        rc = L.cachalot_moe_decode_fp4(x.data_ptr(), pool.storage.data_ptr(), layout, slot_table.data_ptr(),
                                       idx.data_ptr(), weights.data_ptr(), d, f, e, k, float(swiglu_limit),
                                       _lib.ptr(addend), _lib.ptr(routed), _lib.ptr(out), ws.data_ptr(), nbytes,
                                       stream)
        _lib.check(rc, "moe_decode_fp4")
    else:
        raise ValueError(f"unknown expert format {fmt.kind!r}")
    return routed, out


def moe_layer_decode(x: torch.Tensor, gate_weight: torch.Tensor, gate_bias: torch.Tensor, pool: HBMSlotPool,
                     slot_table: torch.Tensor, *, topk: int = 6, gate_temp: float = 1.0, route_scale: float = 1.5,
                     norm_topk_prob: bool = True, score_fn: str = "sqrt_softplus", order: str = "ascending",
                     swiglu_limit: float = 10.0, addend: torch.Tensor | None = None, want_routed: bool = False,
                     want_out: bool = True, shared: dict | None = None):
    """One token through one MoE layer with routing on the device (three launches).

    ``shared``: the layer's FP8 shared expert as ``shared_args`` bundles it;
    out = bf16(routed + shared expert), the shared expert's tiles carried by the
    routed launches where the shapes allow (``moe_layer_metal.py:381-397``).

    Returns (routed fp32 [D] or None, out bf16 [D] or None, RouterResult)."""
    fmt: ExpertFormat = pool.expert_format()
    d, f = fmt.d_model, fmt.d_ff
    if x.ndim != 1 or x.shape[0] != d:
        raise ValueError(f"x must be 1D with {d} elements, got {tuple(x.shape)}")
    if x.dtype != torch.bfloat16 or gate_weight.dtype != torch.bfloat16:
        raise TypeError("decode expects bf16 activations and a bf16 gate weight")
    n_experts = gate_weight.shape[0]
    if tuple(gate_weight.shape) != (n_experts, d) or tuple(gate_bias.shape) != (n_experts,):
        raise ValueError(f"gate weight {tuple(gate_weight.shape)} / bias {tuple(gate_bias.shape)} do not match D={d}")
    if slot_table.numel() != n_experts:
        raise ValueError(f"slot table has {slot_table.numel()} entries for {n_experts} experts")
    if not 1 <= topk <= min(n_experts, 8):
        raise ValueError(f"Invalid topk={topk} for {n_experts} experts")
    if score_fn not in _lib.SCORE_FNS or order not in _lib.ORDERS:
        raise ValueError(f"unknown score_fn / order {score_fn!r} / {order!r}")
    _lib.require_cuda(x, gate_weight, gate_bias, slot_table, addend)
    dev = x.device
    gate_bias = gate_bias.to(torch.float32).contiguous()
    slot_table = slot_table.to(torch.int32).contiguous()
    if addend is not None and (addend.dtype != torch.bfloat16 or addend.shape != x.shape):
        raise ValueError("addend must be a bf16 vector shaped like x")
    idx = torch.empty((topk,), dtype=torch.int32, device=dev)
    w = torch.empty((topk,), dtype=torch.float32, device=dev)
    scores = torch.empty((n_experts,), dtype=torch.float32, device=dev)
    routed = torch.empty((d,), dtype=torch.float32, device=dev) if want_routed else None
    out = torch.empty((d,), dtype=torch.bfloat16, device=dev) if want_out else None
    L = _lib.lib()
    x = x.contiguous()                      # bound to names: a temporary could be freed and its
    gate_weight = gate_weight.contiguous()  # memory reused before the kernels read it
    args_route = (x.data_ptr(), gate_weight.data_ptr(), gate_bias.data_ptr(), n_experts,
                  topk, _lib.SCORE_FNS[score_fn], float(gate_temp), float(route_scale),
                  1 if norm_topk_prob else 0, _lib.ORDERS[order], pool.storage.data_ptr(), pool.layout(),
                  slot_table.data_ptr(), d, f)
    tail = (_lib.ptr(addend), idx.data_ptr(), w.data_ptr(), scores.data_ptr(), _lib.ptr(routed), _lib.ptr(out))
    stream = _lib.stream_handle(dev)
    if shared is not None and fmt.kind == "affine" and not is_q2_g128(fmt):
        # the generic affine kernels carry no shared tiles: the shared expert runs first
        # and enters as the addend (the same out = bf16(routed + y_sh))
        from .shared_expert import shared_expert_forward

        if addend is not None:
            raise ValueError("pass either the shared expert weights or addend, not both")
        addend = shared_expert_forward(x, **shared, swiglu_limit=swiglu_limit)
        tail = (_lib.ptr(addend),) + tail[1:]
        shared = None
    if shared is not None:
        if fmt.kind not in ("affine", "fp4"):
            raise ValueError(f"unknown expert format {fmt.kind!r}")
        if addend is not None:
            raise ValueError("pass either the shared expert weights or addend, not both")
        if not want_out:
            raise ValueError("the shared expert enters through out (want_out=True)")
        from .shared_expert import shared_weights

        sw = shared_weights(shared, d)
        _lib.require_cuda(*sw[:6])
        ptrs = tuple(t.data_ptr() for t in sw[:6])
        if fmt.kind == "affine":
            nbytes = L.cachalot_moe_layer_decode_q2_shared_workspace_bytes(d, f, topk, sw[6])
            ws = workspace(dev, nbytes)
            rc = L.cachalot_moe_layer_decode_q2_shared(*args_route, fmt.group_size, float(swiglu_limit), *ptrs, sw[6],
                                                       *tail[1:], ws.data_ptr(), nbytes, stream)
        else:
            nbytes = L.cachalot_moe_layer_decode_fp4_shared_workspace_bytes(d, f, topk, sw[6])
            ws = workspace(dev, nbytes)
            rc = L.cachalot_moe_layer_decode_fp4_shared(*args_route, float(swiglu_limit), *ptrs, sw[6], *tail[1:],
                                                        ws.data_ptr(), nbytes, stream)
    elif fmt.kind == "affine" and not is_q2_g128(fmt):
        nbytes = L.cachalot_moe_decode_affine_workspace_bytes(d, f, topk)
        ws = workspace(dev, nbytes)
        rc = L.cachalot_moe_layer_decode_affine(*args_route, fmt.bits, fmt.group_size, float(swiglu_limit), *tail,
                                                ws.data_ptr(), nbytes, stream)
    elif fmt.kind == "affine":
        nbytes = L.cachalot_moe_decode_q2_workspace_bytes(d, f, topk)
        ws = workspace(dev, nbytes)
        rc = L.cachalot_moe_layer_decode_q2(*args_route, fmt.group_size, float(swiglu_limit), *tail, ws.data_ptr(),
                                            nbytes, stream)
    elif fmt.kind == "fp4":
        nbytes = L.cachalot_moe_decode_fp4_workspace_bytes(d, f, topk)
        ws = workspace(dev, nbytes)
        rc = L.cachalot_moe_layer_decode_fp4(*args_route, float(swiglu_limit), *tail, ws.data_ptr(), nbytes, stream)
    else:
        raise ValueError(f"unknown expert format {fmt.kind!r}")
    _lib.check(rc, "moe_layer_decode")
    return routed, out, RouterResult(indices=idx, weights=w, scores=scores)


def _experts_table(experts):
    pools = {id(ex.slot.pool) for ex in experts}
    if len(pools) != 1 or experts[0].slot.pool is None:
        raise ValueError("experts must live in one HBM slot pool")
    pool = experts[0].slot.pool
    dev = pool.device
    slots = torch.tensor([ex.slot.index for ex in experts], dtype=torch.int32).to(dev)
    idx = torch.arange(len(experts), dtype=torch.int32).to(dev)
    return pool, slots, idx


def fused_routed_experts(x: torch.Tensor, experts, router_weights: torch.Tensor, *, hidden_size: int = 4096,
                         intermediate: int = 2880, swiglu_limit: float = 10.0) -> torch.Tensor:
    """FP4 experts: fp32 [hidden_size] = sum_e w_e * W2_e(silu(W1_e x) * W3_e x) (clamped)."""
    pool, slots, idx = _experts_table(experts)
    fmt = pool.expert_format()
    if fmt.kind != "fp4":
        raise ValueError("fused_routed_experts needs an FP4 bank")
    if (hidden_size, intermediate) != (fmt.d_model, fmt.d_ff):
        raise ValueError(f"shape {(hidden_size, intermediate)} != bank {(fmt.d_model, fmt.d_ff)}")
    w = router_weights.to(device=pool.device, dtype=torch.float32)
    routed, _ = decode_experts(x.to(torch.bfloat16), pool, slots, idx, w, swiglu_limit=swiglu_limit,
                               want_out=False)
    return routed


def affine_routed_experts(x: torch.Tensor, experts, fmt: ExpertFormat, weights: torch.Tensor,
                          swiglu_limit: float = 10.0) -> torch.Tensor:
    """2-bit experts: fp32 [D] sum over experts in order (bf16 rounding points of the reference)."""
    pool, slots, idx = _experts_table(experts)
    if pool.expert_format().kind != "affine" or fmt.kind != "affine":
        raise ValueError("affine_routed_experts needs an affine bank")
    w = weights.to(device=pool.device, dtype=torch.float32)
    routed, _ = decode_experts(x, pool, slots, idx, w, swiglu_limit=swiglu_limit, want_out=False)
    return routed


def affine_expert_forward(x: torch.Tensor, expert, fmt: ExpertFormat, weight: float,
                          swiglu_limit: float = 10.0) -> torch.Tensor:
    """One affine expert: fp32 [D] = bf16(W2(bf16(silu(min(W1 x, L)) * clip(W3 x) * weight)))."""
    w = torch.tensor([float(weight)], dtype=torch.float32)
    return affine_routed_experts(x, [expert], fmt, w, swiglu_limit)
