"""Expert-major MoE for many tokens: prefill chunks and batched decode.

Keeps the call-site signature of ``moe_prefill_grouped``
(``src/cachalot/model/moe_prefill_grouped.py:74-103``) and its return value
``(output [T, D] in x.dtype, RouterResult)``.

Mechanism: route all tokens on the device, permute the T*k routes into rows
grouped by expert (tokens ascending inside an expert, the order the
reference's assignment loop produces, ``:199-225``), run every expert's SwiGLU
over its rows as two grouped matrix-core launches (``y = bf16(W2 bf16(silu(
bf16 g) * bf16 u * w))`` per row, the rounding points of
``affine_expert_forward_batched`` / ``routed_expert_forward_sgmm``), and sum the
route slots in decode order (``:526-545``).  The host reads nothing back when
the layer is fully resident in HBM; otherwise one synchronisation fetches the
routed expert ids so that ``get_many`` can load the misses first.

The FP8 shared expert (``shared_*``, ``:532-545``) runs over all rows and its
bf16 output is added in the combine: ``out = bf16(routed + shared)``.
``addend`` ([T, D] bf16) is the same hook for a caller that computes the
shared branch itself; it cannot be combined with ``shared_*``.
"""
from __future__ import annotations

import torch

from . import _lib
from .cache.resident_store import ResidentExpertStore
from .cache.slots import HBMSlotPool
from .router import RouterResult, route_topk_batch, route_topk_rows
from .shared_expert import shared_args, shared_expert_forward_batched
from .storage.index import ExpertEntry

_WORKSPACES: dict[int, torch.Tensor] = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Scratch for grouped calls, cached per device (grown on demand); calls sharing it must be ordered."""
    ws = _WORKSPACES.get(device.index)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        _WORKSPACES[device.index] = ws
    return ws


def permute(indices: torch.Tensor, weights: torch.Tensor, n_experts: int):
    """Routes [T, k] -> (offsets [E+1], row_token, row_slot, row_w) grouped by expert (device tensors)."""
    if indices.ndim != 2 or tuple(weights.shape) != tuple(indices.shape):
        raise ValueError(f"indices {tuple(indices.shape)} / weights {tuple(weights.shape)} must be [T, k]")
    _lib.require_cuda(indices, weights)
    t, k = indices.shape
    dev = indices.device
    indices = indices.to(torch.int32).contiguous()
    weights = weights.to(torch.float32).contiguous()
    offsets = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    row_token = torch.empty(t * k, dtype=torch.int32, device=dev)
    row_slot = torch.empty(t * k, dtype=torch.int32, device=dev)
    row_w = torch.empty(t * k, dtype=torch.float32, device=dev)
    rc = _lib.lib().cachalot_permute(indices.data_ptr(), weights.data_ptr(), t, k, n_experts, offsets.data_ptr(),
                                     row_token.data_ptr(), row_slot.data_ptr(), row_w.data_ptr(),
                                     _lib.stream_handle(dev))
    _lib.check(rc, "permute")
    return offsets, row_token, row_slot, row_w


def grouped_experts(x: torch.Tensor, indices: torch.Tensor, weights: torch.Tensor, pool: HBMSlotPool,
                    slot_table: torch.Tensor, *, swiglu_limit: float = 10.0, addend: torch.Tensor | None = None,
                    want_routed: bool = False, want_out: bool = True, want_terms: bool = False,
                    addend_ready: torch.cuda.Event | None = None):
    """x [T, D] bf16, routes [T, k] -> (routed fp32 [T, D] or None, out bf16 [T, D] or None).

    routed[t] = sum over route slots s (in order) of expert idx[t, s] applied to x[t]
    with router weight w[t, s]; out = bf16(routed + addend).  A route whose expert
    id lies outside [0, E), or whose expert has no slot, contributes zero.  With
    ``want_terms`` the per-route expert outputs y [T, k, D] bf16 (each one the
    reference's bf16 cast of its expert's output) come back as a third value.
    ``addend_ready``, when given, is an event recorded after the work that
    writes ``addend`` on another stream: the combine waits for it, the grouped
    GEMMs before it do not."""
    fmt = pool.expert_format()
    d, f = fmt.d_model, fmt.d_ff
    if x.ndim != 2 or x.shape[1] != d:
        raise ValueError(f"x must be [tokens, {d}], got {tuple(x.shape)}")
    if x.shape[0] == 0:
        raise ValueError("x must contain at least one token")
    if x.dtype != torch.bfloat16:
        raise TypeError("grouped experts expect bf16 activations")
    if indices.shape[0] != x.shape[0]:
        raise ValueError(f"{indices.shape[0]} routes for {x.shape[0]} tokens")
    if addend is not None and (addend.dtype != torch.bfloat16 or tuple(addend.shape) != tuple(x.shape)):
        raise ValueError("addend must be bf16 shaped like x")
    _lib.require_cuda(x, slot_table, addend)
    t, k = indices.shape
    n_experts = slot_table.numel()
    dev = x.device
    x = x.contiguous()
    slot_table = slot_table.to(torch.int32).contiguous()
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    y = torch.empty((t, k, d), dtype=torch.bfloat16, device=dev)
    generic = fmt.kind == "affine" and not (fmt.bits == 2 and fmt.group_size == 128)
    if generic:
        nbytes = L.cachalot_grouped_experts_affine_workspace_bytes(t, k, n_experts, d, f)
    else:
        nbytes = L.cachalot_grouped_experts_workspace_bytes(t, k, n_experts, d, f)
    ws = _workspace(dev, nbytes)
    if generic:
        # 3- / 4-bit codes or groups of 32 / 64: the generic affine kernels (csrc/affine.hip)
        offsets, row_token, row_slot, row_w = permute(indices, weights, n_experts)
        rc = L.cachalot_grouped_experts_affine(x.data_ptr(), pool.storage.data_ptr(), pool.layout(),
                                               slot_table.data_ptr(), offsets.data_ptr(), row_token.data_ptr(),
                                               row_slot.data_ptr(), row_w.data_ptr(), t, d, f, n_experts, k, fmt.bits,
                                               fmt.group_size, float(swiglu_limit), y.data_ptr(), ws.data_ptr(),
                                               nbytes, stream)
    elif fmt.kind == "affine":
        # the routes go in as they are: a batched decode permutes them inside its prep launch
        if indices.ndim != 2 or tuple(weights.shape) != tuple(indices.shape):
            raise ValueError(f"indices {tuple(indices.shape)} / weights {tuple(weights.shape)} must be [T, k]")
        _lib.require_cuda(indices, weights)
        ids = indices.to(torch.int32).contiguous()
        wts = weights.to(torch.float32).contiguous()
        offsets = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
        row_token = torch.empty(t * k, dtype=torch.int32, device=dev)
        row_slot = torch.empty(t * k, dtype=torch.int32, device=dev)
        row_w = torch.empty(t * k, dtype=torch.float32, device=dev)
        rc = L.cachalot_grouped_experts_q2_routes(x.data_ptr(), pool.storage.data_ptr(), pool.layout(),
                                                  slot_table.data_ptr(), ids.data_ptr(), wts.data_ptr(),
                                                  offsets.data_ptr(), row_token.data_ptr(), row_slot.data_ptr(),
                                                  row_w.data_ptr(), t, d, f, n_experts, k, fmt.group_size,
                                                  float(swiglu_limit), y.data_ptr(), ws.data_ptr(), nbytes, stream)
    elif fmt.kind == "fp4":
        offsets, row_token, row_slot, row_w = permute(indices, weights, n_experts)
        common = (x.data_ptr(), pool.storage.data_ptr(), pool.layout(), slot_table.data_ptr(), offsets.data_ptr(),
                  row_token.data_ptr(), row_slot.data_ptr(), row_w.data_ptr(), t, d, f, n_experts, k)
        rc = L.cachalot_grouped_experts_fp4(*common, float(swiglu_limit), y.data_ptr(), ws.data_ptr(), nbytes, stream)
    else:
        raise ValueError(f"unknown expert format {fmt.kind!r}")
    _lib.check(rc, "grouped_experts")
    routed = torch.empty((t, d), dtype=torch.float32, device=dev) if want_routed else None
    out = torch.empty((t, d), dtype=torch.bfloat16, device=dev) if want_out else None
    if addend_ready is not None:
        torch.cuda.current_stream(dev).wait_event(addend_ready)
    rc = L.cachalot_unpermute_combine(y.data_ptr(), _lib.ptr(addend), t, k, d, _lib.ptr(routed), _lib.ptr(out), stream)
    _lib.check(rc, "unpermute_combine")
    return (routed, out, y) if want_terms else (routed, out)


_SIDE_STREAMS: dict[int, torch.cuda.Stream] = {}
# From this many tokens on the shared expert's GEMMs run beside the router and
# the routed grouped GEMMs; below it the launches are too short to gain.
SIDE_STREAM_MIN_TOKENS = 256


def _shared_on_side_stream(x: torch.Tensor, shared: dict, swiglu_limit: float):
    """Shared expert of x -> (bf16 [T, D], event or None).

    Many-token calls outside graph capture run it on a second stream (default
    priority) forked from the current one; the returned event marks its end."""
    xb = x.to(torch.bfloat16)
    if x.shape[0] < SIDE_STREAM_MIN_TOKENS or torch.cuda.is_current_stream_capturing():
        return shared_expert_forward_batched(xb, **shared, swiglu_limit=swiglu_limit), None
    dev = x.device
    main = torch.cuda.current_stream(dev)
    side = _SIDE_STREAMS.get(dev.index)
    if side is None:
        side = torch.cuda.Stream(device=dev)
        _SIDE_STREAMS[dev.index] = side
    side.wait_stream(main)
    with torch.cuda.stream(side):
        addend = shared_expert_forward_batched(xb, **shared, swiglu_limit=swiglu_limit)
        done = torch.cuda.Event()
        done.record(side)
    # tensors made or read on the side stream stay allocated until it is done
    xb.record_stream(side)
    addend.record_stream(main)
    for v in shared.values():
        if isinstance(v, torch.Tensor):
            v.record_stream(side)
    return addend, done


def moe_prefill_grouped(
    x: torch.Tensor,
    *,
    layer_id: int,
    gate_weight: torch.Tensor,
    gate_bias: torch.Tensor,
    expert_index: dict | None,
    expert_store: ResidentExpertStore,
    expert_prefetcher=None,
    shared_w1=None,
    shared_w1_scales=None,
    shared_w2=None,
    shared_w2_scales=None,
    shared_w3=None,
    shared_w3_scales=None,
    topk: int = 6,
    gate_temp: float = 1.0,
    route_scale: float = 1.5,
    norm_topk_prob: bool = True,
    swiglu_limit: float = 10.0,
    batched: bool = True,
    gate_bias_vl: torch.Tensor | None = None,
    image_mask: torch.Tensor | None = None,
    score_fn: str = "sqrt_softplus",
    order: str = "ascending",
    addend: torch.Tensor | None = None,
) -> tuple[torch.Tensor, RouterResult]:
    if x.ndim != 2:
        raise ValueError(f"x must be 2D [tokens, hidden], got {tuple(x.shape)}")
    if x.shape[0] == 0:
        raise ValueError("x must contain at least one token")
    if image_mask is not None and not batched:
        raise NotImplementedError(
            "per-token bias_vl selection is only wired for the batched (route_topk_rows) path; "
            "batched=False has no image_mask support")
    shared = shared_args(shared_w1, shared_w1_scales, shared_w2, shared_w2_scales, shared_w3, shared_w3_scales)
    if shared is not None:
        if addend is not None:
            raise ValueError("pass either the shared expert weights or addend, not both")
        addend, addend_ready = _shared_on_side_stream(x, shared, swiglu_limit)
    else:
        addend_ready = None
    if batched:
        indices, weights, scores = route_topk_rows(x, gate_weight, gate_bias, topk=topk, gate_temp=gate_temp,
                                                   route_scale=route_scale, norm_topk_prob=norm_topk_prob,
                                                   bias_vl=gate_bias_vl, image_mask=image_mask, score_fn=score_fn,
                                                   order=order)
        route = RouterResult(indices=indices, weights=weights, scores=scores)
    else:
        route = route_topk_batch(x, gate_weight, gate_bias, topk=topk, gate_temp=gate_temp,
                                 route_scale=route_scale, norm_topk_prob=norm_topk_prob, score_fn=score_fn,
                                 order=order)
    bypass = False
    if not expert_store.layer_fully_resident(layer_id):
        # host-addressed (moe_prefill_grouped.py:297-309): one sync for the routed
        # ids; with a prefetcher the layer's resident set is planned first; then
        # every touched expert gets a slot at once (residents as they are, misses
        # admitted or in transient slots), since one grouped launch reads them all
        ids = sorted({int(e) for e in route.indices.reshape(-1).tolist()})
        entries = []
        for e in ids:
            key = (layer_id, e)
            entry = expert_index.get(key) if expert_index is not None else ExpertEntry(*key)
            if entry is None:
                raise KeyError(f"Missing routed expert layer={layer_id}, expert={e}")
            entries.append(entry)
        if expert_prefetcher is not None:
            expert_store.prepare_prefill_layer(layer_id, entries, num_layers=expert_store.n_layers)
        got = expert_store.get_many_prefill(entries)
        table = expert_store.prefill_slot_table(layer_id, got)
        bypass = True
    else:
        table = expert_store.layer_table(layer_id)
    _, out = grouped_experts(x.to(torch.bfloat16), route.indices, route.weights, expert_store.pool, table,
                             swiglu_limit=swiglu_limit, addend=addend, addend_ready=addend_ready)
    if bypass:
        # the launches are enqueued; a transient slot's next load queues behind them
        expert_store.release_prefill_layer(layer_id)
    return out.to(x.dtype), route
