"""Decode MoE layer: router -> top-k routed experts -> combine, one token.

Keeps the call-site signature of ``moe_layer_forward``
(``src/cachalot/model/moe_layer_metal.py:133-153``) and its return value
``(out, RouterResult)`` with ``out`` in the activation dtype.

Difference in mechanism, not in result: the reference evaluates the routing,
reads the ids on the host, asks the store for the experts and launches the
expert kernels (``moe_layer_metal.py:220-300``).  Here the whole bank is
resident in HBM and the store's (layer, expert) -> slot table lives on the
device, so the router's ids go straight into the expert kernels: three
launches (router scores; top-k + slot lookup + gate/up; down + route-order
combine), no host synchronisation.  When a layer is not fully resident the host path is taken:
one synchronisation, ``get_many`` (which loads misses), then the same kernels, with the
store's opt-in approximations (``decode_substitute_tau`` router-share substitution and
``decode_miss_budget`` drop-and-rescale, ``decode_substitution``).  With gates in
``expert_store.decode_gates``, the next layer's experts are predicted from this layer's
input and loaded ahead (``predict_routes``; nothing to do while the bank is resident).

``fused`` is accepted for call-site compatibility and changes nothing: in the
reference it picks between the two-launch FP4 kernel and a per-expert
``fp4_gemv`` loop (``moe_layer_metal.py:165-166,348-376``), which share their
rounding points (fp32 outputs throughout, ``fp4_gemv_metal.py:102-103``), and
it is not consulted for affine banks; this build has the one device path.

The FP8 shared expert (``shared_*``, ``moe_layer_metal.py:381-397``) is added
in the combine: ``out = bf16(routed + shared)``.  On the device path its tiles
run inside the routed gate/up and down launches (one weight stream); otherwise it
runs first, on the same stream, and its bf16 output is the combine's addend.
Both give the same bits.  ``addend`` (bf16 [D]) is the same hook for a
caller that computes the shared branch itself; it cannot be combined with
``shared_*``.
"""
from __future__ import annotations

import os

import torch

from .cache.resident_store import ResidentExpertStore
from .moe_decode import decode_experts, moe_layer_decode
from .router import RouterResult, route_topk, route_topk_fused
from .shared_expert import shared_args, shared_expert_forward
from .storage.index import ExpertEntry

# One-layer-early routing prediction for partial residency (moe_layer_metal.py:17-68):
# layer L+n's router applied to layer L's input names experts that are loaded into
# free slots ahead of their layer.  PREDICT_TOPK experts per predicted layer (0 =
# off); PREDICT_LEAD is the first layer ahead, PREDICT_AHEAD how many layers from
# there; PREDICT_SUBMIT = 0 computes the prediction and discards it.
PREDICT_TOPK = int(os.environ.get("CACHALOT_PREDICT_TOPK", "6"))
PREDICT_AHEAD = int(os.environ.get("CACHALOT_PREDICT_AHEAD", "1"))
PREDICT_LEAD = int(os.environ.get("CACHALOT_PREDICT_LEAD", "1"))
PREDICT_SUBMIT = os.environ.get("CACHALOT_PREDICT_SUBMIT", "1") != "0"


def predict_routes(x: torch.Tensor, layer_id: int, expert_store: ResidentExpertStore, *, gate_temp: float = 1.0,
                   score_fn: str = "sqrt_softplus", order: str = "ascending") -> list[tuple[int, torch.Tensor]]:
    """(layer, predicted ids) for the layers PREDICT_LEAD .. PREDICT_LEAD + PREDICT_AHEAD - 1
    ahead whose gates the store holds (``expert_store.decode_gates``) and that are not
    fully resident (``moe_layer_metal.py:186-202``): that layer's router on this
    layer's input, top PREDICT_TOPK.  The ids stay on the device until the caller's
    one synchronisation."""
    gates = expert_store.decode_gates if PREDICT_TOPK > 0 else None
    out = []
    if not gates or torch.cuda.is_current_stream_capturing():   # submitting one needs the ids on the host
        return out
    for ahead in range(PREDICT_LEAD, PREDICT_LEAD + PREDICT_AHEAD):
        nxt = layer_id + ahead
        if nxt in gates and not expert_store.layer_fully_resident(nxt):
            w_next, b_next = gates[nxt]
            p = route_topk_fused(x, w_next, b_next, topk=PREDICT_TOPK, gate_temp=gate_temp, score_fn=score_fn,
                                 order=order)
            out.append((nxt, p.indices))
    return out


def prediction_entries(predicted, expert_index: dict | None, order: str = "ascending") -> list[ExpertEntry]:
    """Entries of the predicted experts, strongest first within each layer
    (``moe_layer_metal.py:236-244``; ascending order lists the strongest last)."""
    ents = []
    for nxt, p_idx in predicted:
        ids = [int(e) for e in p_idx.tolist()]
        if order == "ascending":
            ids = ids[::-1]
        for e in ids:
            entry = expert_index.get((nxt, e)) if expert_index is not None else ExpertEntry(nxt, e)
            if entry is not None:
                ents.append(entry)
    return ents


def moe_layer_forward(
    x: torch.Tensor,
    *,
    layer_id: int,
    gate_weight: torch.Tensor,
    gate_bias: torch.Tensor,
    expert_index: dict | None,
    expert_store: ResidentExpertStore,
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
    fused: bool | None = None,
    score_fn: str = "sqrt_softplus",
    order: str = "ascending",
    addend: torch.Tensor | None = None,
) -> tuple[torch.Tensor, RouterResult]:
    if x.ndim != 1:
        raise ValueError(f"x must be 1D for decode, got {tuple(x.shape)}")
    shared = shared_args(shared_w1, shared_w1_scales, shared_w2, shared_w2_scales, shared_w3, shared_w3_scales)
    if shared is not None and addend is not None:
        raise ValueError("pass either the shared expert weights or addend, not both")
    pool = expert_store.pool
    device_path = expert_store.layer_fully_resident(layer_id) and x.dtype == torch.bfloat16 and topk <= 8
    if shared is not None and not device_path:
        addend = shared_expert_forward(x.to(torch.bfloat16), **shared, swiglu_limit=swiglu_limit)
        shared = None
    if device_path:
        # routing, slot lookup and experts on the device, no host round trip (the
        # decode launches also carry the shared expert)
        _, out, route = moe_layer_decode(x, gate_weight, gate_bias, pool, expert_store.layer_table(layer_id),
                                         topk=topk, gate_temp=gate_temp, route_scale=route_scale,
                                         norm_topk_prob=norm_topk_prob, score_fn=score_fn, order=order,
                                         swiglu_limit=swiglu_limit, addend=addend, shared=shared)
        # a later layer that is not fully resident: its predicted experts load after
        # this layer's launches (one synchronisation, only then); the store's walk
        # advances here too, so the predictions' deadlines count from this layer
        expert_store.note_decode_layer(layer_id)
        predicted = predict_routes(x, layer_id, expert_store, gate_temp=gate_temp, score_fn=score_fn, order=order)
        if predicted and PREDICT_SUBMIT:
            expert_store.prefetch_decode(prediction_entries(predicted, expert_index, order))
        return out, route
    router = route_topk_fused if norm_topk_prob else route_topk
    route = router(x, gate_weight, gate_bias, topk=topk, gate_temp=gate_temp, route_scale=route_scale,
                   norm_topk_prob=norm_topk_prob, score_fn=score_fn, order=order)
    idx, weights = route.indices, route.weights
    if not expert_store.layer_fully_resident(layer_id):
        predicted = predict_routes(x, layer_id, expert_store, gate_temp=gate_temp, score_fn=score_fn, order=order)
        # host-addressed path: one sync for the ids, then load what is missing
        # (moe_layer_metal.py:220-310), with the store's opt-in approximations
        ids = [int(e) for e in route.indices.tolist()]
        wts = route.weights.tolist()
        tau = getattr(expert_store, "decode_substitute_tau", None)
        if tau is not None:
            from .decode_substitution import plan_substitution, ranked_candidates

            selection = route.scores.float().cpu().numpy() + gate_bias.float().cpu().numpy()
            ids, replaced = plan_substitution(
                ids, wts, ranked_candidates(selection, ids, getattr(expert_store, "decode_substitute_ranks", 4)),
                lambda e: expert_store.is_cached((layer_id, e)), tau)
            expert_store.substituted_experts += replaced
        entries = []
        for e in ids:
            key = (layer_id, e)
            entry = expert_index.get(key) if expert_index is not None else ExpertEntry(*key)
            if entry is None:
                raise KeyError(f"Missing routed expert layer={layer_id}, expert={e}")
            entries.append(entry)
        budget = getattr(expert_store, "decode_miss_budget", None)
        prefetch = prediction_entries(predicted, expert_index, order) if PREDICT_SUBMIT else None
        got = expert_store.get_many(entries, max_misses=budget, priorities=wts, prefetch=prefetch or None)
        if budget is not None and any(g is None for g in got):
            # dropped experts; the kept weights carry the layer's routing mass
            from .decode_substitution import rescale_kept

            kept = [i for i, g in enumerate(got) if g is not None]
            wts = rescale_kept(wts, kept)
            ids = [ids[i] for i in kept]
        if not ids:
            out = torch.zeros_like(x, dtype=torch.float32)
            if addend is not None:
                out = out + addend.float()
            return out.to(x.dtype), route
        idx = torch.tensor(ids, dtype=torch.int32, device=x.device)
        weights = torch.tensor(wts, dtype=torch.float32, device=x.device)
    table = expert_store.layer_table(layer_id)
    _, out = decode_experts(x, pool, table, idx, weights, swiglu_limit=swiglu_limit, addend=addend,
                            want_routed=False, want_out=True)
    return out.to(x.dtype), route
