"""Router entry points on the GPU (one kernel pair for every variant).

Same contracts as the reference:

* ``route_topk``        -- ``src/cachalot/model/router_mlx.py:16-118`` (1-D x)
* ``route_topk_fused``  -- ``router_fused_metal.py:111-148`` (norm_topk_prob must be True)
* ``route_topk_batch``  -- ``router_mlx.py:121-211`` (per-token, stacked)
* ``route_topk_rows``   -- ``moe_prefill_batched.py:128-178`` (rows, optional bias_vl/image_mask)

``score_fn`` ("sqrt_softplus" = DeepSeek, "sigmoid" = MiniMax/GLM) and ``order``
("ascending" = ``argsort(sel)[-k:]``, tie to the larger index; "rank" =
``argpartition(-sel)``, tie to the lower index) are explicit keywords; the
defaults are the reference's DeepSeek call sites.  Every variant runs the same
fixed-order fp32 logit reduction, so batched and single-token routing agree bit
for bit (the property ``tests/test_route_topk_bias_vl.py:106-113`` checks in the
reference).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib


@dataclass(frozen=True)
class RouterResult:
    indices: torch.Tensor
    weights: torch.Tensor
    scores: torch.Tensor


def _launch(x2: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, *, topk: int, gate_temp: float,
            route_scale: float, norm_topk_prob: bool, score_fn: str, order: str, bias_vl=None, image_mask=None):
    if weight.ndim != 2:
        raise ValueError(f"weight must be 2D, got {tuple(weight.shape)}")
    n_experts, hidden = weight.shape
    if x2.shape[-1] != hidden:
        raise ValueError(f"x has {x2.shape[-1]} elements, gate expects {hidden}")
    if tuple(bias.shape) != (n_experts,):
        raise ValueError(f"bias shape {tuple(bias.shape)} != ({n_experts},)")
    if not 1 <= topk <= n_experts:
        raise ValueError(f"Invalid topk={topk} for {n_experts} experts")
    if (bias_vl is None) != (image_mask is None):
        raise ValueError("bias_vl and image_mask must be supplied together, or neither")
    if score_fn not in _lib.SCORE_FNS:
        raise ValueError(f"unknown score_fn {score_fn!r}")
    if order not in _lib.ORDERS:
        raise ValueError(f"unknown order {order!r}")
    if x2.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("router expects bf16 activations and a bf16 gate weight")
    _lib.require_cuda(x2, weight, bias)
    t = x2.shape[0]
    dev = x2.device
    x2 = x2.contiguous()
    weight = weight.contiguous()
    bias = bias.to(torch.float32).contiguous()
    if image_mask is not None:
        if tuple(image_mask.shape) != (t,):
            raise ValueError(f"image_mask must be [{t}], got {tuple(image_mask.shape)}")
        image_mask = image_mask.to(device=dev, dtype=torch.uint8).contiguous()
        bias_vl = bias_vl.to(device=dev, dtype=torch.float32).contiguous()
    idx = torch.empty((t, topk), dtype=torch.int32, device=dev)
    w = torch.empty((t, topk), dtype=torch.float32, device=dev)
    scores = torch.empty((t, n_experts), dtype=torch.float32, device=dev)
    rc = _lib.lib().cachalot_router_topk(
        x2.data_ptr(), weight.data_ptr(), bias.data_ptr(), _lib.ptr(bias_vl), _lib.ptr(image_mask),
        t, hidden, n_experts, topk, _lib.SCORE_FNS[score_fn], float(gate_temp), float(route_scale),
        1 if norm_topk_prob else 0, _lib.ORDERS[order], idx.data_ptr(), w.data_ptr(), scores.data_ptr(),
        _lib.stream_handle(dev))
    _lib.check(rc, "router")
    return idx, w, scores


def route_topk(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, *, topk: int = 6, gate_temp: float = 1.0,
               route_scale: float = 1.5, norm_topk_prob: bool = True, score_fn: str = "sqrt_softplus",
               order: str = "ascending") -> RouterResult:
    if x.ndim != 1:
        raise ValueError(f"x must be 1D, got {tuple(x.shape)}")
    idx, w, scores = _launch(x[None], weight, bias, topk=topk, gate_temp=gate_temp, route_scale=route_scale,
                             norm_topk_prob=norm_topk_prob, score_fn=score_fn, order=order)
    return RouterResult(indices=idx[0], weights=w[0], scores=scores[0])


def route_topk_fused(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, *, topk: int = 6,
                     gate_temp: float = 1.0, route_scale: float = 1.5, norm_topk_prob: bool = True,
                     score_fn: str = "sqrt_softplus", order: str = "ascending") -> RouterResult:
    if not norm_topk_prob:
        raise ValueError("route_topk_fused implements norm_topk_prob=True only")
    if x.ndim != 1 or x.shape[0] != weight.shape[-1]:
        raise ValueError(f"x must be 1-D with {weight.shape[-1]} elements, got {tuple(x.shape)}")
    return route_topk(x, weight, bias, topk=topk, gate_temp=gate_temp, route_scale=route_scale,
                      norm_topk_prob=True, score_fn=score_fn, order=order)


def route_topk_batch(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, *, topk: int = 6,
                     gate_temp: float = 1.0, route_scale: float = 1.5, norm_topk_prob: bool = True,
                     score_fn: str = "sqrt_softplus", order: str = "ascending") -> RouterResult:
    if x.ndim != 2:
        raise ValueError(f"x must be 2D [tokens, hidden], got {tuple(x.shape)}")
    if x.shape[0] == 0:
        raise ValueError("x must contain at least one token")
    idx, w, scores = _launch(x, weight, bias, topk=topk, gate_temp=gate_temp, route_scale=route_scale,
                             norm_topk_prob=norm_topk_prob, score_fn=score_fn, order=order)
    return RouterResult(indices=idx, weights=w, scores=scores)


def route_topk_rows(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, *, topk: int = 6,
                    gate_temp: float = 1.0, route_scale: float = 1.5, norm_topk_prob: bool = True,
                    bias_vl: torch.Tensor | None = None, image_mask: torch.Tensor | None = None,
                    score_fn: str = "sqrt_softplus", order: str = "ascending"):
    """-> (indices [T, k] int32, weights [T, k] fp32, scores [T, E] fp32)."""
    if (bias_vl is None) != (image_mask is None):
        raise ValueError("bias_vl and image_mask must be supplied together, or neither")
    if x.ndim != 2:
        raise ValueError(f"x must be 2D [tokens, hidden], got {tuple(x.shape)}")
    if x.shape[0] == 0:
        raise ValueError("x must contain at least one token")
    return _launch(x, weight, bias, topk=topk, gate_temp=gate_temp, route_scale=route_scale,
                   norm_topk_prob=norm_topk_prob, score_fn=score_fn, order=order, bias_vl=bias_vl,
                   image_mask=image_mask)
