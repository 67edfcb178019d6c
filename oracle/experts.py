"""Routed-expert SwiGLU math at the reference's rounding points (float64 inside).

Each function evaluates the matrix products in float64 (the accuracy
reference) and applies the reference's casts exactly where it applies them:

* ``fp4_decode`` -- ``src/cachalot/model/moe_fused_metal.py:189-233``:
  x read as fp32, gate/up accumulated in fp32 (no bf16 rounding),
  ``h = silu(min(g, L)) * clip(u, -L, L) * w_e`` in fp32
  (``moe_fused_metal.py:127-135``), ``out = sum_e W2_e h_e`` in fp32, experts in
  route order (``:160-178``).  Output fp32.
* ``affine_decode`` -- ``src/cachalot/model/expert_affine.py:65-81,117-152``:
  ``g = bf16(qmm(x_bf16, W1))``, ``u = bf16(qmm(x, W3))`` read back as fp32; clamp;
  ``h = bf16(silu(g) * u * w_e)``; ``y_e = bf16(qmm(h, W2))`` as fp32;
  ``routed = 0 + y_0 + ... + y_{k-1}`` in fp32; the MoE layer returns
  ``bf16(routed + shared)`` (``moe_layer_metal.py:128,394-397``).
* ``swiglu_rows`` -- batched form: ``affine_expert_forward_batched``
  (``expert_affine.py:84-99``) and the FP4 prefill kernels
  (``fp4_sgmm_metal.py:205-226,318-333``): the same bf16 rounding points as
  the affine decode, per row, with a per-row router weight.

``silu(g) = g * sigmoid(g)`` (MLX ``nn.silu``) and ``g / (1 + exp(-g))`` (the
Metal kernels) are the same function; float64 is used for both.
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_bf16


def _silu64(g: np.ndarray) -> np.ndarray:
    return g / (1.0 + np.exp(-g))


def _clamp(g, u, limit):
    if limit > 0:
        u = np.clip(u, -limit, limit)
        g = np.minimum(g, limit)
    return g, u


def fp4_decode(x, dense_experts, weights, limit: float = 10.0) -> np.ndarray:
    """x [D]; dense_experts: list of (W1 [F,D], W3 [F,D], W2 [D,F]) exact fp32 -> fp32 [D]."""
    x = np.asarray(x, dtype=np.float64)
    out = np.zeros(dense_experts[0][2].shape[0], dtype=np.float64)
    for (w1, w3, w2), w in zip(dense_experts, weights, strict=True):
        g = w1.astype(np.float64) @ x
        u = w3.astype(np.float64) @ x
        g, u = _clamp(g, u, limit)
        h = _silu64(g) * u * float(np.float32(w))
        out += w2.astype(np.float64) @ h
    return out.astype(np.float32)


def swiglu_rows(x, mm1, mm3, mm2, weights, limit: float = 10.0, *, raw: bool = False):
    """Rows with the bf16 rounding points.

    x [M, K] bf16-exact values; mm1/mm3/mm2 map a float64 [M, K] array to its
    float64 product with W1^T / W3^T / W2^T; weights [M] fp32.  -> fp32 [M, D]
    (each value bf16-exact).  With ``raw`` also the float64 value of the last
    product before its casts (fp32, then bf16), which tells how close each
    output lies to a bf16 rounding boundary."""
    x = np.asarray(x, dtype=np.float64)
    g = round_bf16(mm1(x).astype(np.float32)).astype(np.float64)
    u = round_bf16(mm3(x).astype(np.float32)).astype(np.float64)
    g, u = _clamp(g, u, limit)
    w = np.asarray(weights, dtype=np.float32).astype(np.float64)[:, None]
    h = round_bf16((_silu64(g) * u * w).astype(np.float32)).astype(np.float64)
    y64 = mm2(h)
    y = round_bf16(y64.astype(np.float32))
    return (y, y64) if raw else y


def affine_decode(x, mats, weights, limit: float = 10.0, addend=None, *, terms: bool = False,
                  raw: bool = False):
    """x [D] bf16-exact; mats: per expert (mm1, mm3, mm2) as in ``swiglu_rows``.

    -> (routed fp32 [D], out fp32 [D] holding bf16(routed + addend)), plus the
    per-expert outputs y_e (bf16-exact fp32 [k, D]) when ``terms``, plus their
    float64 values before the casts (``swiglu_rows(raw=True)``) when ``raw``."""
    x = np.asarray(x, dtype=np.float64)[None, :]
    routed = None
    ys, raws = [], []
    for (mm1, mm3, mm2), w in zip(mats, weights, strict=True):
        y, y64 = swiglu_rows(x, mm1, mm3, mm2, np.asarray([w], np.float32), limit, raw=True)
        ys.append(y[0])
        raws.append(y64[0])
        routed = (np.float32(0.0) + y[0]) if routed is None else (routed + y[0])
    routed = routed.astype(np.float32)
    total = routed if addend is None else routed + np.asarray(addend, np.float32)
    res = (routed, round_bf16(total))
    if terms:
        res += (np.stack(ys),)
    if raw:
        res += (np.stack(raws),)
    return res
