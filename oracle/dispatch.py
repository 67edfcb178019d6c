"""Expert-major dispatch and slot-ordered combine, restated.

* permute: ``src/cachalot/model/moe_prefill_grouped.py:199-225`` builds
  ``assignments[expert] = [(token, route_slot, weight), ...]`` by walking tokens
  in order, so within one expert the rows are in ascending token order.  The
  reference walks experts in first-appearance order; the order of experts does
  not change any sum because every (token, slot) pair receives exactly one
  contribution (``:346-348``).  This build lays experts out in ascending id.
* combine: ``slot_buffer[token, slot] = y`` (``:464-467``), then
  ``slot 0 + slot 1 + ... + slot k-1`` in fp32 (``:526-531``), then
  ``+ shared`` and the cast to the activation dtype (``:543-545``).
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_bf16


def permute(idx, n_experts: int):
    """idx [T, k] -> dict(offsets [E+1], token [T*k], slot [T*k], pos [T, k]).

    Ids outside [0, E) are dropped routes (the reference raises ``KeyError`` for a
    missing expert, ``moe_layer_metal.py:279-283``; this build gives them zero
    rows): they follow every expert's rows, in route order."""
    idx = np.asarray(idx, dtype=np.int64)
    t, k = idx.shape
    flat = idx.reshape(-1)
    flat = np.where((flat >= 0) & (flat < n_experts), flat, n_experts)
    order = np.argsort(flat, kind="stable")           # (token, slot) row-major -> stable by expert
    counts = np.bincount(flat, minlength=n_experts + 1)[:n_experts]
    offsets = np.zeros(n_experts + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    pos = np.empty(t * k, dtype=np.int64)
    pos[order] = np.arange(t * k)
    return {
        "offsets": offsets.astype(np.int32),
        "token": (order // k).astype(np.int32),
        "slot": (order % k).astype(np.int32),
        "pos": pos.reshape(t, k).astype(np.int32),
    }


def combine(y_rows, pos, addend=None):
    """y_rows [T*k, D] fp32, pos [T, k] -> (routed fp32 [T, D], out fp32 holding bf16 values)."""
    y_rows = np.asarray(y_rows, dtype=np.float32)
    pos = np.asarray(pos)
    routed = np.float32(0.0) + y_rows[pos[:, 0]]      # slot_buffer starts at zeros (:244-247)
    for s in range(1, pos.shape[1]):
        routed = routed + y_rows[pos[:, s]]
    total = routed if addend is None else routed + np.asarray(addend, np.float32)
    return routed, round_bf16(total)
