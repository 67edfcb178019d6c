"""Partial-residency approximations for decode (opt-in; exact inference leaves them off).

With the whole bank resident in HBM no routed expert is ever missing and
neither rule runs.  They matter when the store holds part of the bank
(``ResidentExpertStore`` with fewer slots than experts) and a miss costs a
host-side load.  Both follow ``src/cachalot/model/moe_layer_metal.py:247-310``:

* substitution (``decode_substitution.py:1-52``): a non-resident routed expert
  whose share of the layer's router weight is below ``tau`` takes no load; the
  best resident expert among the next ``ranks`` by selection score (router
  score + correction bias) takes its place and its weight.  Weakest routed
  experts are replaced first, each by the best unused candidate.  Total routing
  mass is unchanged.
* miss budget (``moe_layer_metal.py:286-310``, ``resident_store.py:851-857``):
  ``get_many`` loads at most ``max_misses`` missing experts, strongest router
  weight first; the others are dropped and the kept weights rescaled by
  ``total / kept_sum`` so the layer keeps its routing mass.
"""
from __future__ import annotations

from collections.abc import Callable, Sequence

import numpy as np


def ranked_candidates(selection_scores, expert_ids: Sequence[int], ranks: int) -> list[int]:
    """The ``ranks`` best experts by selection score outside ``expert_ids``, best first (ties: lower id)."""
    taken = {int(e) for e in expert_ids}
    sel = np.asarray(selection_scores, dtype=np.float64).reshape(-1)
    order = np.argsort(-sel, kind="stable")
    out: list[int] = []
    for e in order[: len(taken) + max(0, int(ranks))]:
        if int(e) not in taken:
            out.append(int(e))
    return out[: max(0, int(ranks))]


def plan_substitution(expert_ids: Sequence[int], weights: Sequence[float], candidates: Sequence[int],
                      is_resident: Callable[[int], bool], tau: float) -> tuple[list[int], int]:
    """Routed ids with weak non-resident experts replaced by resident candidates.

    Positions are kept, so ``weights`` stay aligned.  Returns (ids, replaced)."""
    ids = [int(e) for e in expert_ids]
    total = float(sum(float(w) for w in weights))
    if total <= 0.0:
        return ids, 0
    routed = set(ids)
    spare = [int(c) for c in candidates if int(c) not in routed and is_resident(int(c))]
    replaced = 0
    for pos in sorted(range(len(ids)), key=lambda j: float(weights[j])):   # weakest first
        if replaced >= len(spare):
            break
        if float(weights[pos]) >= tau * total or is_resident(ids[pos]):
            continue
        ids[pos] = spare[replaced]
        replaced += 1
    return ids, replaced


def rescale_kept(weights: Sequence[float], kept: Sequence[int]) -> list[float]:
    """Weights of the kept positions scaled by total / kept_sum (float64, as the reference's Python floats)."""
    w = [float(v) for v in weights]
    total = sum(w)
    kept_sum = sum(w[i] for i in kept) or 1.0
    return [w[i] * total / kept_sum for i in kept]
