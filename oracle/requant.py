"""FP4 expert -> affine requantization (the bank tool's fits) -- CPU restatement.

TEST INFRASTRUCTURE ONLY: imported by tests/ and nothing on the product path.

Reference: ``benchmarks/quant_affine.py`` -- ``_quantize`` (:113-116),
``_error`` (:119-123), ``fit_minmax`` (:138-149), ``SHRINKS`` (:155),
``fit_search`` (:158-186), ``quantize_affine`` (:303-329); the source weights are
the FP4 checkpoint dequantized to fp32 (``benchmarks/expert_requant_error.py:68-84``,
``build_affine_bank.py:165-189``).  All arithmetic is float32, as in MLX:

* per 128-element group: ``lo = min``, ``hi = max``, ``mid = (lo + hi) / 2``;
* min/max fit: ``scale = max((hi - lo) / 3, 1e-8)``, ``bias = lo``;
* candidate (s_lo, s_hi) over SHRINKS x SHRINKS except (1, 1), in that order:
  ``new_lo = mid + (lo - mid) * s_lo``, ``new_hi = mid + (hi - mid) * s_hi``,
  ``scale = max((new_hi - new_lo) / 3, 1e-8)``, ``bias = new_lo``; taken when its
  error is strictly below the best so far;
* error: ``sum((scale * q + bias - w)^2)`` with ``q = clip(round_half_even((w - bias) / scale), 0, 3)``;
* output: scale and bias rounded to bf16 (the reference bank's type,
  ``build_affine_bank.py:76``), or RNE to fp16 for an fp16 bank; codes
  recomputed against the rounded pair (code 0 where an fp16 scale rounds to
  zero: only a constant group, whose min/max scale is 1e-8, does), packed 16
  per uint32, low field first.

The other fits of the bank tool (``build_affine_bank.py:74-75``, ``FITS``):
``minmax``; ``search-lsq`` (the search, then 4 least-squares refinements,
``_lsq_step``/``refine_lsq``/``fit_search_lsq`` at ``quant_affine.py:207-245,255-261``);
``wide-lsq`` (the search over ``SHRINKS_WIDE``, then the refinement, ``:281-287``);
every fit optionally weighted per column by activation importance (``group_weights``,
``:126-135``; the weights enter ``_error`` and the normal equations).  Widths:
2, 3 or 4 bits (levels 2^bits - 1), groups of 32, 64 or 128.  A refinement step
rounds its scale and bias to the bank's storage type (bf16, as the reference;
fp16 for an fp16 bank), keeps the previous pair where the normal equations are
singular (|den| < 1e-12) or the new scale is not positive, and the best iterate
(strictly smaller error) is kept.  It also keeps the previous pair where the new
one is not finite (a zero importance total, or a scale beyond fp16's range): the
reference carries such a pair on, but neither its error nor that of any iterate
after it is finite, so none of them is ever taken as the best, and the fit
returned is the same.  The normal-equation sums run in index order.
``mlx`` (mx.quantize's own fit) lives in the third-party MLX and is not restated.

Two things the reference leaves open are fixed here and stated:
* the error sum runs over the group's elements in index order (MLX's reduction
  order is inside the framework; only near-ties between candidates depend on
  it), and the GPU kernel sums in the same order, so the two agree bit for bit;
* K not a whole number of groups (w2 at d_ff = 2880): the last group's fit runs
  over its real elements only and its padding codes are 0 (the reference bank
  tool only ever ran K = 2304, a whole number of groups).
"""
from __future__ import annotations

import numpy as np

from .affine2 import pack_bits
from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits

LEVELS = 3
SHRINKS = (1.0, 0.925, 0.85, 0.775, 0.7)
SHRINKS_WIDE = (1.0, 0.925, 0.85, 0.775, 0.7, 0.625, 0.55, 0.475, 0.4)
LSQ_ITERS = 4
FITS = ("minmax", "search", "search-lsq", "wide-lsq")
F32 = np.float32


def _q(w, scale, bias, levels=LEVELS):
    return np.clip(np.round((w - bias) / scale), F32(0), F32(levels)).astype(F32)


def group_error(w, valid, scale, bias, levels=LEVELS, weights=None):
    """Sequential float32 sum over the group's elements of a (scale*q + bias - w)^2; w [G, n]."""
    d = scale * _q(w, scale, bias, levels) + bias - w
    sq = (d * d).astype(F32)
    if weights is not None:
        sq = (weights * sq).astype(F32)
    err = np.zeros(w.shape[0], F32)
    for i in range(w.shape[1]):
        err = np.where(valid[:, i], (err + sq[:, i]).astype(F32), err)
    return err


def fit_minmax(w, valid, levels=LEVELS):
    big = F32(np.finfo(np.float32).max)
    lo = np.where(valid, w, big).min(axis=1, keepdims=True).astype(F32)
    hi = np.where(valid, w, -big).max(axis=1, keepdims=True).astype(F32)
    return np.maximum(((hi - lo) / F32(levels)).astype(F32), F32(1e-8)), lo, hi


def fit_search(w, valid, shrinks=SHRINKS, levels=LEVELS, weights=None):
    """(scale, bias) float32 [G, 1] of the searched fit for groups w [G, n] (valid masks real elements)."""
    best_s, lo, hi = fit_minmax(w, valid, levels)
    mid = ((lo + hi) / F32(2)).astype(F32)
    tiny = F32(1e-8)
    best_b = lo
    best = group_error(w, valid, best_s, best_b, levels, weights)
    for s_lo in shrinks:
        for s_hi in shrinks:
            if s_lo == 1.0 and s_hi == 1.0:
                continue
            new_lo = (mid + ((lo - mid) * F32(s_lo)).astype(F32)).astype(F32)
            new_hi = (mid + ((hi - mid) * F32(s_hi)).astype(F32)).astype(F32)
            s = np.maximum(((new_hi - new_lo) / F32(levels)).astype(F32), tiny)
            err = group_error(w, valid, s, new_lo, levels, weights)
            take = (err < best)[:, None]
            best_s = np.where(take, s, best_s)
            best_b = np.where(take, new_lo, best_b)
            best = np.minimum(err, best)
    return best_s, best_b


def _store(v, scale_dtype):
    """Round to the bank's storage type and back to float32."""
    if scale_dtype == "bfloat16":
        return bf16_bits_to_f32(f32_to_bf16_bits(v))
    return np.asarray(v, F32).astype(np.float16).astype(F32)


def _seq_sum(v, valid):
    acc = np.zeros(v.shape[0], F32)
    for i in range(v.shape[1]):
        acc = np.where(valid[:, i], (acc + v[:, i]).astype(F32), acc)
    return acc[:, None]


def lsq_step(w, valid, scale, bias, levels=LEVELS, weights=None, scale_dtype="bfloat16"):
    """quant_affine.py:207-228: assign levels, then the (weighted) least-squares line through (q, w)."""
    q = _q(w, scale, bias, levels)
    a = np.ones_like(w) if weights is None else weights.astype(F32)
    n = _seq_sum(a, valid)
    sq = _seq_sum((a * q).astype(F32), valid)
    sqq = _seq_sum(((a * q).astype(F32) * q).astype(F32), valid)
    sw = _seq_sum((a * w).astype(F32), valid)
    sqw = _seq_sum(((a * q).astype(F32) * w).astype(F32), valid)
    den = ((n * sqq).astype(F32) - (sq * sq).astype(F32)).astype(F32)
    sing = np.abs(den) < F32(1e-12)
    with np.errstate(divide="ignore", invalid="ignore"):
        ns = (((n * sqw).astype(F32) - (sq * sw).astype(F32)).astype(F32) / np.where(sing, F32(1), den)).astype(F32)
        nb = ((sw - (ns * sq).astype(F32)).astype(F32) / n).astype(F32)
    ns, nb = _store(ns, scale_dtype), _store(nb, scale_dtype)
    keep = sing | (ns <= 0) | ~np.isfinite(ns) | ~np.isfinite(nb)
    return np.where(keep, scale, ns), np.where(keep, bias, nb)


def refine_lsq(w, valid, scale, bias, iters=LSQ_ITERS, levels=LEVELS, weights=None, scale_dtype="bfloat16"):
    """quant_affine.py:231-245: alternate assignment and refit, keeping the best iterate per group."""
    scale, bias = _store(scale, scale_dtype), _store(bias, scale_dtype)
    best_s, best_b = scale, bias
    best = group_error(w, valid, best_s, best_b, levels, weights)
    for _ in range(iters):
        scale, bias = lsq_step(w, valid, scale, bias, levels, weights, scale_dtype)
        err = group_error(w, valid, scale, bias, levels, weights)
        take = (err < best)[:, None]
        best_s = np.where(take, scale, best_s)
        best_b = np.where(take, bias, best_b)
        best = np.minimum(err, best)
    return best_s, best_b


def fit(w, valid, name="search", levels=LEVELS, weights=None, scale_dtype="bfloat16"):
    if name == "minmax":
        s, lo, _ = fit_minmax(w, valid, levels)
        return s, lo
    if name == "search":
        return fit_search(w, valid, SHRINKS, levels, weights)
    if name == "search-lsq":
        s, b = fit_search(w, valid, SHRINKS, levels, weights)
        return refine_lsq(w, valid, s, b, LSQ_ITERS, levels, weights, scale_dtype)
    if name == "wide-lsq":
        s, b = fit_search(w, valid, SHRINKS_WIDE, levels, weights)
        return refine_lsq(w, valid, s, b, LSQ_ITERS, levels, weights, scale_dtype)
    raise ValueError(f"unknown fit {name!r} (one of {FITS})")


def requantize(dense: np.ndarray, group: int = 128, scale_dtype: str = "bfloat16", *, bits: int = 2,
               fit_name: str = "search", importance: np.ndarray | None = None):
    """dense float32 [N, K] -> (packed uint32 [N, Kp * bits / 32], scale bits [N, Kp/g], bias bits), the
    bits bf16 or fp16 (``scale_dtype``); ``importance`` [K] weights the fit per column."""
    n, k = dense.shape
    levels = (1 << bits) - 1
    groups = -(-k // group)
    kp = groups * group
    w = np.zeros((n, kp), F32)
    w[:, :k] = dense
    valid = np.zeros((n, kp), bool)
    valid[:, :k] = True
    g = w.reshape(-1, group)
    v = valid.reshape(-1, group)
    wts = None
    if importance is not None:
        imp = np.zeros(kp, F32)
        imp[:k] = np.asarray(importance, F32)
        wts = np.tile(imp.reshape(-1, group), (n, 1))
    s, b = fit(g, v, fit_name, levels, wts, scale_dtype)
    if scale_dtype == "bfloat16":
        sb, bb = f32_to_bf16_bits(s), f32_to_bf16_bits(b)
        s16, b16 = bf16_bits_to_f32(sb), bf16_bits_to_f32(bb)
    elif scale_dtype == "float16":
        sb, bb = s.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
        s16, b16 = sb.view(np.float16).astype(F32), bb.view(np.float16).astype(F32)
    else:
        raise ValueError(f"scale dtype {scale_dtype!r}")
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(v & (s16 != 0), _q(g, s16, b16, levels), F32(0)).astype(np.uint8)
    return pack_bits(q.reshape(n, kp), bits), sb.reshape(n, groups), bb.reshape(n, groups)
