"""FP4 expert -> 2-bit affine g128 requantization (the searched fit) -- CPU restatement.

TEST INFRASTRUCTURE ONLY: imported by tests/ and nothing on the product path.

Reference: ``benchmarks/quant_affine.py`` -- ``_quantize`` (:130-133),
``_error`` (:136-140), ``fit_minmax`` (:157-167), ``SHRINKS`` (:174),
``fit_search`` (:177-205), ``quantize_affine`` (:330-359); the source weights are
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

from .affine2 import pack_2bit
from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits

LEVELS = 3
SHRINKS = (1.0, 0.925, 0.85, 0.775, 0.7)
F32 = np.float32


def _q(w, scale, bias):
    return np.clip(np.round((w - bias) / scale), F32(0), F32(LEVELS)).astype(F32)


def group_error(w, valid, scale, bias):
    """Sequential float32 sum over the group's elements of (scale*q + bias - w)^2; w [G, 128]."""
    d = scale * _q(w, scale, bias) + bias - w
    sq = (d * d).astype(F32)
    err = np.zeros(w.shape[0], F32)
    for i in range(w.shape[1]):
        err = np.where(valid[:, i], (err + sq[:, i]).astype(F32), err)
    return err


def fit_search(w, valid):
    """(scale, bias) float32 [G, 1] of the searched fit for groups w [G, 128] (valid masks real elements)."""
    big = F32(np.finfo(np.float32).max)
    lo = np.where(valid, w, big).min(axis=1, keepdims=True).astype(F32)
    hi = np.where(valid, w, -big).max(axis=1, keepdims=True).astype(F32)
    mid = ((lo + hi) / F32(2)).astype(F32)
    tiny = F32(1e-8)
    best_s = np.maximum(((hi - lo) / F32(LEVELS)).astype(F32), tiny)
    best_b = lo
    best = group_error(w, valid, best_s, best_b)
    for s_lo in SHRINKS:
        for s_hi in SHRINKS:
            if s_lo == 1.0 and s_hi == 1.0:
                continue
            new_lo = (mid + ((lo - mid) * F32(s_lo)).astype(F32)).astype(F32)
            new_hi = (mid + ((hi - mid) * F32(s_hi)).astype(F32)).astype(F32)
            s = np.maximum(((new_hi - new_lo) / F32(LEVELS)).astype(F32), tiny)
            err = group_error(w, valid, s, new_lo)
            take = (err < best)[:, None]
            best_s = np.where(take, s, best_s)
            best_b = np.where(take, new_lo, best_b)
            best = np.minimum(err, best)
    return best_s, best_b


def requantize(dense: np.ndarray, group: int = 128, scale_dtype: str = "bfloat16"):
    """dense float32 [N, K] -> (packed uint32 [N, Kp/16], scale bits [N, Kp/g], bias bits), the bits
    bf16 or fp16 (``scale_dtype``)."""
    n, k = dense.shape
    groups = -(-k // group)
    kp = groups * group
    w = np.zeros((n, kp), F32)
    w[:, :k] = dense
    valid = np.zeros((n, kp), bool)
    valid[:, :k] = True
    g = w.reshape(-1, group)
    v = valid.reshape(-1, group)
    s, b = fit_search(g, v)
    if scale_dtype == "bfloat16":
        sb, bb = f32_to_bf16_bits(s), f32_to_bf16_bits(b)
        s16, b16 = bf16_bits_to_f32(sb), bf16_bits_to_f32(bb)
    elif scale_dtype == "float16":
        sb, bb = s.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
        s16, b16 = sb.view(np.float16).astype(F32), bb.view(np.float16).astype(F32)
    else:
        raise ValueError(f"scale dtype {scale_dtype!r}")
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(v & (s16 != 0), _q(g, s16, b16), F32(0)).astype(np.uint8)
    return pack_2bit(q.reshape(n, kp)), sb.reshape(n, groups), bb.reshape(n, groups)
