"""Router restatement: logits, score function, top-k, weight normalisation.

Reference semantics (``src/cachalot/model/router_mlx.py:29-37``)::

    scores  = score_fn(linear(x.float(), weight.float()) / gate_temp)
    indices = topk(scores + bias)          # bias affects selection only
    weights = scores[indices]
    weights /= sum(weights) + 1e-20        # when norm_topk_prob and topk > 1
    weights *= route_scale

* ``score_fn``: ``sqrt(softplus(.))`` (DeepSeek, ``router_mlx.py:189-191``,
  stable softplus form ``router_fused_metal.py:47-49``) or ``sigmoid``
  (MiniMax/GLM, ``minimax/language.py:280-283``).
* order ``ORDER_ASCENDING``: stable ``argsort(sel)[-k:]`` -- ascending, on a tie
  the larger index wins (``router_mlx.py:197-202``, ``router_fused_metal.py:78-91``).
  ``ORDER_RANK``: ``argpartition(-sel)`` in rank order, on a tie the lower index
  wins (``minimax/gpu_select.py:81-84,101-106``).
* weight sum in output order, then ``w / (sum + 1e-20) * route_scale``
  (``router_fused_metal.py:95-100``).

The reference leaves the fp32 summation order of the logit dot product to MLX.
This build fixes one so ids are reproducible bit for bit on any device:

* D is split into 64 contiguous chunks (one per lane of a wave64); each chunk
  is summed sequentially in fp32 from 0 (bf16 x bf16 products are exact in fp32
  unless |x w| < 2^-126: there a separate multiply rounds the product and the
  GPU's fma does not, so such inputs may differ in the last bit -- far outside
  any real activation and gate weight);
* the 64 partials are combined by the butterfly ``p[i] + p[i ^ s]`` for
  s = 1, 2, 4, 8, 16, 32 (pairwise summation over the chunks in natural order);
* ``logit = tree / gate_temp`` in fp32.

Score functions are evaluated with IEEE basic operations only, so that the
GPU and NumPy agree exactly:

* ``exp64(a)`` for a <= 0: Cody-Waite reduction with fdlibm's ln2_hi/ln2_lo,
  degree-13 Taylor polynomial in Horner form, ``ldexp``; 0 below -200;
* ``log1p64(t)`` for t in [0, 1]: ``2 atanh(t / (2 + t))`` as an odd series
  (17 terms, |u| <= 1/3);
* sigmoid: ``t = fp32(exp64(-|z|))``; ``1 / (1 + t)`` or ``t / (1 + t)`` in fp32;
* sqrt-softplus: ``sqrt_fp32(fp32(max(z, 0) + log1p64(exp64(-|z|))))``.

Both are within an fp32 ulp of the reference's fp32 evaluation.
"""
from __future__ import annotations

import math

import numpy as np

SCORE_SQRT_SOFTPLUS = 0
SCORE_SIGMOID = 1
ORDER_ASCENDING = 0
ORDER_RANK = 1
N_CHUNKS = 64

INV_LN2 = 1.4426950408889634
LN2_HI = 6.93147180369123816490e-01
LN2_LO = 1.90821492927058770002e-10
EXP_COEF = [1.0 / math.factorial(k) for k in range(14)]
LOG1P_COEF = [2.0 / (2 * j + 1) for j in range(17)]


def exp64(a: np.ndarray) -> np.ndarray:
    a = np.asarray(a, dtype=np.float64)
    n = np.rint(a * INV_LN2)
    r = (a - n * LN2_HI) - n * LN2_LO
    p = np.full_like(r, EXP_COEF[13])
    for c in EXP_COEF[12::-1]:
        p = p * r + c
    out = np.ldexp(p, n.astype(np.int32))
    return np.where(a < -200.0, 0.0, out)


def log1p64(t: np.ndarray) -> np.ndarray:
    t = np.asarray(t, dtype=np.float64)
    u = t / (2.0 + t)
    u2 = u * u
    q = np.full_like(u, LOG1P_COEF[16])
    for c in LOG1P_COEF[15::-1]:
        q = q * u2 + c
    return u * q


def score_fn(z32: np.ndarray, kind: int) -> np.ndarray:
    z32 = np.asarray(z32, dtype=np.float32)
    z = z32.astype(np.float64)
    t = exp64(-np.abs(z))
    if kind == SCORE_SIGMOID:
        t32 = t.astype(np.float32)
        one = np.float32(1.0)
        return np.where(z32 >= 0, one / (one + t32), t32 / (one + t32)).astype(np.float32)
    if kind == SCORE_SQRT_SOFTPLUS:
        sp = np.maximum(z, 0.0) + log1p64(t)
        return np.sqrt(sp.astype(np.float32))
    raise ValueError(f"unknown score function {kind}")


def logits(x32: np.ndarray, w32: np.ndarray, gate_temp: float = 1.0, *, block: int = 16,
           workers: int = 1) -> np.ndarray:
    """x [T, D], w [E, D] (bf16-exact fp32 values) -> fp32 [T, E] in the fixed order.

    ``workers`` > 1 evaluates blocks of tokens on that many threads (NumPy
    releases the GIL inside the element-wise loops); every token's arithmetic is
    the same either way."""
    x32 = np.asarray(x32, dtype=np.float32)
    w32 = np.asarray(w32, dtype=np.float32)
    t, d = x32.shape
    e = w32.shape[0]
    if d % N_CHUNKS:
        raise ValueError(f"D={d} must be a multiple of {N_CHUNKS}")
    ch = d // N_CHUNKS
    out = np.empty((t, e), dtype=np.float32)
    xr = x32.reshape(t, N_CHUNKS, ch)
    wr = w32.reshape(e, N_CHUNKS, ch)
    lane = np.arange(N_CHUNKS)

    def one(t0):
        xs = xr[t0:t0 + block]
        acc = np.zeros((xs.shape[0], e, N_CHUNKS), dtype=np.float32)
        for j in range(ch):
            acc += xs[:, None, :, j] * wr[None, :, :, j]
        for s in (1, 2, 4, 8, 16, 32):
            acc = acc + acc[..., lane ^ s]
        out[t0:t0 + block] = acc[..., 0]

    starts = range(0, t, block)
    if workers > 1 and t > block:
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(max_workers=workers) as ex:
            list(ex.map(one, starts))
    else:
        for t0 in starts:
            one(t0)
    return out / np.float32(gate_temp)


def topk_select(sel: np.ndarray, k: int, order: int) -> np.ndarray:
    """sel [T, E] fp32 -> int32 [T, k]."""
    sel = np.asarray(sel, dtype=np.float32)
    if order == ORDER_ASCENDING:
        return np.argsort(sel, axis=-1, kind="stable")[:, -k:].astype(np.int32)
    if order == ORDER_RANK:
        return np.argsort(-sel, axis=-1, kind="stable")[:, :k].astype(np.int32)
    raise ValueError(f"unknown order {order}")


def normalise(w: np.ndarray, route_scale: float, norm: bool) -> np.ndarray:
    w = np.asarray(w, dtype=np.float32)
    scale = np.float32(route_scale)
    if norm and w.shape[-1] > 1:
        total = np.zeros(w.shape[:-1], dtype=np.float32)
        for j in range(w.shape[-1]):
            total = total + w[..., j]
        denom = total + np.float32(1e-20)
        return (w / denom[..., None]) * scale
    return w * scale


def route(x32, w32, bias, *, topk: int = 6, gate_temp: float = 1.0, route_scale: float = 1.5,
          norm_topk_prob: bool = True, score: int = SCORE_SQRT_SOFTPLUS, order: int = ORDER_ASCENDING,
          bias_vl=None, image_mask=None, workers: int = 1):
    """-> (indices int32 [T,k], weights fp32 [T,k], scores fp32 [T,E])."""
    x32 = np.atleast_2d(np.asarray(x32, dtype=np.float32))
    scores = score_fn(logits(x32, w32, gate_temp, workers=workers), score)
    b = np.asarray(bias, dtype=np.float32)[None, :]
    if image_mask is not None:
        b = np.where(np.asarray(image_mask, bool)[:, None], np.asarray(bias_vl, np.float32)[None, :], b)
    sel = scores + b
    idx = topk_select(sel, topk, order)
    w = np.take_along_axis(scores, idx, axis=-1)
    return idx, normalise(w, route_scale, norm_topk_prob), scores
