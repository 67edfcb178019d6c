"""FP8 (E4M3FN + E8M0) linear and the shared FP8 expert -- CPU restatement.

TEST INFRASTRUCTURE ONLY: imported by tests/ and nothing on the product path.

Reference: ``src/cachalot/model/fp8_ref.py`` (the reference's own CPU oracle):
``quantize_activation_fp8`` (:28-93), ``fp8_gemv_reference`` (:96-231), and the
shared expert ``src/cachalot/model/shared_expert_metal.py:46-125`` /
``:128-188`` (w1 and w3 concatenated, bit-identical by construction).

* E4M3FN: 1 sign, 4 exponent (bias 7), 3 mantissa bits; exponent field 0 is
  subnormal (m / 8 x 2^-6); 0x7F / 0xFF are NaN; the largest finite value is 448.
* act_quant, per 32-element block: ``amax = max(max|x|, 1e-4)``,
  ``scale = 2^ceil(log2(amax / 448))``, ``q = E4M3(clip(x / scale, -448, 448))``
  rounded to nearest, ties to even.  The exponent here is the exact
  ``ceil(log2(fl32(amax / 448)))`` (frexp of the float32 quotient): numpy's
  float32 ``log2`` in ``fp8_ref.py`` can round a quotient a few ulps above a power
  of two down onto it, which would give the next smaller scale; that case is
  stated, not reproduced.
* linear: ``y[n] = sum_kb (sum_{i in kb} q_i w_{n,i}) * act_scale[kb] *
  w_scale[n // 32, kb]`` accumulated exactly (float64), weights E4M3 bytes
  ``[N, K]`` with E8M0 block scales ``[ceil(N / 32), K / 32]``; the result is
  cast to bf16 (``fp8_linear_metal.py:67-107``, ``.astype(mx.bfloat16)``).
* shared expert: ``gate = float(bf16(w1(x)))``, ``up = float(bf16(w3(x)))``,
  ``up = clip(up, -L, L)``, ``gate = min(gate, L)``, ``h = bf16(silu(gate) * up)``,
  ``y = bf16(w2(act_quant(h)))``.
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_bf16

BLOCK = 32
FP8_MAX = 448.0
MIN_AMAX = 1e-4


def e4m3_decode(b) -> np.ndarray:
    """E4M3FN bytes -> float32 (NaN for 0x7F / 0xFF)."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int32)
    s = (b >> 7) & 1
    e = (b >> 3) & 15
    m = b & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    v = np.where(s == 1, -mag, mag)
    v = np.where((b & 0x7F) == 0x7F, np.nan, v)
    return v.astype(np.float32)


_POS = e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)   # codes 0..126, ascending


def e4m3_encode(x) -> np.ndarray:
    """float -> E4M3FN bytes, round to nearest, ties to the even code; |x| <= 448 expected."""
    x = np.asarray(x, dtype=np.float64)
    a = np.minimum(np.abs(x), FP8_MAX)
    hi = np.clip(np.searchsorted(_POS, a, side="left"), 0, 126)       # first code >= a
    lo = np.clip(hi - 1, 0, 126)
    d_hi = np.abs(_POS[hi] - a)
    d_lo = np.abs(a - _POS[lo])
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    return np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)   # -0 and negative underflow keep the sign


def act_quant(x) -> tuple[np.ndarray, np.ndarray]:
    """x [..., K] (float32 values) -> (E4M3 bytes [..., K], scale exponents int [..., K / 32])."""
    x = np.asarray(x, dtype=np.float32)
    k = x.shape[-1]
    if k % BLOCK:
        raise ValueError(f"K={k} must be a multiple of {BLOCK}")
    blocks = x.reshape(*x.shape[:-1], k // BLOCK, BLOCK)
    amax = np.maximum(np.max(np.abs(blocks), axis=-1), np.float32(MIN_AMAX)).astype(np.float32)
    r = (amax / np.float32(FP8_MAX)).astype(np.float32)
    mant, ex = np.frexp(r)                      # r = mant * 2^ex, mant in [0.5, 1)
    e = np.where(mant == 0.5, ex - 1, ex).astype(np.int32)   # exact ceil(log2 r)
    scaled = blocks.astype(np.float64) * np.exp2(-e.astype(np.float64))[..., None]
    q = e4m3_encode(np.clip(scaled, -FP8_MAX, FP8_MAX))
    return q.reshape(x.shape), e


def linear(q, e_act, w_bytes, w_scale_raw) -> np.ndarray:
    """q [M, K] E4M3 bytes, e_act [M, K/32] int, w [N, K] E4M3 bytes, w scales [ceil(N/32), K/32] u8
    -> float64 [M, N] (the exact block-scaled sum; the reference casts it to bf16)."""
    q = np.atleast_2d(q)
    e_act = np.atleast_2d(e_act)
    n, k = w_bytes.shape
    qa = e4m3_decode(q).astype(np.float64)
    wd = e4m3_decode(w_bytes).astype(np.float64)
    ws = np.exp2(np.asarray(w_scale_raw, dtype=np.float64) - 127.0)
    out = np.zeros((qa.shape[0], n))
    for kb in range(k // BLOCK):
        sl = slice(kb * BLOCK, (kb + 1) * BLOCK)
        part = qa[:, sl] @ wd[:, sl].T                                     # [M, N]
        out += part * np.exp2(e_act[:, kb].astype(np.float64))[:, None] * ws[np.arange(n) // BLOCK, kb][None, :]
    return out


def shared_expert(x, w1, s1, w3, s3, w2, s2, limit: float = 10.0) -> np.ndarray:
    """x [M, D] bf16-exact values -> float32 [M, D] (bf16-exact): the shared FP8 expert."""
    x = np.atleast_2d(np.asarray(x, dtype=np.float32))
    q, e = act_quant(x)
    g = round_bf16(linear(q, e, w1, s1).astype(np.float32)).astype(np.float64)
    u = round_bf16(linear(q, e, w3, s3).astype(np.float32)).astype(np.float64)
    if limit > 0:
        u = np.clip(u, -limit, limit)
        g = np.minimum(g, limit)
    with np.errstate(over="ignore"):
        h = round_bf16((g / (1.0 + np.exp(-g)) * u).astype(np.float32))
    qh, eh = act_quant(h)
    return round_bf16(linear(qh, eh, w2, s2).astype(np.float32))
