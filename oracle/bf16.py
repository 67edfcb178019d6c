"""bf16 <-> fp32 helpers (round to nearest even), as MLX's ``astype(mx.bfloat16)``.

The rounding rule is the IEEE one; the bit form used here is the standard
``(u + 0x7FFF + ((u >> 16) & 1)) >> 16`` on the fp32 bit pattern, which the
reference itself writes out at ``src/cachalot/minimax/codes_qmv.py:98``.
NaNs keep a quiet NaN pattern.
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(a) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(a) -> np.ndarray:
    """fp32 values rounded to the nearest bf16 (returned as fp32)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))
