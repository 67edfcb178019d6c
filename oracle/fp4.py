"""FP4 E2M1 / E8M0 codec, restated from ``src/cachalot/model/fp4.py``.

* ``FP4_E2M1_TABLE``        ``model/fp4.py:5-25``  (code -> value, sign in bit 3)
* ``decode_e8m0``           ``model/fp4.py:28-41`` (2 ** (raw - 127))
* ``unpack_fp4_e2m1``       ``model/fp4.py:44-64`` (low nibble = even index)
* ``dequantize_fp4_weight`` ``model/fp4.py:67-109`` (value * scale per 32-block)

Pinned in ``tests/test_oracle_fp4.py`` against the E2M1 bit-field definition
(OCP MX spec: sign, 2-bit exponent with bias 1, 1-bit mantissa, subnormal at
exponent 0) and hand-worked bytes.
"""
from __future__ import annotations

import numpy as np

FP4_E2M1_TABLE = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
     0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)
# Code 8 (negative zero) is stored as +0.0, as the reference does
# (model/fp4.py:15).  Hardware converters may produce -0.0 for it; the
# parity tests compare values, for which -0.0 == +0.0.


def decode_e8m0(raw) -> np.ndarray:
    """2 ** (raw - 127) exactly.  The reference writes ``np.exp2`` on int16, whose
    float32 loop is off by 2^-23 relative at raw = 254 only; the Metal kernels
    (``exp2(float(int(raw) - 127))``) and this restatement give the exact power."""
    raw = np.asarray(raw, dtype=np.uint8)
    with np.errstate(over="ignore"):
        return np.ldexp(np.float32(1.0), raw.astype(np.int32) - 127).astype(np.float32)


def unpack_fp4_e2m1(packed) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.float32)
    out[..., 0::2] = FP4_E2M1_TABLE[packed & 0x0F]
    out[..., 1::2] = FP4_E2M1_TABLE[(packed >> 4) & 0x0F]
    return out


def dequantize_fp4_weight(packed, scales, block_size: int = 32) -> np.ndarray:
    """packed [N, K/2] u8, scales [N, K/32] u8 -> [N, K] fp32 (exact)."""
    unpacked = unpack_fp4_e2m1(packed)
    n, k = unpacked.shape
    if k % block_size:
        raise ValueError(f"K={k} must be divisible by block_size={block_size}")
    scales = np.asarray(scales)
    if scales.shape != (n, k // block_size):
        raise ValueError(f"Scale shape {scales.shape} does not match expected {(n, k // block_size)}")
    return (unpacked.reshape(n, -1, block_size) * decode_e8m0(scales)[..., None]).reshape(n, k)
