"""MLX affine layouts (2-bit g128 and the other widths) and the group formula, restated.

* packing: 16 codes per uint32, least-significant field first
  (``benchmarks/quant_affine.py:11-16,60-66``; layout pinned by the reference's
  own ``tests/test_quant_affine.py:45-51`` against ``mx.quantize``); at 3 and 4
  bits (``pack_bits``, ``quant_affine.py:69-105``) a row's codes are one
  little-endian bit stream, code i at bits [i b, (i+1) b), a code straddling a
  word boundary split between the two words;
* dequantised value ``w = scale * q + bias`` per ``group``-element group along K
  (``benchmarks/quant_affine.py:11-15``), scales/biases stored bf16
  (``benchmarks/build_affine_bank.py:76,165-174``) or fp16 (the oQ3e banks,
  ``src/cachalot/model/expert_affine.py:1-10``; ``ExpertFormat.dtypes`` carries
  which, ``storage/index.py:18,153``);
* ``quantized_matmul(x, w, s, b, transpose=True)``: per group
  ``s * sum(x_i q_i) + b * sum(x_i)`` with fp32 accumulation
  (MLX ``qdot``, shown at ``src/cachalot/minimax/codes_qmv.py:86-100``).

K that is not a whole number of groups (d_ff = 2880 at g128) is stored padded
to ``ceil(K/g)*g`` with zero codes; padded activation lanes are 0, so the last
group's ``sum(x_i)`` runs over the real K only.

``qmv`` here accumulates in float64 (the accuracy reference); MLX's own fp32
summation order lives inside a third-party kernel and is not restated, so the
GPU path is checked to a tolerance, not bit for bit.
"""
from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32

PER_WORD = 16


def pack_2bit(q) -> np.ndarray:
    """[..., K] codes 0..3 -> [..., K/16] uint32, low field first."""
    q = np.asarray(q)
    if q.shape[-1] % PER_WORD:
        raise ValueError(f"K={q.shape[-1]} is not a multiple of {PER_WORD}")
    f = q.astype(np.uint64).reshape(*q.shape[:-1], -1, PER_WORD)
    shifts = (np.arange(PER_WORD, dtype=np.uint64) * np.uint64(2))
    return np.bitwise_or.reduce(f << shifts, axis=-1).astype(np.uint32)


def unpack_2bit(w, k: int | None = None) -> np.ndarray:
    """[..., W] uint32 -> [..., k] uint8 codes (k defaults to 16 * W)."""
    w = np.asarray(w, dtype=np.uint32)
    shifts = (np.arange(PER_WORD, dtype=np.uint32) * np.uint32(2))
    q = ((w[..., None] >> shifts) & np.uint32(3)).astype(np.uint8)
    q = q.reshape(*w.shape[:-1], -1)
    return q if k is None else q[..., :k]


def scale_values(bits, dtype: str = "bfloat16") -> np.ndarray:
    """Stored scale / bias bits -> exact fp32 values (bf16: the high half of an
    fp32; fp16: IEEE half precision, subnormals included)."""
    bits = np.asarray(bits, dtype=np.uint16)
    if dtype == "bfloat16":
        return bf16_bits_to_f32(bits)
    if dtype == "float16":
        return bits.view(np.float16).astype(np.float32)
    raise ValueError(f"scale dtype {dtype!r}")


def pack_bits(q, bits: int) -> np.ndarray:
    """[..., K] codes in 0 .. 2^bits - 1 -> [..., K * bits / 32] uint32: the row as one
    little-endian bit stream (numpy's little-endian bit packing of the code bits,
    each code least significant bit first)."""
    q = np.asarray(q, dtype=np.uint32)
    if (q.shape[-1] * bits) % 32:
        raise ValueError(f"K={q.shape[-1]} at {bits} bits is not a whole number of words")
    if bits == 2:
        return pack_2bit(q)
    bitplane = ((q[..., None] >> np.arange(bits, dtype=np.uint32)) & 1).astype(np.uint8)
    stream = bitplane.reshape(*q.shape[:-1], -1)                       # bit i*bits + j = bit j of code i
    by = np.packbits(stream, axis=-1, bitorder="little")               # byte m = stream bits 8m .. 8m+7
    return np.ascontiguousarray(by).view("<u4").astype(np.uint32)


def unpack_bits(w, bits: int, k: int | None = None) -> np.ndarray:
    """Inverse of ``pack_bits``: [..., W] uint32 -> [..., k] uint8 codes (k defaults to 32 W / bits)."""
    if bits == 2:
        return unpack_2bit(w, k)
    w = np.ascontiguousarray(np.asarray(w, dtype="<u4"))
    stream = np.unpackbits(w.view(np.uint8), axis=-1, bitorder="little")
    n = stream.shape[-1] // bits
    codes = stream[..., : n * bits].reshape(*w.shape[:-1], n, bits).astype(np.uint32)
    q = (codes << np.arange(bits, dtype=np.uint32)).sum(axis=-1).astype(np.uint8)
    return q if k is None else q[..., :k]


def dequantize_affine(w, scales_bits, biases_bits, *, k: int, group: int = 128,
                      scale_dtype: str = "bfloat16", bits: int = 2) -> np.ndarray:
    """[N, K] fp32 with the declared rounding ``fl(fl(s * q) + b)`` (s, b exact from their storage type)."""
    q = unpack_bits(w, bits, k).astype(np.float32)
    s = np.repeat(scale_values(scales_bits, scale_dtype), group, axis=-1)[..., :k]
    b = np.repeat(scale_values(biases_bits, scale_dtype), group, axis=-1)[..., :k]
    return (s * q) + b


def dequantize_affine64(w, scales_bits, biases_bits, *, k: int, group: int = 128,
                        scale_dtype: str = "bfloat16", bits: int = 2) -> np.ndarray:
    q = unpack_bits(w, bits, k).astype(np.float64)
    s = np.repeat(scale_values(scales_bits, scale_dtype).astype(np.float64), group, axis=-1)[..., :k]
    b = np.repeat(scale_values(biases_bits, scale_dtype).astype(np.float64), group, axis=-1)[..., :k]
    return s * q + b


def qmv64(x, w, scales_bits, biases_bits, *, k: int, group: int = 128, scale_dtype: str = "bfloat16",
          bits: int = 2) -> np.ndarray:
    """x [M, K] (bf16-exact values) -> float64 [M, N] = sum_g s_g*sum(x q) + b_g*sum(x).

    s*q+b is exact in float64 for bf16 or fp16 s, b and q below 2^bits, so this
    equals x @ dequant(W)^T evaluated in float64."""
    x = np.asarray(x, dtype=np.float64)
    return x @ dequantize_affine64(w, scales_bits, biases_bits, k=k, group=group, scale_dtype=scale_dtype,
                                   bits=bits).T
