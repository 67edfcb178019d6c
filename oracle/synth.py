"""NumPy twin of the seeded synthetic-bank generator (test infrastructure).

The GPU fill kernel in ``cachalot_amd/csrc/synth.hip`` writes expert banks of
up to ~150 GB directly in HBM; the parity tests regenerate any expert they
need here, bit for bit, from the same definition:

* counter-based stream: ``rand(key, i) = fmix64(key + (i + 1) * GAMMA)`` with
  SplitMix64's finaliser (Steele, Lea & Flood, OOPSLA 2014);
* ``stream_key(seed, layer, expert, tensor)`` chains the finaliser over the
  four identifiers;
* kinds: raw uint32 words (optionally zero past ``row_valid`` words of each
  ``row_total``-word row), E8M0 bytes uniform in ``[lo, hi]``, bf16 uniform
  ``a + w * t`` with ``t = (r >> 40) * 2^-24``, bf16 / fp32 "normal" as the
  Irwin-Hall sum of the four 16-bit fields of ``r`` scaled to the requested
  standard deviation (bounded at 3.46 sigma; it is a synthetic-data choice).

All float steps are single IEEE operations in float64 followed by one
round to fp32 (and RNE to bf16), so both sides agree exactly.

The configs describe the data the reference's own benchmarks would use
(``BASELINE.json`` configs); the reference has no generator of its own to
restate, so this module cites none.
"""
from __future__ import annotations

import math

import numpy as np

from .bf16 import f32_to_bf16_bits

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

KIND_U32 = 0
KIND_E8M0 = 1
KIND_BF16_UNIFORM = 2
KIND_BF16_NORMAL = 3
KIND_F32_NORMAL = 4
KIND_F16_UNIFORM = 5
KIND_F16_NORMAL = 6

IRWIN_HALL_STD = math.sqrt((65536.0 ** 2 - 1.0) / 3.0)

TENSOR_IDS = {
    "w1.weight": 0, "w1.scale": 1, "w1.scales": 1, "w1.biases": 2,
    "w2.weight": 3, "w2.scale": 4, "w2.scales": 4, "w2.biases": 5,
    "w3.weight": 6, "w3.scale": 7, "w3.scales": 7, "w3.biases": 8,
}
# pseudo expert ids for the small per-layer / per-step tensors
ROUTER_W = 1 << 20
ROUTER_BIAS = (1 << 20) + 1
ACTIVATION = (1 << 20) + 2


def fmix64(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.asarray(z, dtype=np.uint64)
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def stream_key(seed: int, layer: int, expert: int, tensor: int) -> int:
    with np.errstate(over="ignore"):
        k = fmix64(np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + GAMMA)
        k = fmix64(k ^ (np.uint64(layer) * GAMMA))
        k = fmix64(k ^ np.uint64(expert))
        k = fmix64(k + np.uint64(tensor) * M2)
    return int(k)


def rand(key: int, start: int, n: int) -> np.ndarray:
    i = np.arange(start, start + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return fmix64(np.uint64(key) + (i + np.uint64(1)) * GAMMA)


def _normal_f64(r: np.ndarray, sigma: float) -> np.ndarray:
    s = np.zeros(r.shape, dtype=np.float64)
    for j in range(4):
        s += ((r >> np.uint64(16 * j)) & np.uint64(0xFFFF)).astype(np.float64)
    c = sigma / IRWIN_HALL_STD
    return (s - 131070.0) * c


def fill(kind: int, n: int, key: int, p0: float = 0.0, p1: float = 0.0,
         row_total: int = 0, row_valid: int = 0, start: int = 0) -> np.ndarray:
    """Elements [start, start+n) of one synthetic tensor; dtype follows the kind
    (uint32 words, uint8 E8M0, uint16 bf16 bits, float32)."""
    r = rand(key, start, n)
    if kind == KIND_U32:
        out = (r & np.uint64(0xFFFFFFFF)).astype(np.uint32)
        if row_total > 0:
            col = np.arange(start, start + n, dtype=np.int64) % row_total
            out[col >= row_valid] = 0
        return out
    if kind == KIND_E8M0:
        lo, hi = int(p0), int(p1)
        return (lo + ((r >> np.uint64(32)) % np.uint64(hi - lo + 1)).astype(np.int64)).astype(np.uint8)
    if kind == KIND_BF16_UNIFORM:
        t = (r >> np.uint64(40)).astype(np.float64) * (2.0 ** -24)
        v = p0 + p1 * t
        return f32_to_bf16_bits(v.astype(np.float32))
    if kind == KIND_BF16_NORMAL:
        return f32_to_bf16_bits(_normal_f64(r, p0).astype(np.float32))
    if kind == KIND_F32_NORMAL:
        return _normal_f64(r, p0).astype(np.float32)
    if kind == KIND_F16_UNIFORM:     # fp64 -> fp32 -> fp16 (RNE), as the GPU fill
        t = (r >> np.uint64(40)).astype(np.float64) * (2.0 ** -24)
        return (p0 + p1 * t).astype(np.float32).astype(np.float16).view(np.uint16)
    if kind == KIND_F16_NORMAL:
        return _normal_f64(r, p0).astype(np.float32).astype(np.float16).view(np.uint16)
    raise ValueError(f"unknown kind {kind}")


# ----------------------------------------------------------------------------
# Bank specs: (name, shape, dtype, kind, p0, p1, row_total, row_valid) per tensor
# ----------------------------------------------------------------------------

def fp4_tensor_specs(d_model: int, d_ff: int, e8m0_lo: int = 119, e8m0_hi: int = 127):
    """FP4 E2M1 expert (model/fp4.py layout): packed [N, K/2] u8, E8M0 [N, K/32] u8."""
    specs = []
    for proj, (n, k) in (("w1", (d_ff, d_model)), ("w2", (d_model, d_ff)), ("w3", (d_ff, d_model))):
        specs.append((f"{proj}.weight", (n, k // 2), np.uint8, KIND_U32, 0.0, 0.0, 0, 0))
        specs.append((f"{proj}.scale", (n, k // 32), np.uint8, KIND_E8M0, float(e8m0_lo), float(e8m0_hi), 0, 0))
    return specs


def q2_tensor_specs(d_model: int, d_ff: int, group: int = 128,
                    scale_lo: float = 0.005, scale_hi: float = 0.05, bias_sigma: float = 0.02,
                    scale_dtype: str = "bfloat16", bits: int = 2):
    """Affine expert (MLX layout): weight [N, Kp * bits / 32] u32 (uniform random words: every
    code uniform), scales/biases [N, Kp/g] bf16 (or fp16 with ``scale_dtype="float16"``,
    BASELINE config 1's "fp16 scale and bias").

    Kp is K rounded up to a whole group; codes past K are zero (K * bits is a whole
    number of words for every shape used)."""
    specs = []
    for proj, (n, k) in (("w1", (d_ff, d_model)), ("w2", (d_model, d_ff)), ("w3", (d_ff, d_model))):
        groups = -(-k // group)
        kp = groups * group
        if (k * bits) % 32:
            raise ValueError(f"K={k} at {bits} bits ends inside a word")
        row_total = kp * bits // 32
        row_valid = k * bits // 32 if kp != k else 0
        specs.append((f"{proj}.weight", (n, row_total), np.uint32, KIND_U32, 0.0, 0.0,
                      row_total if row_valid else 0, row_valid))
        f16 = scale_dtype == "float16"
        specs.append((f"{proj}.scales", (n, groups), np.uint16, KIND_F16_UNIFORM if f16 else KIND_BF16_UNIFORM,
                      float(scale_lo), float(scale_hi) - float(scale_lo), 0, 0))
        specs.append((f"{proj}.biases", (n, groups), np.uint16, KIND_F16_NORMAL if f16 else KIND_BF16_NORMAL,
                      float(bias_sigma), 0.0, 0, 0))
    return specs


def expert_tensors(seed: int, layer: int, expert: int, specs) -> dict[str, np.ndarray]:
    out = {}
    for name, shape, dtype, kind, p0, p1, rt, rv in specs:
        key = stream_key(seed, layer, expert, TENSOR_IDS[name])
        if kind == KIND_U32 and dtype == np.uint8:
            words = fill(KIND_U32, int(np.prod(shape)) // 4, key)
            out[name] = words.view(np.uint8).reshape(shape)
        else:
            n = int(np.prod(shape))
            out[name] = fill(kind, n, key, p0, p1, rt, rv).astype(dtype, copy=False).reshape(shape)
    return out


def router_tensors(seed: int, layer: int, n_experts: int, d_model: int,
                   w_sigma: float = 0.02, b_sigma: float = 0.01):
    """Router weight [E, D] bf16 bits and bias [E] fp32."""
    w = fill(KIND_BF16_NORMAL, n_experts * d_model, stream_key(seed, layer, ROUTER_W, 0), w_sigma)
    b = fill(KIND_F32_NORMAL, n_experts, stream_key(seed, layer, ROUTER_BIAS, 0), b_sigma)
    return w.reshape(n_experts, d_model), b


def activations(seed: int, stream: int, n_tokens: int, d_model: int, sigma: float = 1.0) -> np.ndarray:
    """bf16 bits [T, D] ~ N(0, sigma) (Irwin-Hall)."""
    x = fill(KIND_BF16_NORMAL, n_tokens * d_model, stream_key(seed, 0, ACTIVATION, stream), sigma)
    return x.reshape(n_tokens, d_model)
