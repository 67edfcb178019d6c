"""Seeded synthetic banks, router weights and activations, generated on the GPU.

The reference loads real checkpoints; the configs this build is measured on
use seeded synthetic data instead (no checkpoint is available offline).  Data
is produced in HBM by ``cachalot_fill_synthetic`` (counter-based SplitMix64
stream, see ``csrc/synth.hip``) so a 150 GB bank fills in seconds.

Distributions: FP4 nibbles uniform, E8M0 raw uniform in
[119, 127] (2^-8 .. 2^0); 2-bit codes uniform, scales U(0.005, 0.05), biases
N(0, 0.02) as bf16; router weight N(0, 0.02) bf16, bias N(0, 0.01) fp32;
activations N(0, 1) bf16.  "Normal" is the Irwin-Hall sum of four 16-bit
uniforms scaled to the requested standard deviation.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from .storage.index import ExpertFormat

MASK = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15
M1 = 0xBF58476D1CE4E5B9
M2 = 0x94D049BB133111EB

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
ROUTER_W = 1 << 20
ROUTER_BIAS = (1 << 20) + 1
ACTIVATION = (1 << 20) + 2


def fmix64(z: int) -> int:
    z &= MASK
    z = ((z ^ (z >> 30)) * M1) & MASK
    z = ((z ^ (z >> 27)) * M2) & MASK
    return z ^ (z >> 31)


def stream_key(seed: int, layer: int, expert: int, tensor: int) -> int:
    k = fmix64((seed + GAMMA) & MASK)
    k = fmix64(k ^ ((layer * GAMMA) & MASK))
    k = fmix64(k ^ expert)
    k = fmix64((k + tensor * M2) & MASK)
    return k


def fill(dst: torch.Tensor, kind: int, key: int, p0: float = 0.0, p1: float = 0.0,
         row_total: int = 0, row_valid: int = 0, start: int = 0, n: int | None = None) -> None:
    """Fill `dst` (a contiguous device tensor) element-wise; element size follows the kind."""
    _lib.require_cuda(dst)
    item = {KIND_U32: 4, KIND_E8M0: 1, KIND_BF16_UNIFORM: 2, KIND_BF16_NORMAL: 2, KIND_F32_NORMAL: 4,
            KIND_F16_UNIFORM: 2, KIND_F16_NORMAL: 2}[kind]
    if n is None:
        n = dst.numel() * dst.element_size() // item
    if kind in (KIND_BF16_NORMAL, KIND_F32_NORMAL, KIND_F16_NORMAL):
        p1 = p0 / IRWIN_HALL_STD
    rc = _lib.lib().cachalot_fill_synthetic(dst.data_ptr(), n, start, key, kind, float(p0), float(p1),
                                            row_total, row_valid, _lib.stream_handle(dst.device))
    _lib.check(rc, "fill_synthetic")


def tensor_specs(fmt: ExpertFormat, *, e8m0_lo: int = 119, e8m0_hi: int = 127, scale_lo: float = 0.005,
                 scale_hi: float = 0.05, bias_sigma: float = 0.02):
    """(name, kind, p0, p1, row_total, row_valid) per tensor of one expert."""
    specs = []
    if fmt.kind == "fp4":
        for proj in ("w1", "w2", "w3"):
            specs.append((f"{proj}.weight", KIND_U32, 0.0, 0.0, 0, 0))
            specs.append((f"{proj}.scale", KIND_E8M0, float(e8m0_lo), float(e8m0_hi), 0, 0))
        return specs
    for proj, k in (("w1", fmt.d_model), ("w2", fmt.d_ff), ("w3", fmt.d_model)):
        row_total = fmt.shapes[f"{proj}.weight"][1]
        row_valid = k * fmt.bits // 32
        pad = row_valid != row_total
        specs.append((f"{proj}.weight", KIND_U32, 0.0, 0.0, row_total if pad else 0, row_valid if pad else 0))
        f16 = fmt.dtypes[f"{proj}.scales"] == "float16"
        specs.append((f"{proj}.scales", KIND_F16_UNIFORM if f16 else KIND_BF16_UNIFORM, float(scale_lo),
                      float(scale_hi) - float(scale_lo), 0, 0))
        specs.append((f"{proj}.biases", KIND_F16_NORMAL if f16 else KIND_BF16_NORMAL, float(bias_sigma), 0.0, 0, 0))
    return specs


def fill_expert(arrays: dict[str, torch.Tensor], fmt: ExpertFormat, seed: int, layer: int, expert: int,
                **spec_kw) -> None:
    """Write one synthetic expert into its slot views (uint8 device tensors)."""
    for name, kind, p0, p1, rt, rv in tensor_specs(fmt, **spec_kw):
        fill(arrays[name], kind, stream_key(seed, layer, expert, TENSOR_IDS[name]), p0, p1, rt, rv)


def router_weights(seed: int, layer: int, n_experts: int, d_model: int, device, *, w_sigma: float = 0.02,
                   b_sigma: float = 0.01):
    """(weight [E, D] bf16, bias [E] fp32) on `device`."""
    w = torch.empty((n_experts, d_model), dtype=torch.bfloat16, device=device)
    b = torch.empty((n_experts,), dtype=torch.float32, device=device)
    fill(w, KIND_BF16_NORMAL, stream_key(seed, layer, ROUTER_W, 0), w_sigma)
    fill(b, KIND_F32_NORMAL, stream_key(seed, layer, ROUTER_BIAS, 0), b_sigma)
    return w, b


def activations(seed: int, stream: int, n_tokens: int, d_model: int, device, sigma: float = 1.0) -> torch.Tensor:
    x = torch.empty((n_tokens, d_model), dtype=torch.bfloat16, device=device)
    fill(x, KIND_BF16_NORMAL, stream_key(seed, 0, ACTIVATION, stream), sigma)
    return x


def zipf_bias(n_experts: int, *, seed: int, exponent: float = 1.1, strength: float = 0.5) -> list[float]:
    """Per-expert additive router bias strength * (rank+1)^-exponent over a seeded
    permutation of ranks (config 3's skewed loads).  Host-side Python floats."""
    order = list(range(n_experts))
    state = seed & MASK
    for i in range(n_experts - 1, 0, -1):  # Fisher-Yates with the same counter stream
        state = fmix64((state + GAMMA) & MASK)
        j = state % (i + 1)
        order[i], order[j] = order[j], order[i]
    bias = [0.0] * n_experts
    for rank, e in enumerate(order):
        bias[e] = strength * (rank + 1) ** (-exponent)
    return bias
