"""Write the committed golden vectors under tests/golden/ from the oracle.

    python tests/golden/make_fixtures.py

The reference's own tests hold no vectors for this path and need MLX, which is
not importable here, so the fixtures are seeded inputs with the oracle's
outputs (the oracle is pinned by tests/test_oracle_*.py).  They freeze those
outputs: tests/test_golden.py checks the oracle still reproduces them, and
tests/test_gpu_golden.py checks the HIP library against them.  Small on
purpose (tens of KB each).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import fp8 as ofp8  # noqa: E402
from oracle import requant as orq  # noqa: E402
from oracle import router as orouter  # noqa: E402
from oracle.affine2 import dequantize_affine, pack_2bit  # noqa: E402
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits  # noqa: E402
from oracle.fp4 import dequantize_fp4_weight  # noqa: E402

SEED = 20260917


def router(rng):
    T, D, E, k = 5, 512, 64, 6
    x = f32_to_bf16_bits(rng.standard_normal((T, D)).astype(np.float32))
    w = f32_to_bf16_bits((rng.standard_normal((E, D)) * 0.02).astype(np.float32))
    b = (rng.standard_normal(E) * 0.01).astype(np.float32)
    out = {"x": x, "w": w, "bias": b}
    for name, score, order in (("softplus_asc", orouter.SCORE_SQRT_SOFTPLUS, orouter.ORDER_ASCENDING),
                               ("sigmoid_rank", orouter.SCORE_SIGMOID, orouter.ORDER_RANK)):
        idx, wt, sc = orouter.route(bf16_bits_to_f32(x), bf16_bits_to_f32(w), b, topk=k, route_scale=1.5,
                                    score=score, order=order)
        out.update({f"{name}_idx": idx, f"{name}_w": wt, f"{name}_scores": sc})
    return out


def fp4(rng):
    packed = rng.integers(0, 256, size=(32, 64), dtype=np.uint8)
    scales = rng.integers(119, 128, size=(32, 4), dtype=np.uint8)
    return {"packed": packed, "scales": scales, "dense": dequantize_fp4_weight(packed, scales).astype(np.float32)}


def q2(rng):
    n, k = 16, 320                               # a partial last group
    kp = 384
    q = rng.integers(0, 4, size=(n, kp), dtype=np.uint8)
    q[:, k:] = 0
    w = pack_2bit(q)
    s = f32_to_bf16_bits(rng.uniform(0.005, 0.05, size=(n, 3)).astype(np.float32))
    b = f32_to_bf16_bits(rng.normal(0, 0.02, size=(n, 3)).astype(np.float32))
    return {"w": w, "scales": s, "biases": b, "k": np.array([k], np.int32), "dense": dequantize_affine(w, s, b, k=k, group=128)}


def fp8(rng):
    x = f32_to_bf16_bits((rng.standard_normal((3, 256)) * np.exp2(rng.integers(-8, 8, size=(3, 1)))).astype(np.float32))
    q, e = ofp8.act_quant(bf16_bits_to_f32(x))
    d, f, m = 128, 96, 2

    def wt(n, kk):
        wb = rng.integers(0, 256, size=(n, kk), dtype=np.uint8)
        wb[(wb & 0x7F) == 0x7F] = 0x3F
        return wb, rng.integers(120, 131, size=(-(-n // 32), kk // 32), dtype=np.uint8)

    (w1, s1), (w3, s3), (w2, s2) = wt(f, d), wt(f, d), wt(d, f)
    xs = f32_to_bf16_bits(rng.standard_normal((m, d)).astype(np.float32))
    y = ofp8.shared_expert(bf16_bits_to_f32(xs), w1, s1, w3, s3, w2, s2, limit=10.0)
    return {"x": x, "q": q, "e": (e + 127).astype(np.uint8), "xs": xs, "w1": w1, "s1": s1, "w3": w3, "s3": s3,
            "w2": w2, "s2": s2, "y": f32_to_bf16_bits(y)}


def requant(rng):
    packed = rng.integers(0, 256, size=(8, 80), dtype=np.uint8)      # K = 160: a partial last group
    scales = rng.integers(119, 128, size=(8, 5), dtype=np.uint8)
    q, s, b = orq.requantize(dequantize_fp4_weight(packed, scales).astype(np.float32))
    return {"packed": packed, "scales": scales, "q": q, "q_scales": s, "q_biases": b}


FIXTURES = {"router": router, "fp4_dequant": fp4, "q2_dequant": q2, "fp8": fp8, "requant": requant}


def build(name: str) -> dict:
    return FIXTURES[name](np.random.default_rng([SEED, sorted(FIXTURES).index(name)]))


if __name__ == "__main__":
    for name in FIXTURES:
        np.savez_compressed(HERE / f"{name}.npz", **build(name))
        print(f"wrote {name}.npz ({(HERE / f'{name}.npz').stat().st_size} bytes)")
