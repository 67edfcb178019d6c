"""Pins for the expert math and dispatch restatements.

Independent checks: torch float64 matmuls and torch's own sigmoid / bf16
casts for the SwiGLU expert at the reference's rounding points, the E2M1 bit
definition for FP4 weights, and the reference's dict-of-lists assignment loop
(moe_prefill_grouped.py:199-225, re-run here as plain Python) for the permute.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import dispatch, experts
from oracle.affine2 import dequantize_affine64, pack_2bit, qmv64
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16
from oracle.fp4 import dequantize_fp4_weight


def _affine_expert(rng, d, f, group):
    def mat(n, k):
        kp = -(-k // group) * group
        q = rng.integers(0, 4, size=(n, kp), dtype=np.uint8)
        q[:, k:] = 0
        s = f32_to_bf16_bits(rng.uniform(0.005, 0.05, size=(n, kp // group)).astype(np.float32))
        b = f32_to_bf16_bits(rng.normal(0, 0.02, size=(n, kp // group)).astype(np.float32))
        return pack_2bit(q), s, b, k
    return mat(f, d), mat(f, d), mat(d, f)


def _mm(m, group):
    w, s, b, k = m
    return lambda x: qmv64(x, w, s, b, k=k, group=group)


def _torch_expert(x, mats, weight, limit, group):
    """Same expert in torch float64 with torch's bf16 casts."""
    def dense(m):
        w, s, b, k = m
        return torch.from_numpy(dequantize_affine64(w, s, b, k=k, group=group))
    w1, w3, w2 = (dense(m) for m in mats)
    xt = torch.from_numpy(x.astype(np.float64))
    bf = lambda t: t.float().to(torch.bfloat16).double()  # noqa: E731
    g = bf(w1 @ xt)
    u = bf(w3 @ xt)
    u = u.clamp(-limit, limit)
    g = g.clamp(max=limit)
    h = bf(torch.nn.functional.silu(g) * u * float(np.float32(weight)))
    return bf(w2 @ h).float().numpy()


def test_affine_decode_matches_torch_reference():
    rng = np.random.default_rng(7)
    d, f, group = 64, 40, 16          # F = 2.5 groups: exercises the padded last group
    x = round_bf16(rng.normal(size=d).astype(np.float32))
    ex = [_affine_expert(rng, d, f, group) for _ in range(3)]
    weights = np.array([0.5, 0.3, 0.2], np.float32)
    addend = round_bf16(rng.normal(size=d).astype(np.float32))
    routed, out = experts.affine_decode(x, [tuple(_mm(m, group) for m in e) for e in ex], weights, 10.0, addend)
    want = np.zeros(d, np.float32)
    for e, w in zip(ex, weights):
        want = want + _torch_expert(x, e, w, 10.0, group)
    assert np.allclose(routed, want, rtol=0, atol=4e-3 * np.abs(want).max())
    tb = torch.from_numpy(routed + addend).to(torch.bfloat16).float().numpy()
    assert np.array_equal(out, tb)


def test_swiglu_limit_zero_disables_clamp():
    rng = np.random.default_rng(8)
    d, f, group = 32, 32, 16
    x = round_bf16((rng.normal(size=(2, d)) * 40).astype(np.float32))
    e = _affine_expert(rng, d, f, group)
    mm = [_mm(m, group) for m in e]
    a = experts.swiglu_rows(x, *mm, np.array([1.0, 1.0], np.float32), limit=0.0)
    b = experts.swiglu_rows(x, *mm, np.array([1.0, 1.0], np.float32), limit=1.0)
    assert not np.array_equal(a, b)


def test_fp4_decode_matches_torch_reference():
    rng = np.random.default_rng(9)
    d, f = 64, 96
    x = round_bf16(rng.normal(size=d).astype(np.float32))

    def mat(n, k):
        return dequantize_fp4_weight(rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8),
                                     rng.integers(119, 128, size=(n, k // 32), dtype=np.uint8))
    dense = [(mat(f, d), mat(f, d), mat(d, f)) for _ in range(2)]
    weights = np.array([0.7, 0.3], np.float32)
    got = experts.fp4_decode(x, dense, weights, 10.0)
    xt = torch.from_numpy(x.astype(np.float64))
    want = torch.zeros(d, dtype=torch.float64)
    for (w1, w3, w2), w in zip(dense, weights):
        g = (torch.from_numpy(w1).double() @ xt).clamp(max=10.0)
        u = (torch.from_numpy(w3).double() @ xt).clamp(-10.0, 10.0)
        want += torch.from_numpy(w2).double() @ (torch.nn.functional.silu(g) * u * float(w))
    assert np.allclose(got, want.numpy(), rtol=1e-6, atol=1e-6 * float(want.abs().max()))


def test_permute_matches_reference_assignment_loop():
    rng = np.random.default_rng(10)
    t, k, e = 50, 6, 20
    idx = np.stack([rng.choice(e, size=k, replace=False) for _ in range(t)])
    got = dispatch.permute(idx, e)
    # reference construction: assignments[expert] = [(token, slot), ...] in token order
    assignments: dict[int, list] = {}
    for token in range(t):
        for slot, ex in enumerate(idx[token]):
            assignments.setdefault(int(ex), []).append((token, slot))
    pos = 0
    for ex in range(e):
        rows = assignments.get(ex, [])
        assert got["offsets"][ex] == pos and got["offsets"][ex + 1] == pos + len(rows)
        for token, slot in rows:
            assert (got["token"][pos], got["slot"][pos]) == (token, slot)
            assert got["pos"][token, slot] == pos
            pos += 1
    assert pos == t * k


def test_combine_slot_order_and_cast():
    rng = np.random.default_rng(11)
    t, k, d = 5, 3, 8
    y = round_bf16(rng.normal(size=(t * k, d)).astype(np.float32))
    pos = rng.permutation(t * k).reshape(t, k)
    add = round_bf16(rng.normal(size=(t, d)).astype(np.float32))
    routed, out = dispatch.combine(y, pos, add)
    for i in range(t):
        acc = y[pos[i, 0]].copy()
        for s in range(1, k):
            acc = (acc + y[pos[i, s]]).astype(np.float32)
        assert np.array_equal(routed[i], acc)
        assert np.array_equal(out[i], torch.from_numpy(acc + add[i]).to(torch.bfloat16).float().numpy())


def test_bf16_helpers_roundtrip():
    v = np.array([1.0, -2.5, 3.140625], np.float32)
    assert np.array_equal(bf16_bits_to_f32(f32_to_bf16_bits(v)), v)
