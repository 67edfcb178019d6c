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


def _torch_rows(x, mats, weights, limit, group):
    """The SwiGLU expert over rows in torch float64 with torch's own bf16 casts
    (fp64 -> fp32 -> bf16, as an fp32 accumulator cast to bf16), at the points of
    expert_affine.py:65-81 (g, u, h, y each cast to bf16; clamp skipped for limit 0)."""
    def dense(m):
        w, s, b, k = m
        return torch.from_numpy(dequantize_affine64(w, s, b, k=k, group=group))
    w1, w3, w2 = (dense(m) for m in mats)
    xt = torch.from_numpy(np.atleast_2d(x).astype(np.float64))
    bf = lambda t: t.float().to(torch.bfloat16).double()  # noqa: E731
    g = bf(xt @ w1.T)
    u = bf(xt @ w3.T)
    if limit > 0:
        u = u.clamp(-limit, limit)
        g = g.clamp(max=limit)
    wt = torch.from_numpy(np.asarray(weights, np.float32).astype(np.float64))[:, None]
    h = bf(torch.nn.functional.silu(g) * u * wt)
    return bf(h @ w2.T).float().numpy()


def _torch_expert(x, mats, weight, limit, group):
    return _torch_rows(x, mats, [weight], limit, group)[0]


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
    # bit-equal: the route-order fp32 sum of bf16-exact terms, each at the same casts
    assert np.array_equal(routed, want)
    tb = torch.from_numpy(routed + addend).to(torch.bfloat16).float().numpy()
    assert np.array_equal(out, tb)


def _rows_case(seed, limit):
    rng = np.random.default_rng(seed)
    d, f, group = 80, 56, 16        # D = 5 groups, F = 3.5 groups: a partial last group in W2
    m = 7
    # scaled so that some g and u exceed the clamp limit
    x = round_bf16((rng.normal(size=(m, d)) * 6).astype(np.float32))
    e = _affine_expert(rng, d, f, group)
    weights = rng.uniform(0.05, 1.5, size=m).astype(np.float32)
    return x, e, weights, group


def _oracle_rows(x, e, weights, limit, group):
    return experts.swiglu_rows(x, *[_mm(mm, group) for mm in e], weights, limit=limit)


def test_swiglu_rows_bit_equal_torch():
    for seed, limit in [(21, 10.0), (22, 1.0), (23, 0.0)]:
        x, e, weights, group = _rows_case(seed, limit)
        got = _oracle_rows(x, e, weights, limit, group)
        want = _torch_rows(x, e, weights, limit, group)
        assert np.array_equal(got, want), (seed, limit)


def test_swiglu_rows_clamp_engaged():
    """The limit-1 case clamps some g and u (else the clamp would go unpinned)."""
    x, e, weights, group = _rows_case(22, 1.0)
    a = _oracle_rows(x, e, weights, 1.0, group)
    b = _oracle_rows(x, e, weights, 0.0, group)
    assert not np.array_equal(a, b)


def test_swiglu_rows_pin_catches_each_dropped_cast(monkeypatch):
    """Mutation check: skipping any one of the g, u, h, y casts breaks bit-equality
    with torch, for the rows pin and for the decode pin."""
    real = experts.round_bf16
    for skip in range(4):
        calls = {"n": 0}

        def mutated(v, _skip=skip, _calls=calls):
            i = _calls["n"] % 4
            _calls["n"] += 1
            return np.asarray(v, np.float32) if i == _skip else real(v)

        monkeypatch.setattr(experts, "round_bf16", mutated)
        x, e, weights, group = _rows_case(21, 10.0)
        got = _oracle_rows(x, e, weights, 10.0, group)
        want = _torch_rows(x, e, weights, 10.0, group)
        assert not np.array_equal(got, want), f"dropping cast {skip} went unnoticed (rows)"
        calls["n"] = 0
        rng = np.random.default_rng(7)
        d, f, g16 = 64, 40, 16
        xd = round_bf16(rng.normal(size=d).astype(np.float32))
        ex = [_affine_expert(rng, d, f, g16) for _ in range(3)]
        wts = np.array([0.5, 0.3, 0.2], np.float32)
        routed, _ = experts.affine_decode(xd, [tuple(_mm(m, g16) for m in q) for q in ex], wts, 10.0)
        want_d = np.zeros(d, np.float32)
        for q, w in zip(ex, wts):
            want_d = want_d + _torch_expert(xd, q, w, 10.0, g16)
        assert not np.array_equal(routed, want_d), f"dropping cast {skip} went unnoticed (decode)"
        monkeypatch.setattr(experts, "round_bf16", real)


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
