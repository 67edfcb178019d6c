"""Pins for the router restatement (oracle/router.py).

Independent checks: the score functions against Python's libm in float64
(within one fp32 ulp of the correctly rounded value), the logit reduction
against ``math.fsum`` and against an explicit pairwise tree over the chunks in
natural order (the identity the GPU's xor butterfly relies on), top-k against a
brute-force sort with the stated tie rules, and the reference's invariants
(bias affects selection only; weights sum to route_scale).
"""
from __future__ import annotations

import math
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import router as R
from oracle.bf16 import round_bf16

ROOT = Path(__file__).resolve().parents[1]


def test_exp64_against_libm():
    a = np.concatenate([np.linspace(-200.0, 0.0, 20001), -np.abs(np.random.default_rng(0).normal(size=5000) * 30)])
    got = R.exp64(a)
    want = np.array([math.exp(v) for v in a])
    assert np.all(np.abs(got - want) <= 4.5e-16 * want + 1e-300)
    assert R.exp64(np.array([-250.0]))[0] == 0.0 and R.exp64(np.array([0.0]))[0] == 1.0


def test_log1p64_against_libm():
    t = np.concatenate([np.linspace(0.0, 1.0, 20001), np.exp(-np.linspace(0, 700, 5000))])
    got = R.log1p64(t)
    want = np.array([math.log1p(v) for v in t])
    assert np.all(np.abs(got - want) <= 8.9e-16 * want + 1e-300)


def _ulp_diff32(a, b):
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


@pytest.mark.parametrize("kind", [R.SCORE_SIGMOID, R.SCORE_SQRT_SOFTPLUS])
def test_score_fn_within_two_ulp(kind):
    """Both end in fp32 operations (1 / (1 + t) as the reference writes it; sqrt of an
    fp32 softplus), so they sit within 2 fp32 ulps of the correctly rounded value.
    Below z = -87 the fp32 softplus is subnormal and loses relative precision, in
    the reference's fp32 evaluation as here; scores there are < 1e-18."""
    z = np.concatenate([np.random.default_rng(1).normal(size=20000) * 3, np.linspace(-85, 100, 2001)]).astype(np.float32)
    got = R.score_fn(z, kind)
    if kind == R.SCORE_SIGMOID:
        want = np.array([1.0 / (1.0 + math.exp(-float(v))) for v in z])
    else:
        want = np.array([math.sqrt(max(float(v), 0.0) + math.log1p(math.exp(-abs(float(v))))) for v in z])
    assert _ulp_diff32(got, want.astype(np.float32)).max() <= 2


def _tree_pairwise(p):
    """Pairwise tree over the 64 partials in natural chunk order."""
    level = list(p)
    while len(level) > 1:
        level = [np.float32(level[i] + level[i + 1]) for i in range(0, len(level), 2)]
    return level[0]


def test_logits_fixed_order_is_sequential_chunks_then_pairwise_tree():
    rng = np.random.default_rng(2)
    d, e = 512, 5
    x = round_bf16(rng.normal(size=(2, d)).astype(np.float32))
    w = round_bf16((rng.normal(size=(e, d)) * 0.02).astype(np.float32))
    got = R.logits(x, w)
    ch = d // 64
    for t in range(2):
        for r in range(e):
            parts = []
            for c in range(64):
                acc = np.float32(0.0)
                for j in range(ch):
                    acc = np.float32(acc + np.float32(x[t, c * ch + j] * w[r, c * ch + j]))
                parts.append(acc)
            assert got[t, r] == _tree_pairwise(parts)
            exact = math.fsum(float(x[t, i]) * float(w[r, i]) for i in range(d))
            assert abs(got[t, r] - exact) <= 1e-5 * max(1.0, abs(exact))


def test_logits_gate_temp_divides():
    rng = np.random.default_rng(3)
    x = round_bf16(rng.normal(size=(2, 128)).astype(np.float32))
    w = round_bf16(rng.normal(size=(5, 128)).astype(np.float32))
    assert np.array_equal(R.logits(x, w, 2.0), R.logits(x, w) / np.float32(2.0))


def _brute_topk(sel, k, order):
    idx = list(range(len(sel)))
    if order == R.ORDER_ASCENDING:
        return sorted(idx, key=lambda j: (float(sel[j]), j))[-k:]
    return sorted(idx, key=lambda j: (-float(sel[j]), j))[:k]


@pytest.mark.parametrize("order", [R.ORDER_ASCENDING, R.ORDER_RANK])
def test_topk_against_bruteforce_with_ties(order):
    rng = np.random.default_rng(4)
    for trial in range(200):
        e = int(rng.integers(1, 40))
        k = int(rng.integers(1, e + 1))
        sel = rng.integers(0, 6, size=e).astype(np.float32)  # many exact ties
        got = R.topk_select(sel[None], k, order)[0].tolist()
        assert got == _brute_topk(sel, k, order), (trial, sel.tolist(), k)


def test_normalise_sum_order_and_k1():
    w = np.array([[0.25, 0.5, 0.125]], np.float32)
    got = R.normalise(w, 1.5, True)
    denom = np.float32(np.float32(np.float32(0.25) + np.float32(0.5)) + np.float32(0.125)) + np.float32(1e-20)
    assert np.array_equal(got, (w / denom) * np.float32(1.5))
    assert abs(float(got.sum()) - 1.5) < 1e-6
    one = np.array([[0.3]], np.float32)
    assert R.normalise(one, 2.0, True)[0, 0] == np.float32(0.3) * np.float32(2.0)  # topk == 1: no normalisation


def test_route_bias_affects_selection_only_and_bias_vl():
    rng = np.random.default_rng(5)
    x = round_bf16(rng.normal(size=(6, 128)).astype(np.float32))
    w = round_bf16((rng.normal(size=(16, 128)) * 0.1).astype(np.float32))
    b0 = np.zeros(16, np.float32)
    b1 = (rng.normal(size=16) * 0.5).astype(np.float32)
    i0, w0, s0 = R.route(x, w, b0, topk=4, score=R.SCORE_SIGMOID, route_scale=1.0)
    i1, w1, s1 = R.route(x, w, b1, topk=4, score=R.SCORE_SIGMOID, route_scale=1.0)
    assert np.array_equal(s0, s1)
    assert not np.array_equal(i0, i1)
    assert np.allclose(w1.sum(-1), 1.0, atol=1e-6)
    assert np.array_equal(w1, R.normalise(np.take_along_axis(s1, i1, -1), 1.0, True))
    mask = np.array([1, 0, 1, 0, 0, 1], bool)
    im, _, _ = R.route(x, w, b0, topk=4, score=R.SCORE_SIGMOID, bias_vl=b1, image_mask=mask)
    assert np.array_equal(im[mask], i1[mask]) and np.array_equal(im[~mask], i0[~mask])


def test_hip_constants_match_oracle():
    """The polynomial / reduction constants in router_math.h are the oracle's doubles."""
    src = (ROOT / "cachalot_amd/csrc/router_math.h").read_text()

    def arr(name):
        body = re.search(name + r"\[\d+\] = \{([^}]*)\}", src).group(1)
        return [float(v) for v in body.replace("\n", " ").split(",") if v.strip()]

    assert arr("EXP_COEF") == R.EXP_COEF
    assert arr("LOG1P_COEF") == R.LOG1P_COEF
    for name in ("INV_LN2", "LN2_HI", "LN2_LO"):
        v = float(re.search(rf"constexpr double {name} = ([0-9.e+-]+);", src).group(1))
        assert v == getattr(R, name)
    assert re.search(r"constexpr int CHUNKS = 64;", src) and R.N_CHUNKS == 64
