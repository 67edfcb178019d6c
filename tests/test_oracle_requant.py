"""Pins for the FP4 -> 2-bit requantizer restatement (oracle/requant.py).

Independent checks: the min/max fit's closed form on an exactly representable
group; the searched fit against a brute-force float64 evaluation of all 25
candidates (it must pick one whose error is the minimum up to float32 rounding);
the codes against a brute-force nearest level; the reference's own fit-quality
property (tests/test_quant_affine.py:63-80: the search beats both the min/max
fit and MLX's symmetric max-abs fit on Gaussian weights); a partial last group.
"""
from __future__ import annotations

import numpy as np

from oracle import requant as R
from oracle.affine2 import unpack_2bit
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits


def _candidates64(w):
    lo, hi = w.min(), w.max()
    mid = (lo + hi) / 2
    out = [(max((hi - lo) / 3, 1e-8), lo)]
    for a in R.SHRINKS:
        for b in R.SHRINKS:
            if a == 1.0 and b == 1.0:
                continue
            nl, nh = mid + (lo - mid) * a, mid + (hi - mid) * b
            out.append((max((nh - nl) / 3, 1e-8), nl))
    return out


def _err64(w, s, b):
    q = np.clip(np.round((w - b) / s), 0, 3)
    return float(np.sum((s * q + b - w) ** 2))


def test_minmax_closed_form_and_exact_group():
    w = (np.arange(128) % 4 * 0.5 + 1.0).astype(np.float32)[None]
    s, b = R.fit_search(w, np.ones_like(w, bool))
    assert s[0, 0] == np.float32(0.5) and b[0, 0] == np.float32(1.0)
    packed, sb, bb = R.requantize(w)
    assert np.array_equal(unpack_2bit(packed, 128)[0], np.arange(128) % 4)
    assert bf16_bits_to_f32(sb)[0, 0] == 0.5 and bf16_bits_to_f32(bb)[0, 0] == 1.0


def test_search_picks_the_least_error_candidate():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((400, 128)) * rng.uniform(0.01, 2.0, size=(400, 1))).astype(np.float32)
    w[::7] = np.sign(w[::7]) * np.abs(w[::7]) ** 3                      # heavy tails
    s, b = R.fit_search(w, np.ones_like(w, bool))
    for g in range(w.shape[0]):
        x = w[g].astype(np.float64)
        errs = [_err64(x, cs, cb) for cs, cb in _candidates64(x)]
        got = _err64(x, float(s[g, 0]), float(b[g, 0]))
        assert got <= min(errs) * (1 + 1e-4) + 1e-12, g


def test_codes_are_the_nearest_level():
    rng = np.random.default_rng(4)
    dense = rng.standard_normal((64, 256)).astype(np.float32)
    packed, sb, bb = R.requantize(dense)
    q = unpack_2bit(packed, 256).astype(np.float64)
    s = np.repeat(bf16_bits_to_f32(sb), 128, axis=1).astype(np.float64)
    b = np.repeat(bf16_bits_to_f32(bb), 128, axis=1).astype(np.float64)
    dist = np.abs(s[..., None] * np.arange(4) + b[..., None] - dense[..., None])
    best = dist.min(axis=-1)
    mine = np.abs(s * q + b - dense)
    assert np.all(mine <= best + 1e-6 * np.abs(dense).max())


def test_search_beats_minmax_and_symmetric_fit():
    rng = np.random.default_rng(13)
    w = rng.standard_normal((32, 512)).astype(np.float32)
    packed, sb, bb = R.requantize(w)
    deq = (unpack_2bit(packed, 512) * np.repeat(bf16_bits_to_f32(sb), 128, 1) + np.repeat(bf16_bits_to_f32(bb), 128, 1))
    g = w.reshape(-1, 128).astype(np.float64)
    # min/max fit
    lo, hi = g.min(1, keepdims=True), g.max(1, keepdims=True)
    sm = (hi - lo) / 3
    mm = np.clip(np.round((g - lo) / sm), 0, 3) * sm + lo
    # MLX's symmetric fit: levels (q - 2) * amax / 2
    sa = np.abs(g).max(1, keepdims=True) / 2
    sym = np.clip(np.round(g / sa) + 2, 0, 3) * sa - 2 * sa

    def rel(d):
        return np.sqrt(np.sum((d.reshape(w.shape) - w) ** 2) / np.sum(w.astype(np.float64) ** 2))

    assert rel(deq) < rel(mm) and rel(deq) < rel(sym)


def test_partial_last_group_fits_real_elements_only():
    rng = np.random.default_rng(5)
    dense = rng.standard_normal((8, 160)).astype(np.float32)
    packed, sb, bb = R.requantize(dense)
    assert packed.shape == (8, 16) and sb.shape == (8, 2)
    assert np.all(unpack_2bit(packed, 256)[:, 160:] == 0)
    # the last group's fit equals the fit of its 32 real values alone
    s, b = R.fit_search(dense[:, 128:], np.ones((8, 32), bool))
    assert np.array_equal(sb[:, 1], f32_to_bf16_bits(s[:, 0])) and np.array_equal(bb[:, 1], f32_to_bf16_bits(b[:, 0]))


def _rel(dense, packed, sb, bb, group, bits):
    from oracle.affine2 import dequantize_affine

    got = dequantize_affine(packed, sb, bb, k=dense.shape[1], group=group, bits=bits).astype(np.float64)
    return float(np.linalg.norm(got - dense) / np.linalg.norm(dense))


def test_lsq_refinement_never_loses_to_the_grid_it_refines():
    """The reference's own pin (tests/test_quant_affine.py:112-126): per group the refinement
    keeps the grid's fit unless it beats it, so search-lsq <= search and wide-lsq <= search-lsq
    on Gaussian weights; levels stay inside the width."""
    from oracle.affine2 import unpack_bits

    rng = np.random.default_rng(15)
    w = rng.standard_normal((32, 512)).astype(np.float32)
    for group in (64, 128):
        err = {f: _rel(w, *R.requantize(w, group, fit_name=f), group, 2) for f in ("search", "search-lsq", "wide-lsq")}
        assert err["search-lsq"] <= err["search"] and err["wide-lsq"] <= err["search-lsq"], err
    packed, _, _ = R.requantize(w, 128, fit_name="wide-lsq")
    assert unpack_bits(packed, 2).max() <= 3


def test_lsq_step_is_the_least_squares_line():
    """With the levels fixed, the refit is the float64 least-squares line through (q, w)
    (numpy.polyfit), rounded to bf16 -- an independent closed form."""
    rng = np.random.default_rng(3)
    w = rng.standard_normal((6, 64)).astype(np.float32)
    v = np.ones_like(w, bool)
    s, b = R.fit_search(w, v)
    ns, nb = R.lsq_step(w, v, s, b)
    q = R._q(w, s, b)
    for i in range(6):
        slope, icpt = np.polyfit(q[i].astype(np.float64), w[i].astype(np.float64), 1)
        assert abs(ns[i, 0] - slope) <= 2 ** -7 * abs(slope) + 1e-6
        assert abs(nb[i, 0] - icpt) <= 2 ** -7 * abs(icpt) + 1e-6


def test_search_fit_beats_minmax_every_width_and_group():
    """tests/test_quant_affine.py:70-86 and :206-220 at 2 and 3 bits, every group size; 4 bits too."""
    rng = np.random.default_rng(13)
    w = rng.standard_normal((32, 512)).astype(np.float32)
    for bits in (2, 3, 4):
        for group in (32, 64, 128):
            e_s = _rel(w, *R.requantize(w, group, bits=bits), group, bits)
            e_m = _rel(w, *R.requantize(w, group, bits=bits, fit_name="minmax"), group, bits)
            assert e_s < e_m, (bits, group)
    e2 = _rel(w, *R.requantize(w, 64, bits=2), 64, 2)
    e3 = _rel(w, *R.requantize(w, 64, bits=3), 64, 3)
    e4 = _rel(w, *R.requantize(w, 64, bits=4), 64, 4)
    assert e4 < e3 < e2


def test_importance_weighting():
    """quant_affine.py:125-134: unit importance is the unweighted fit bit for bit; columns of
    zero importance do not move the fit; the weighted error on the important columns is no
    worse than the unweighted fit's."""
    rng = np.random.default_rng(21)
    w = rng.standard_normal((8, 256)).astype(np.float32)
    for f in ("search", "search-lsq", "wide-lsq"):
        a = R.requantize(w, 64, fit_name=f)
        b = R.requantize(w, 64, fit_name=f, importance=np.ones(256, np.float32))
        assert all(np.array_equal(x, y) for x, y in zip(a, b)), f
    # the weighted search picks, among the same candidates, the one of least weighted error:
    # never worse (in its own float32 error) than the unweighted winner
    imp = rng.uniform(0.0, 2.0, size=256).astype(np.float32)
    g = w.reshape(-1, 64)
    v = np.ones_like(g, bool)
    wts = np.tile(imp.reshape(-1, 64), (8, 1))
    s_u, b_u = R.fit_search(g, v)
    s_w, b_w = R.fit_search(g, v, weights=wts)
    e_u = R.group_error(g, v, s_u, b_u, weights=wts)
    e_w = R.group_error(g, v, s_w, b_w, weights=wts)
    assert np.all(e_w <= e_u) and np.any(e_w < e_u)


def test_lsq_step_keeps_the_pair_where_the_line_is_not_defined():
    """A group whose levels collapse (every code equal: |den| < 1e-12) and a group whose
    importance is zero throughout (a zero weight total) keep the pair they came in with."""
    w = np.full((1, 64), 0.75, np.float32)
    v = np.ones_like(w, bool)
    s0, b0 = np.array([[0.25]], np.float32), np.array([[0.5]], np.float32)
    ns, nb = R.lsq_step(w, v, s0, b0)
    assert ns[0, 0] == s0[0, 0] and nb[0, 0] == b0[0, 0]
    rng = np.random.default_rng(4)
    w = rng.standard_normal((1, 64)).astype(np.float32)
    s, b = R.fit_search(w, v)
    ns, nb = R.lsq_step(w, v, s, b, weights=np.zeros_like(w))
    assert ns[0, 0] == s[0, 0] and nb[0, 0] == b[0, 0]
