"""GPU parity of the expert-major (prefill / batched decode) path.

permute: bit-exact against ``oracle.dispatch.permute`` (the reference's
assignment order, ``moe_prefill_grouped.py:199-225``).  Grouped experts: every
(token, route slot) row against ``oracle.experts.swiglu_rows`` (bf16 rounding
points of ``affine_expert_forward_batched`` / ``routed_expert_forward_sgmm``),
combined in slot order (``oracle.dispatch.combine``); bar 2e-3 of max|want| plus
one bf16 ulp per summed expert term (each y is a bf16 cast).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import SEED, bf16_terms_ok, bf16_ulp, fp4_dense, make_store, oracle_tensors, q2_mats, rel_err
from oracle import dispatch as odispatch
from oracle import experts as oexperts
from oracle import router as orouter
from oracle import synth as osynth
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _np(t):
    return t.detach().cpu().numpy()


def _bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)


def _bits(t):
    return _np(t.contiguous().view(torch.int16)).view(np.uint16)


def _zipf_routes(rng, t, k, experts):
    """Distinct experts per token, drawn with a Zipf-like skew over `experts`."""
    experts = np.asarray(experts)
    p = 1.0 / np.arange(1, len(experts) + 1) ** 1.1
    p /= p.sum()
    idx = np.stack([rng.choice(experts, size=k, replace=False, p=p) for _ in range(t)]).astype(np.int32)
    w = rng.dirichlet(np.ones(k), size=t).astype(np.float32)
    return idx, w


def _mats(fmt, layer, e):
    tens = oracle_tensors(fmt, layer, e)
    if fmt.kind == "affine":
        return q2_mats(fmt, tens)
    w1, w3, w2 = fp4_dense(tens)

    def mm(w):
        w64 = np.asarray(w, np.float64)
        return lambda v: np.asarray(v, np.float64) @ w64.T

    return mm(w1), mm(w3), mm(w2)


def _oracle_grouped(fmt, layer, x, idx, w, drop=()):
    """-> (routed fp32 [T, D], y [T, k, D] bf16-exact) with the reference's rounding points."""
    t, k = idx.shape
    y = np.zeros((t, k, fmt.d_model), np.float32)
    for e in np.unique(idx):
        if int(e) in drop:
            continue
        rows = np.argwhere(idx == e)
        mm1, mm3, mm2 = _mats(fmt, layer, int(e))
        ye = oexperts.swiglu_rows(x[rows[:, 0]], mm1, mm3, mm2, w[rows[:, 0], rows[:, 1]], 10.0)
        y[rows[:, 0], rows[:, 1]] = ye
    p = odispatch.permute(idx, 1 << 20)
    y_rows = np.zeros((t * k, fmt.d_model), np.float32)
    y_rows[p["pos"].reshape(-1)] = y.reshape(t * k, -1)
    routed, _ = odispatch.combine(y_rows, p["pos"])
    return routed, y


def _check_rows(routed, want, ys, what):
    for r in range(want.shape[0]):
        assert bf16_terms_ok(routed[r], want[r], ys[r], TOL), (what, r, rel_err(routed[r], want[r]))
    frac = np.mean(np.abs(routed.astype(np.float64) - want) > TOL * np.abs(want).max())
    assert frac <= 0.01, (what, frac)


def test_permute_matches_oracle(cuda):
    from cachalot_amd.moe_prefill import permute

    rng = np.random.default_rng(3)
    # one-workgroup permute up to 1024 routes, the two-kernel one past it; the last
    # two cases carry ids outside [0, E) (dropped routes, weight 0, after every expert)
    cases = [(1, 6, 384), (5, 1, 7), (170, 6, 384), (171, 6, 384), (128, 8, 1024), (300, 6, 384), (1000, 8, 64),
             (32, 6, 384), (200, 6, 64)]
    for n_case, (t, k, e) in enumerate(cases):
        idx, w = _zipf_routes(rng, t, k, np.arange(e))
        if n_case >= len(cases) - 2:
            idx = idx.copy()
            idx[0, 1], idx[t // 2, 0], idx[t - 1, k - 1] = -3, e, 1 << 30
        offs, tok, slot, rw = permute(torch.from_numpy(idx).to(cuda), torch.from_numpy(w).to(cuda), e)
        p = odispatch.permute(idx, e)
        assert np.array_equal(_np(offs), p["offsets"])
        assert np.array_equal(_np(tok), p["token"]) and np.array_equal(_np(slot), p["slot"])
        keep = (idx >= 0) & (idx < e)
        assert np.array_equal(_np(rw), np.where(keep, w, 0)[p["token"], p["slot"]])


def test_permute_errors(cuda):
    from cachalot_amd import _lib

    L = _lib.lib()
    assert L.cachalot_permute(None, None, 1, 6, 384, None, None, None, None, None) == _lib.EINVAL
    assert L.cachalot_permute(1, 1, 1, 6, 2000, 1, 1, 1, 1, None) == _lib.EINVAL
    assert "E=2000" in _lib.last_error()


@pytest.mark.parametrize("kind", ["affine", "fp4", "affine_f16"])
def test_grouped_experts_prefill_tiles(cuda, kind, prefill_path):
    """64-row tiles (T*k >= 4E): an expert with more rows than one tile, ragged tails
    (2-bit banks with bf16 and with fp16 scales / biases)."""
    from cachalot_amd.moe_prefill import grouped_experts
    from cachalot_amd.storage.index import affine_format, fp4_format

    fmt = (fp4_format(4096, 2880) if kind == "fp4" else
           affine_format(4096, 2880, scale_dtype="float16" if kind == "affine_f16" else "bfloat16"))
    E = 8
    store = make_store(fmt, n_layers=1, n_experts=E)
    rng = np.random.default_rng(11)
    t, k = 90, 2
    idx, w = _zipf_routes(rng, t, k, np.arange(E))
    idx[:, 0] = 0                                  # expert 0: 90 rows -> two tiles
    idx[:, 1] = np.where(idx[:, 1] == 0, 1, idx[:, 1])
    xb = osynth.activations(SEED, 300, t, 4096)
    x = bf16_bits_to_f32(xb)
    routed, out = grouped_experts(_bf16(xb, cuda), torch.from_numpy(idx).to(cuda), torch.from_numpy(w).to(cuda),
                                  store.pool, store.layer_table(0), want_routed=True)
    want, ys = _oracle_grouped(fmt, 0, x, idx, w)
    _check_rows(_np(routed), want, ys, kind)
    got_out = bf16_bits_to_f32(_bits(out))
    assert np.all(np.abs(got_out - want) <= TOL * np.abs(want).max() + np.sum(bf16_ulp(ys), axis=1)
                  + bf16_ulp(want))


@pytest.mark.parametrize("kind", ["affine", "fp4", "affine_f16"])
def test_grouped_experts_batched_decode(cuda, kind):
    """16-row tiles (few rows per expert, BASELINE config 2 shape), a missing expert, an addend."""
    from cachalot_amd.moe_prefill import grouped_experts
    from cachalot_amd.storage.index import affine_format, fp4_format

    fmt = (fp4_format(4096, 2880) if kind == "fp4" else
           affine_format(4096, 2880, scale_dtype="float16" if kind == "affine_f16" else "bfloat16"))
    rng = np.random.default_rng(12)
    t, k = 4, 6
    experts = [3, 17, 100, 101, 250, 383, 42, 7]
    idx, w = _zipf_routes(rng, t, k, experts)
    store = make_store(fmt, n_layers=1, n_experts=384, keys=[(0, e) for e in experts], n_slots=len(experts))
    store.track_slots()[0, 42] = -1                  # expert 42 lost its slot: zero rows
    xb = osynth.activations(SEED, 400, t, 4096)
    ab = osynth.activations(SEED, 401, t, 4096)
    routed, out = grouped_experts(_bf16(xb, cuda), torch.from_numpy(idx).to(cuda), torch.from_numpy(w).to(cuda),
                                  store.pool, store.layer_table(0), addend=_bf16(ab, cuda), want_routed=True)
    want, ys = _oracle_grouped(fmt, 0, bf16_bits_to_f32(xb), idx, w, drop=(42,))
    _check_rows(_np(routed), want, ys, kind)
    a = bf16_bits_to_f32(ab)
    got_out = bf16_bits_to_f32(_bits(out))
    assert np.all(np.abs(got_out - (want + a)) <= TOL * np.abs(want + a).max() + np.sum(bf16_ulp(ys), axis=1)
                  + bf16_ulp(want + a))


@pytest.mark.parametrize("t", [1, 4, 7, 200])
def test_grouped_batched_routes_outside_range(cuda, t):
    """The batched 2-bit decode permutes its routes inside the prep launch (up to 1,024
    routes; T = 200, 1,200 routes, goes through the separate permute first): ids outside
    [0, E) are dropped (zero y rows, after every expert) and the rest match the oracle."""
    from cachalot_amd.moe_prefill import grouped_experts
    from cachalot_amd.storage.index import affine_format

    fmt = affine_format(4096, 2880)
    rng = np.random.default_rng(40 + t)
    k = 6
    experts = [3, 17, 100, 101, 250, 383, 7]
    idx, w = _zipf_routes(rng, t, k, experts)
    idx[0, 1] = -3
    idx[t - 1, k - 1] = 384
    if t > 7:
        idx[t // 2, 0] = -3
        idx[t // 3, 2] = 384
    store = make_store(fmt, n_layers=1, n_experts=384, keys=[(0, e) for e in experts], n_slots=len(experts))
    xb = osynth.activations(SEED, 410 + t, t, 4096)
    routed, _ = grouped_experts(_bf16(xb, cuda), torch.from_numpy(idx).to(cuda), torch.from_numpy(w).to(cuda),
                                store.pool, store.layer_table(0), want_routed=True)
    want, ys = _oracle_grouped(fmt, 0, bf16_bits_to_f32(xb), idx, w, drop=(-3, 384))
    _check_rows(_np(routed), want, ys, f"routes outside [0, E), T={t}")


@pytest.mark.parametrize("path", ["matrix_core", "bf16"])
@pytest.mark.parametrize("shape", [(4096, 2880), (5120, 2304)])
def test_grouped_batched_decode_many_rows(cuda, path, shape, monkeypatch):
    """2-bit batched decode with several rows per expert (B = 32 tokens over 40 experts):
    the matrix-core batched kernels (default) and the bf16 grouped kernels
    (CACHALOT_GROUPED_SMALL=1) against the oracle."""
    from cachalot_amd.moe_prefill import grouped_experts
    from cachalot_amd.storage.index import affine_format

    monkeypatch.setenv("CACHALOT_GROUPED_SMALL", "1" if path == "bf16" else "0")
    D, F = shape
    fmt = affine_format(D, F)
    rng = np.random.default_rng(13)
    t, k = 32, 6
    experts = list(rng.choice(384, size=40, replace=False))
    idx, w = _zipf_routes(rng, t, k, experts)
    store = make_store(fmt, n_layers=1, n_experts=384, keys=[(0, int(e)) for e in experts], n_slots=len(experts))
    xb = osynth.activations(SEED, 700, t, D)
    routed, out = grouped_experts(_bf16(xb, cuda), torch.from_numpy(idx).to(cuda), torch.from_numpy(w).to(cuda),
                                  store.pool, store.layer_table(0), want_routed=True)
    want, ys = _oracle_grouped(fmt, 0, bf16_bits_to_f32(xb), idx, w)
    _check_rows(_np(routed), want, ys, path)


def test_grouped_is_deterministic(cuda):
    from cachalot_amd.moe_prefill import grouped_experts
    from cachalot_amd.storage.index import affine_format

    fmt = affine_format(512, 256)
    store = make_store(fmt, n_layers=1, n_experts=16)
    rng = np.random.default_rng(5)
    idx, w = _zipf_routes(rng, 200, 6, np.arange(16))
    xb = osynth.activations(SEED, 500, 200, 512)
    args = (_bf16(xb, cuda), torch.from_numpy(idx).to(cuda), torch.from_numpy(w).to(cuda), store.pool,
            store.layer_table(0))
    r1, o1 = grouped_experts(*args, want_routed=True)
    r2, o2 = grouped_experts(*args, want_routed=True)
    assert torch.equal(r1, r2) and torch.equal(o1, o2)
    want, ys = _oracle_grouped(fmt, 0, bf16_bits_to_f32(xb), idx, w)
    _check_rows(_np(r1), want, ys, "small shape")


@pytest.mark.parametrize("kind", ["affine", "fp4"])
def test_moe_prefill_grouped_end_to_end(cuda, kind, prefill_path):
    """Router (bit-exact ids) -> permute -> grouped experts -> combine, small model shape."""
    from cachalot_amd.moe_prefill import moe_prefill_grouped
    from cachalot_amd.storage.index import affine_format, fp4_format

    d, f, E, t, k = 512, 256, 32, 150, 6
    fmt = affine_format(d, f) if kind == "affine" else fp4_format(d, f)
    store = make_store(fmt, n_layers=2, n_experts=E)
    wb, bias = osynth.router_tensors(SEED, 1, E, d)
    xb = osynth.activations(SEED, 600, t, d)
    out, route = moe_prefill_grouped(_bf16(xb, cuda), layer_id=1, gate_weight=_bf16(wb, cuda),
                                     gate_bias=torch.from_numpy(bias).to(cuda), expert_index=None,
                                     expert_store=store, topk=k, route_scale=1.0, score_fn="sigmoid")
    x = bf16_bits_to_f32(xb)
    idx, w, _ = orouter.route(x, bf16_bits_to_f32(wb), bias, topk=k, route_scale=1.0, score=orouter.SCORE_SIGMOID)
    assert np.array_equal(_np(route.indices), idx) and np.array_equal(_np(route.weights), w)
    want, ys = _oracle_grouped(fmt, 1, x, idx, w)
    got = bf16_bits_to_f32(_bits(out))
    assert np.all(np.abs(got - want) <= TOL * np.abs(want).max() + np.sum(bf16_ulp(ys), axis=1) + bf16_ulp(want))


@pytest.mark.parametrize("t,k,d,with_addend,offset", [(37, 6, 4096, True, 0), (5, 8, 4096, False, 0),
                                                      (3, 1, 1024, True, 0), (7, 6, 6, True, 0),
                                                      (9, 6, 4096, True, 2)])
def test_unpermute_combine_bit_exact(cuda, t, k, d, with_addend, offset):
    """cachalot_unpermute_combine against the oracle's route-order sum (moe_prefill_grouped.py:
    526-545): routed fp32 and out bf16 bit for bit -- the 16-byte kernel (D % 8 == 0, aligned)
    and the pair kernel (D = 6; y 4 bytes past a 16-byte boundary)."""
    from cachalot_amd import _lib

    rng = np.random.default_rng(SEED + t * d + k)
    yv = round_bf16(rng.standard_normal((t, k, d)).astype(np.float32) * np.exp2(rng.integers(-8, 8, (t, k, 1))))
    av = round_bf16(rng.standard_normal((t, d)).astype(np.float32)) if with_addend else None
    buf = torch.zeros(t * k * d + offset + 8, dtype=torch.int16, device=cuda)
    y = buf[offset:offset + t * k * d].view(t, k, d)
    y.copy_(torch.from_numpy(f32_to_bf16_bits(yv).view(np.int16)).to(cuda))
    add = torch.from_numpy(f32_to_bf16_bits(av).view(np.int16)).to(cuda) if with_addend else None
    routed = torch.empty((t, d), dtype=torch.float32, device=cuda)
    out = torch.empty((t, d), dtype=torch.int16, device=cuda)
    L = _lib.lib()
    rc = L.cachalot_unpermute_combine(y.data_ptr(), _lib.ptr(add), t, k, d, routed.data_ptr(), out.data_ptr(),
                                      _lib.stream_handle(cuda))
    _lib.check(rc, "unpermute_combine")
    pos = np.arange(t * k, dtype=np.int32).reshape(t, k)
    want_r, want_o = odispatch.combine(yv.reshape(t * k, d), pos, av)
    assert np.array_equal(_np(routed).view(np.uint32), want_r.astype(np.float32).view(np.uint32))
    assert np.array_equal(_np(out).view(np.uint16), f32_to_bf16_bits(want_o))


@pytest.mark.parametrize("kind", ["affine", "fp4"])
def test_one_expert_over_rows(cuda, kind):
    """routed_expert_forward_batched / routed_expert_forward_sgmm (FP4; a resident
    expert in place, and the reference's keyword tensors copied into a scratch slot:
    bit-identical) and affine_expert_forward_batched (2-bit): 150 rows of one expert
    (three 64-row tiles, the last ragged) against oracle swiglu_rows, the rounding
    points of moe_prefill_batched.py:31-61 / expert_affine.py:84-99."""
    from cachalot_amd.expert_rows import (affine_expert_forward_batched, routed_expert_forward_batched,
                                          routed_expert_forward_sgmm)
    from cachalot_amd.storage.index import ExpertEntry, affine_format, fp4_format

    fmt = affine_format(1024, 640) if kind == "affine" else fp4_format(1024, 640)
    store = make_store(fmt, n_layers=1, n_experts=4)
    ex = store.get(ExpertEntry(0, 2))
    rng = np.random.default_rng(19)
    m = 150
    x = round_bf16(rng.standard_normal((m, fmt.d_model)).astype(np.float32))
    w = rng.uniform(0.05, 1.0, m).astype(np.float32)
    xd = _bf16(f32_to_bf16_bits(x), cuda)
    wd = torch.from_numpy(w).to(cuda)
    if kind == "affine":
        got = affine_expert_forward_batched(xd, ex, fmt, wd)
    else:
        got = routed_expert_forward_batched(xd, expert=ex, weights=wd)
        arrays = {n: t.clone() for n, t in ex.as_model_dict().items()}
        copied = routed_expert_forward_sgmm(xd, w1_packed=arrays["w1.weight"], w1_scales=arrays["w1.scale"],
                                            w2_packed=arrays["w2.weight"], w2_scales=arrays["w2.scale"],
                                            w3_packed=arrays["w3.weight"], w3_scales=arrays["w3.scale"], weights=wd)
        assert torch.equal(got, copied)
        with pytest.raises(ValueError):
            routed_expert_forward_batched(xd, w1_packed=arrays["w1.weight"], weights=wd)
    assert got.dtype == torch.float32 and tuple(got.shape) == (m, fmt.d_model)
    mm1, mm3, mm2 = _mats(fmt, 0, 2)
    want = oexperts.swiglu_rows(x, mm1, mm3, mm2, w, 10.0)
    g = _np(got)
    assert np.array_equal(round_bf16(g), g)                 # each value a bf16 cast, as in the reference
    _check_rows(g, want, want[:, None, :], f"one expert, {kind}")
