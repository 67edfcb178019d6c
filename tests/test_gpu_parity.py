"""GPU parity: the HIP library against the oracle on seeded inputs.

Bar (``north_star``): top-k ids and dequantised weights bit-exact; expert
outputs within max relative error 2e-3 (max |got - want| / max |want|, fp32
accumulation, bf16 activations).  The router is additionally bit-exact in its
scores and weights, by the fixed reduction order both sides follow.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from helpers import SEED, bf16_out_ok, bf16_terms_ok, bf16_ulp, fp4_dense, make_store, oracle_tensors, q2_mats, rel_err
from oracle import dispatch as odispatch  # noqa: F401  (kept for the prefill tests)
from oracle import experts as oexperts
from oracle import router as orouter
from oracle import synth as osynth
from oracle.affine2 import dequantize_affine
from oracle.bf16 import bf16_bits_to_f32
from oracle.fp4 import dequantize_fp4_weight

pytestmark = pytest.mark.gpu


TOL = 2e-3


def _np(t):
    return t.detach().cpu().numpy()


def _bf16_np(t):
    return _np(t.contiguous().view(torch.int16)).view(np.uint16)


# ----------------------------------------------------------------- synth ---
def test_fill_matches_oracle_every_kind(cuda):
    from cachalot_amd import synth

    key = synth.stream_key(SEED, 3, 7, 2)
    cases = [(synth.KIND_U32, torch.int32, 1000, 0.0, 0.0, 0, 0), (synth.KIND_U32, torch.int32, 999, 0.0, 0.0, 37, 33),
             (synth.KIND_E8M0, torch.uint8, 777, 119.0, 127.0, 0, 0),
             (synth.KIND_BF16_UNIFORM, torch.int16, 1001, 0.005, 0.045, 0, 0),
             (synth.KIND_BF16_NORMAL, torch.int16, 1003, 0.02, 0.0, 0, 0),
             (synth.KIND_F32_NORMAL, torch.float32, 1005, 1.0, 0.0, 0, 0),
             (synth.KIND_F16_UNIFORM, torch.int16, 1007, 0.005, 0.045, 0, 0),
             (synth.KIND_F16_NORMAL, torch.int16, 1009, 0.02, 0.0, 0, 0)]
    for kind, dt, n, p0, p1, rt, rv in cases:
        for start in (0, 12345):
            t = torch.empty(n, dtype=dt, device=cuda)
            synth.fill(t, kind, key, p0, p1, rt, rv, start=start)
            got = _np(t)
            want = osynth.fill(kind, n, key, p0, p1, rt, rv, start=start)
            assert np.array_equal(got.view(want.dtype), want), (kind, start)


@pytest.mark.parametrize("kind", ["affine", "fp4", "affine_f16"])
def test_whole_expert_bytes_match_oracle(cuda, kind):
    from cachalot_amd.storage.index import affine_format, fp4_format

    fmt = (fp4_format(4096, 2880) if kind == "fp4" else
           affine_format(4096, 2880, scale_dtype="float16" if kind == "affine_f16" else "bfloat16"))
    store = make_store(fmt, n_layers=2, n_experts=4, keys=[(1, 3)])
    slot = store.pool.slot(store.layer_table(1)[3].item())
    want = oracle_tensors(fmt, 1, 3)
    for name, arr in want.items():
        got = _np(slot.arrays[name])
        assert np.array_equal(got, arr.view(np.uint8).reshape(-1)), name


# --------------------------------------------------------------- dequant ---
@pytest.mark.parametrize("as_bf16", [0, 1])
def test_dequant_fp4_bit_exact(cuda, as_bf16):
    from cachalot_amd import _lib

    t = oracle_tensors(__import__("cachalot_amd.storage.index", fromlist=["x"]).fp4_format(4096, 2880), 0, 5)
    packed, scales = t["w2.weight"], t["w2.scale"]      # [4096, 1440], [4096, 90]
    n, k = packed.shape[0], packed.shape[1] * 2
    dp = torch.from_numpy(packed).to(cuda)
    ds = torch.from_numpy(scales).to(cuda)
    out = torch.empty((n, k), dtype=torch.float32, device=cuda)
    rc = _lib.lib().cachalot_dequant_fp4(dp.data_ptr(), ds.data_ptr(), n, k, as_bf16, out.data_ptr(),
                                         _lib.stream_handle(cuda))
    _lib.check(rc)
    got = _np(out)
    want = dequantize_fp4_weight(packed, scales)
    assert np.array_equal(got, want)   # value equality (-0.0 == +0.0)


def test_dequant_fp4_special_scales(cuda):
    from cachalot_amd import _lib

    packed = np.arange(256, dtype=np.uint8).reshape(4, 64)     # every byte value
    scales = np.array([[1, 0, 127, 200], [60, 119, 150, 127], [2, 3, 250, 126], [127, 127, 127, 127]], np.uint8)
    dp, ds = torch.from_numpy(packed).to(cuda), torch.from_numpy(scales).to(cuda)
    for as_bf16 in (0, 1):
        out = torch.empty((4, 128), dtype=torch.float32, device=cuda)
        _lib.check(_lib.lib().cachalot_dequant_fp4(dp.data_ptr(), ds.data_ptr(), 4, 128, as_bf16, out.data_ptr(),
                                                   _lib.stream_handle(cuda)))
        assert np.array_equal(_np(out), dequantize_fp4_weight(packed, scales)), as_bf16


@pytest.mark.parametrize("scale_dtype", ["bfloat16", "float16"])
def test_dequant_q2_bit_exact(cuda, scale_dtype):
    from cachalot_amd import _lib
    from cachalot_amd.storage.index import affine_format

    fmt = affine_format(4096, 2880, scale_dtype=scale_dtype)
    t = oracle_tensors(fmt, 0, 9)
    for proj, k in (("w1", 4096), ("w2", 2880)):
        w, s, b = t[f"{proj}.weight"], t[f"{proj}.scales"], t[f"{proj}.biases"]
        n, row_words = w.shape
        groups = s.shape[1]
        dw = torch.from_numpy(w.view(np.int32)).to(cuda)
        dsc = torch.from_numpy(s.view(np.int16)).to(cuda)
        db = torch.from_numpy(b.view(np.int16)).to(cuda)
        out = torch.empty((n, k), dtype=torch.float32, device=cuda)
        _lib.check(_lib.lib().cachalot_dequant_q2(dw.data_ptr(), dsc.data_ptr(), db.data_ptr(), n, k, row_words,
                                                  groups, 128, _lib.scale_dtype_code(scale_dtype),
                                                  out.data_ptr(), _lib.stream_handle(cuda)))
        want = dequantize_affine(w, s, b, k=k, group=128, scale_dtype=scale_dtype)
        assert np.array_equal(_np(out).view(np.uint32), want.view(np.uint32)), proj


# ---------------------------------------------------------------- router ---
ROUTER_CASES = [
    # T, D, E, k, score, order, temp, scale, norm
    (1, 4096, 384, 6, "sigmoid", "ascending", 1.0, 1.0, True),
    (1, 4096, 384, 6, "sqrt_softplus", "ascending", 1.0, 1.5, True),
    (37, 4096, 384, 6, "sigmoid", "rank", 1.0, 2.5, True),
    (64, 4096, 384, 8, "sqrt_softplus", "ascending", 0.7, 1.5, False),
    (5, 128, 100, 1, "sigmoid", "ascending", 1.0, 1.0, True),
    # 4 <= T < 8: two tokens per wave (the batched decode at B = 4)
    (4, 4096, 384, 6, "sigmoid", "ascending", 1.0, 1.0, True),
    (7, 4096, 384, 6, "sqrt_softplus", "rank", 1.0, 1.5, True),
    (3, 256, 64, 64, "sqrt_softplus", "rank", 1.0, 1.0, True),
    (9, 5120, 384, 6, "sqrt_softplus", "ascending", 1.0, 1.5, True),
    (40, 5120, 384, 6, "sigmoid", "ascending", 1.0, 1.0, True),
    # many tokens: the tiled router kernel (partial token and expert tiles, D/64 = 16 and 80)
    (1030, 1024, 100, 4, "sqrt_softplus", "rank", 1.3, 1.5, True),
    (1024, 5120, 64, 6, "sigmoid", "ascending", 1.0, 1.0, True),
    # the production shape of the tiled router (config 3: E = 384, D = 4096), both score functions
    (1024, 4096, 384, 6, "sqrt_softplus", "ascending", 1.0, 1.5, True),
    (1100, 4096, 384, 6, "sigmoid", "ascending", 1.0, 1.0, True),
]


def _router_inputs(cuda, T, D, E, seed=SEED, layer=0):
    from cachalot_amd import synth

    w, b = synth.router_weights(seed, layer, E, D, cuda)
    x = synth.activations(seed, 11, T, D, cuda)
    return x, w, b


def _check_router(cuda, x, w, b, *, k, score, order, temp, scale, norm, bias_vl=None, mask=None):
    from cachalot_amd.router import route_topk_rows

    idx, wt, sc = route_topk_rows(x, w, b, topk=k, gate_temp=temp, route_scale=scale, norm_topk_prob=norm,
                                  score_fn=score, order=order, bias_vl=bias_vl, image_mask=mask)
    oi, ow, osc = orouter.route(bf16_bits_to_f32(_bf16_np(x)), bf16_bits_to_f32(_bf16_np(w)), _np(b), topk=k,
                                gate_temp=temp, route_scale=scale, norm_topk_prob=norm,
                                score=orouter.SCORE_SIGMOID if score == "sigmoid" else orouter.SCORE_SQRT_SOFTPLUS,
                                order=orouter.ORDER_ASCENDING if order == "ascending" else orouter.ORDER_RANK,
                                bias_vl=None if bias_vl is None else _np(bias_vl),
                                image_mask=None if mask is None else _np(mask), workers=min(16, os.cpu_count() or 1))
    assert np.array_equal(_np(sc).view(np.uint32), osc.view(np.uint32)), "scores"
    assert np.array_equal(_np(idx), oi), "indices"
    assert np.array_equal(_np(wt).view(np.uint32), ow.view(np.uint32)), "weights"
    return idx, wt, sc


@pytest.mark.parametrize("case", ROUTER_CASES, ids=[f"T{c[0]}-D{c[1]}-E{c[2]}-k{c[3]}-{c[4]}-{c[5]}" for c in ROUTER_CASES])
def test_router_bit_exact(cuda, case):
    T, D, E, k, score, order, temp, scale, norm = case
    x, w, b = _router_inputs(cuda, T, D, E)
    _check_router(cuda, x, w, b, k=k, score=score, order=order, temp=temp, scale=scale, norm=norm)


def test_router_ties_follow_order_rule(cuda):
    T, D, E = 4, 256, 96
    x, w, b = _router_inputs(cuda, T, D, E)
    w[1::2] = w[0::2]            # pairs of identical rows -> identical scores
    b.zero_()
    for order in ("ascending", "rank"):
        _check_router(cuda, x, w, b, k=7, score="sigmoid", order=order, temp=1.0, scale=1.0, norm=True)
    # ties between experts e and e + 64 and e + 128 (held by one lane in different key registers)
    x, w, b = _router_inputs(cuda, T, D, 384)
    w[64:128] = w[0:64]
    w[128:192] = w[0:64]
    b.zero_()
    for order in ("ascending", "rank"):
        _check_router(cuda, x, w, b, k=9, score="sqrt_softplus", order=order, temp=1.0, scale=1.0, norm=True)


def test_router_bias_vl_and_mask(cuda):
    from cachalot_amd import synth

    T, D, E = 16, 4096, 384
    x, w, b = _router_inputs(cuda, T, D, E)
    _, bvl = synth.router_weights(SEED + 1, 0, E, D, cuda, b_sigma=0.3)
    mask = torch.tensor([i % 3 == 0 for i in range(T)], device=cuda)
    _check_router(cuda, x, w, b, k=6, score="sqrt_softplus", order="ascending", temp=1.0, scale=1.5, norm=True,
                  bias_vl=bvl, mask=mask)


def test_router_batch_equals_single(cuda):
    from cachalot_amd.router import route_topk, route_topk_batch

    x, w, b = _router_inputs(cuda, 12, 4096, 384)
    batch = route_topk_batch(x, w, b, topk=6)
    for t in range(12):
        one = route_topk(x[t], w, b, topk=6)
        assert torch.equal(one.indices, batch.indices[t]) and torch.equal(one.weights, batch.weights[t])
        assert torch.equal(one.scores, batch.scores[t])


def test_router_errors(cuda):
    from cachalot_amd.router import route_topk, route_topk_fused, route_topk_rows

    x, w, b = _router_inputs(cuda, 2, 256, 16)
    with pytest.raises(ValueError):
        route_topk(x, w, b)
    with pytest.raises(ValueError):
        route_topk(x[0], w, b, topk=17)
    with pytest.raises(ValueError):
        route_topk_fused(x[0], w, b, norm_topk_prob=False)
    with pytest.raises(ValueError):
        route_topk_rows(x, w, b, bias_vl=b)
    with pytest.raises(ValueError):
        route_topk(x[0, :128], w, b)


# ---------------------------------------------------------------- decode ---
def _decode_case(cuda, fmt, store, layer, x_np_bits, idx, wts, addend_bits=None):
    from cachalot_amd.moe_decode import decode_experts

    x = torch.from_numpy(x_np_bits.view(np.int16)).to(cuda).view(torch.bfloat16)
    addend = None if addend_bits is None else torch.from_numpy(addend_bits.view(np.int16)).to(cuda).view(torch.bfloat16)
    routed, out = decode_experts(x, store.pool, store.layer_table(layer), torch.tensor(idx, dtype=torch.int32, device=cuda),
                                 torch.tensor(wts, dtype=torch.float32, device=cuda), swiglu_limit=10.0, addend=addend)
    return _np(routed), bf16_bits_to_f32(_bf16_np(out))


def _oracle_q2(fmt, layer, x, idx, wts, addend=None, drop=(), terms=False):
    mats = [q2_mats(fmt, oracle_tensors(fmt, layer, e)) for e in idx]
    keep = [i for i, e in enumerate(idx) if e not in drop]
    return oexperts.affine_decode(x, [mats[i] for i in keep], np.asarray(wts, np.float32)[keep], 10.0, addend,
                                  terms=terms)


def _assert_q2(routed, want, ys, what):
    """Bar: 2e-3 of max|want|, plus one bf16 ulp per expert term (the per-expert cast)."""
    err = rel_err(routed, want)
    assert bf16_terms_ok(routed, want, ys, TOL), (what, err)
    # flips at the cast are rare: the plain bar holds on at least 99 % of elements
    frac = np.mean(np.abs(np.asarray(routed, np.float64) - want) > TOL * np.abs(want).max())
    assert frac <= 0.01, (what, frac)


@pytest.mark.parametrize("shape", [(4096, 2880), (5120, 2304)])
def test_decode_q2_parity(cuda, shape, q2_path):
    from cachalot_amd.storage.index import affine_format

    D, F = shape
    fmt = affine_format(D, F)
    rng = np.random.default_rng(1)
    tokens = []
    keys = set()
    for t in range(3):
        idx = rng.choice(384, size=6, replace=False).tolist()
        w = rng.dirichlet(np.ones(6)).astype(np.float32)
        tokens.append((idx, w))
        keys.update((0, e) for e in idx)
    store = make_store(fmt, n_layers=1, n_experts=384, keys=sorted(keys), n_slots=len(keys))
    for t, (idx, w) in enumerate(tokens):
        xb = osynth.activations(SEED, 100 + t, 1, D)[0]
        ab = osynth.activations(SEED, 200 + t, 1, D)[0]
        x = bf16_bits_to_f32(xb)
        routed, out = _decode_case(cuda, fmt, store, 0, xb, idx, w, ab)
        a = bf16_bits_to_f32(ab)
        want_r, _, ys = _oracle_q2(fmt, 0, x, idx, w, a, terms=True)
        _assert_q2(routed, want_r, ys, t)
        assert bf16_terms_ok(out, want_r + a, np.concatenate([ys, (want_r + a)[None]]), TOL), t


def test_decode_q2_k_range_and_missing_slot(cuda, q2_path):
    from cachalot_amd.storage.index import affine_format

    fmt = affine_format(4096, 2880)
    idx_all = [5, 77, 300, 12, 250, 199, 3, 381]
    store = make_store(fmt, n_layers=1, n_experts=384, keys=[(0, e) for e in idx_all], n_slots=8)
    xb = osynth.activations(SEED, 7, 1, 4096)[0]
    x = bf16_bits_to_f32(xb)
    for k in (1, 2, 8):
        idx = idx_all[:k]
        w = np.linspace(0.1, 1.0, k).astype(np.float32)
        routed, _ = _decode_case(cuda, fmt, store, 0, xb, idx, w)
        want, _, ys = _oracle_q2(fmt, 0, x, idx, w, terms=True)
        _assert_q2(routed, want, ys, k)
    # expert 77 loses its slot: it contributes zero rows
    store.track_slots()[0, 77] = -1
    idx = idx_all[:6]
    w = np.full(6, 1 / 6, np.float32)
    routed, _ = _decode_case(cuda, fmt, store, 0, xb, idx, w)
    want, _, ys = _oracle_q2(fmt, 0, x, idx, w, drop=(77,), terms=True)
    _assert_q2(routed, want, ys, "missing slot")


def test_decode_fp4_parity(cuda):
    from cachalot_amd.storage.index import fp4_format

    fmt = fp4_format(4096, 2880)
    rng = np.random.default_rng(2)
    idx = rng.choice(384, size=6, replace=False).tolist()
    w = rng.dirichlet(np.ones(6)).astype(np.float32)
    store = make_store(fmt, n_layers=1, n_experts=384, keys=[(0, e) for e in idx], n_slots=6)
    xb = osynth.activations(SEED, 5, 1, 4096)[0]
    routed, out = _decode_case(cuda, fmt, store, 0, xb, idx, w)
    dense = [fp4_dense(oracle_tensors(fmt, 0, e)) for e in idx]
    want = oexperts.fp4_decode(bf16_bits_to_f32(xb), dense, w, 10.0)
    assert rel_err(routed, want) <= TOL
    assert rel_err(routed, want) <= 1e-5     # no bf16 rounding point on this path: fp32-level agreement


def test_moe_layer_forward_end_to_end(cuda, q2_path):
    """Router ids bit-exact and the layer output within the bar, through the reference-shaped entry."""
    from cachalot_amd import synth
    from cachalot_amd.moe_layer import moe_layer_forward
    from cachalot_amd.storage.index import affine_format

    fmt = affine_format(4096, 2880)
    store = make_store(fmt, n_layers=2, n_experts=384)
    for layer in (0, 1):
        w, b = synth.router_weights(SEED, layer, 384, 4096, cuda)
        x = synth.activations(SEED, 40 + layer, 1, 4096, cuda)[0]
        out, route = moe_layer_forward(x, layer_id=layer, gate_weight=w, gate_bias=b, expert_index=None,
                                       expert_store=store, topk=6, route_scale=1.0, score_fn="sigmoid")
        xf = bf16_bits_to_f32(_bf16_np(x))
        oi, ow, _ = orouter.route(xf[None], bf16_bits_to_f32(_bf16_np(w)), _np(b), topk=6, route_scale=1.0,
                                  score=orouter.SCORE_SIGMOID)
        assert np.array_equal(_np(route.indices), oi[0])
        want, _, ys = _oracle_q2(fmt, layer, xf, oi[0].tolist(), ow[0], terms=True)
        assert out.dtype == torch.bfloat16
        assert bf16_terms_ok(bf16_bits_to_f32(_bf16_np(out)), want, np.concatenate([ys, want[None]]), TOL)


@pytest.mark.parametrize("kind,score", [("affine", "sqrt_softplus"), ("fp4", "sqrt_softplus"), ("fp4", "sigmoid")])
def test_layer_decode_fused_routing_and_repeat_calls(cuda, kind, score, q2_path):
    """Device-routed decode (scores -> top-k in the gate/up prologue -> down with the
    counter-based combine): ids bit-exact, outputs within the bar, and repeated calls
    on one workspace (counters reset by the kernels) give identical results.  The
    FP4 / sigmoid case is config 0 as BASELINE states it (sigmoid scores, top-6
    renormalised, route scale 1)."""
    from cachalot_amd import synth
    from cachalot_amd.moe_decode import moe_layer_decode
    from cachalot_amd.storage.index import affine_format, fp4_format

    fmt = affine_format(4096, 2880) if kind == "affine" else fp4_format(4096, 2880)
    store = make_store(fmt, n_layers=1, n_experts=384)
    w, b = synth.router_weights(SEED, 0, 384, 4096, cuda)
    rs = 1.5 if score == "sqrt_softplus" else 1.0
    sfn = orouter.SCORE_SQRT_SOFTPLUS if score == "sqrt_softplus" else orouter.SCORE_SIGMOID
    first = None
    for t in range(3):
        x = synth.activations(SEED, 60 + t, 1, 4096, cuda)[0]
        routed, out, route = moe_layer_decode(x, w, b, store.pool, store.layer_table(0), topk=6, route_scale=rs,
                                              score_fn=score, addend=x, want_routed=True)
        xf = bf16_bits_to_f32(_bf16_np(x))
        oi, ow, osc = orouter.route(xf[None], bf16_bits_to_f32(_bf16_np(w)), _np(b), topk=6, route_scale=rs,
                                    score=sfn)
        assert np.array_equal(_np(route.indices), oi[0])
        assert np.array_equal(_np(route.weights).view(np.uint32), ow[0].view(np.uint32))
        assert np.array_equal(_np(route.scores).view(np.uint32), osc[0].view(np.uint32))
        if kind == "affine":
            want, _, ys = _oracle_q2(fmt, 0, xf, oi[0].tolist(), ow[0], terms=True)
            _assert_q2(_np(routed), want, ys, t)
            assert bf16_terms_ok(bf16_bits_to_f32(_bf16_np(out)), want + xf, np.concatenate([ys, (want + xf)[None]]),
                                 TOL)
        else:
            dense = [fp4_dense(oracle_tensors(fmt, 0, int(e))) for e in oi[0]]
            want = oexperts.fp4_decode(xf, dense, ow[0], 10.0)
            assert rel_err(_np(routed), want) <= TOL
            assert bf16_out_ok(bf16_bits_to_f32(_bf16_np(out)), want + xf, TOL)
        if first is None:
            first = (x, routed.clone(), out.clone())
    x0, r0, o0 = first
    for _ in range(3):
        r, o, _ = moe_layer_decode(x0, w, b, store.pool, store.layer_table(0), topk=6, route_scale=rs, addend=x0,
                                   score_fn=score, want_routed=True)
        assert torch.equal(r, r0) and torch.equal(o, o0)


def test_layer_decode_graph_replays_match_eager(cuda, q2_path):
    """A captured chain of decode steps replays identically, several times, with
    eager work and synchronisation between replays."""
    from cachalot_amd import synth
    from cachalot_amd.moe_decode import moe_layer_decode
    from cachalot_amd.storage.index import affine_format

    fmt = affine_format(4096, 2880)
    store = make_store(fmt, n_layers=2, n_experts=384)
    gates = [synth.router_weights(SEED, la, 384, 4096, cuda) for la in range(2)]
    x0 = synth.activations(SEED, 70, 1, 4096, cuda)[0]

    def chain(x):
        for s in range(4):
            w, b = gates[s % 2]
            _, x, _ = moe_layer_decode(x, w, b, store.pool, store.layer_table(s % 2), topk=6, route_scale=1.0,
                                       score_fn="sigmoid", addend=x)
        return x

    eager = chain(x0)
    torch.cuda.synchronize()
    xbuf = x0.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = chain(xbuf)
    for _ in range(3):
        xbuf.copy_(x0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
        _ = chain(x0)                       # eager work between replays
        torch.cuda.synchronize()


def test_store_get_many_loads_and_evicts(cuda):
    from cachalot_amd.storage.index import ExpertEntry, affine_format

    fmt = affine_format(256, 128)
    store = make_store(fmt, n_layers=1, n_experts=16, keys=[], n_slots=3, loader=True)
    got = store.get_many([ExpertEntry(0, 1), ExpertEntry(0, 2)])
    assert [g.expert for g in got] == [1, 2] and store.stats.misses == 2
    store.get_many([ExpertEntry(0, 3), ExpertEntry(0, 1)])
    store.get_many([ExpertEntry(0, 4)])          # evicts expert 2 (least recently used)
    table = store.track_slots().cpu().numpy()[0]
    assert table[2] == -1 and table[4] >= 0 and table[1] >= 0
    slot = store.pool.slot(int(table[4]))
    want = oracle_tensors(fmt, 0, 4)
    assert np.array_equal(_np(slot.arrays["w3.biases"]), want["w3.biases"].view(np.uint8).reshape(-1))
    nl = make_store(fmt, n_layers=1, n_experts=16, keys=[], n_slots=2)
    with pytest.raises(KeyError):
        nl.get_many([ExpertEntry(0, 1)])
