"""GPU parity at the BASELINE workloads' real shapes, with the per-expert terms
checked one by one.

The reference rounds every expert's output y_e to bf16 and sums the route slots
in order in fp32 (``expert_affine.py:81,149-151``, ``moe_prefill_grouped.py:
526-545``).  So the checks here are, per output element:

* each GPU term y_e lies within half a bf16 step (its own cast) plus
  ``TERM_TOL`` * max|y| of the oracle's unrounded value of the same product
  (``helpers.term_flips``); terms equal to the oracle's cast, one step off
  (boundary flips) and further off (moved by a flip at g, u or h) are counted;
* routed = 0 + y_0 + ... + y_{k-1} over the GPU's own terms, bit for bit;
* out = bf16(routed + addend), bit for bit;
* the layer output against the oracle's own bf16 output, in bf16 ulps
  (reported, and bounded by the flips).

Workloads: config 1's decode (matrix-core and bf16-MFMA paths, bf16 and fp16
scales), config 2 with a router-driven union, config 3's 4096-token Zipf prefill on the FP4 bank (tiled router at
E = 384, experts spanning many 128-row tiles), config 4's chained decode over
layers whose slots lie beyond 2^32 bytes, and the grouped path with experts of
several tiles and with out-of-range route ids.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from helpers import (SEED, bf16_ulp, bf16_ulp_dist, fp4_dense, make_store, oracle_tensors, q2_mats, report, route_order_sum,
                     term_flips)
from oracle import dispatch as odispatch
from oracle import experts as oexperts
from oracle import router as orouter
from oracle import synth as osynth
from oracle.bf16 import bf16_bits_to_f32, round_bf16

pytestmark = pytest.mark.gpu
# Expert-output error beyond the output's own bf16 cast, in units of max|y|.
# A flip at g, u or h (a value one bf16 step away because a different fp32 order
# crossed a rounding boundary, as MLX's order would) moves y_d by w2[d, j] times
# one step of h_j, measured up to 3e-4 of max|y| on the FP4 bank; the bar is
# half the north_star bar (2e-3) so that a few such flips pass and a one-step
# error on the largest outputs (3.9e-3) does not.
TERM_TOL = 1e-3
WORKERS = min(16, os.cpu_count() or 1)


def _np(t):
    return t.detach().cpu().numpy()


def _bits(t):
    return _np(t.contiguous().view(torch.int16)).view(np.uint16)


def _f32(t):
    return bf16_bits_to_f32(_bits(t))


def _bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)


def _q2_expert_raw(fmt, layer, e, x_rows, w_rows):
    mm1, mm3, mm2 = q2_mats(fmt, oracle_tensors(fmt, layer, e))
    return oexperts.swiglu_rows(x_rows, mm1, mm3, mm2, w_rows, 10.0, raw=True)


def _fp4_expert_raw(fmt, layer, e, x_rows, w_rows):
    w1, w3, w2 = (np.asarray(w, np.float64) for w in fp4_dense(oracle_tensors(fmt, layer, e)))
    return oexperts.swiglu_rows(x_rows, lambda v: v @ w1.T, lambda v: v @ w3.T, lambda v: v @ w2.T, w_rows, 10.0,
                                raw=True)


# ------------------------------------------------------------ decode (B = 1) ---
def _decode_terms(cuda, store, layer, x, idx, w):
    """GPU y_e of each routed expert: one-expert decode calls (routed = 0 + y_e)."""
    from cachalot_amd.moe_decode import decode_experts

    terms = []
    for e, we in zip(idx, w):
        r, _ = decode_experts(x, store.pool, store.layer_table(layer), torch.tensor([int(e)], dtype=torch.int32,
                                                                                     device=cuda),
                              torch.tensor([float(we)], dtype=torch.float32, device=cuda), want_out=False)
        terms.append(_np(r))
    return np.stack(terms)


def _check_decode(what, fmt, layer, xf, idx, w, routed, out, terms, addend=None):
    """routed / out from a k-expert call; terms from one-expert calls on the same x."""
    want_r, want_out, ys, raws = oexperts.affine_decode(xf, [q2_mats(fmt, oracle_tensors(fmt, layer, int(e)))
                                                             for e in idx], np.asarray(w, np.float32), 10.0, addend,
                                                        terms=True, raw=True)
    st = term_flips(terms, raws, TERM_TOL, what)
    assert np.array_equal(routed.view(np.uint32), route_order_sum(terms).view(np.uint32)), (what, "route-order sum")
    total = routed if addend is None else routed + np.asarray(addend, np.float32)
    assert np.array_equal(out, round_bf16(total)), (what, "output cast")
    ulps = bf16_ulp_dist(out, want_out)
    rel = float(np.abs(routed.astype(np.float64) - want_r).max() / np.abs(want_r).max())
    report(what, terms=st["n"], exact=st["exact"], flips=st["flips"], moved=st["moved"], term_err=f"{st['err']:.2e}",
           out_ulps_max=int(ulps.max()), out_ulps_nonzero=int((ulps > 0).sum()), routed_rel_err=f"{rel:.2e}")
    return st


@pytest.mark.parametrize("shape,scale_dtype", [((4096, 2880), "bfloat16"), ((5120, 2304), "bfloat16"),
                                               ((4096, 2880), "float16")])
def test_decode_q2_terms_exact_up_to_flips(cuda, shape, scale_dtype, q2_path):
    """Config 1 decode: the k-expert call's routed vector is the route-order fp32
    sum of its own per-expert terms (bit for bit), every term is the oracle's
    bf16 cast up to counted boundary flips, and out = bf16(routed + addend).
    Config 1 as BASELINE states it ("fp16 scale and bias") is the float16 case;
    the reference's own bank stores bf16."""
    from cachalot_amd.moe_decode import decode_experts
    from cachalot_amd.storage.index import affine_format

    D, F = shape
    fmt = affine_format(D, F, scale_dtype=scale_dtype)
    rng = np.random.default_rng(21)
    toks = [(rng.choice(384, size=6, replace=False).tolist(), rng.dirichlet(np.ones(6)).astype(np.float32))
            for _ in range(3)]
    keys = sorted({(0, e) for idx, _ in toks for e in idx})
    store = make_store(fmt, n_layers=1, n_experts=384, keys=keys, n_slots=len(keys))
    for t, (idx, w) in enumerate(toks):
        xb = osynth.activations(SEED, 900 + t, 1, D)[0]
        ab = osynth.activations(SEED, 950 + t, 1, D)[0]
        x, a = _bf16(xb, cuda), _bf16(ab, cuda)
        routed, out = decode_experts(x, store.pool, store.layer_table(0), torch.tensor(idx, dtype=torch.int32,
                                                                                       device=cuda),
                                     torch.tensor(w, device=cuda), addend=a)
        terms = _decode_terms(cuda, store, 0, x, idx, w)
        _check_decode(f"decode {q2_path} {D}x{F} {scale_dtype} token {t}", fmt, 0, bf16_bits_to_f32(xb), idx, w, _np(routed),
                      _f32(out), terms, bf16_bits_to_f32(ab))


def test_config4_chain_beyond_4gib(cuda, q2_path):
    """Config 4's chained decode (device routing, residual carried as the addend)
    over three resident layers whose slot records lie at 3.9-15.4 GB of one pool:
    each layer's ids are bit-exact and its output is checked against the oracle
    fed with the GPU's own input for that layer."""
    from cachalot_amd import synth
    from cachalot_amd.moe_decode import moe_layer_decode
    from cachalot_amd.storage.index import affine_format

    fmt = affine_format(4096, 2880)
    store = make_store(fmt, n_layers=4, n_experts=384)          # bulk layout: slot = layer * 384 + expert
    table = store.track_slots()
    assert int(table[3].min()) * store.pool.layout().record_bytes > 2 ** 32
    gates = {la: synth.router_weights(SEED, la, 384, 4096, cuda) for la in (1, 2, 3)}
    x = synth.activations(SEED, 77, 1, 4096, cuda)[0]
    for step, la in enumerate((1, 2, 3, 2)):
        w, b = gates[la]
        routed, out, route = moe_layer_decode(x, w, b, store.pool, table[la], topk=6, route_scale=1.0,
                                              score_fn="sigmoid", addend=x, want_routed=True)
        xf = _f32(x)
        oi, ow, _ = orouter.route(xf[None], _f32(w), _np(b), topk=6, route_scale=1.0, score=orouter.SCORE_SIGMOID)
        assert np.array_equal(_np(route.indices), oi[0]), step
        assert np.array_equal(_np(route.weights).view(np.uint32), ow[0].view(np.uint32)), step
        terms = _decode_terms(cuda, store, la, x, oi[0], ow[0])
        _check_decode(f"config4 chain {q2_path} step {step} layer {la}", fmt, la, xf, oi[0], ow[0], _np(routed),
                      _f32(out), terms, xf)
        x = out


# ------------------------------------------------------------------- grouped ---
def _grouped_check(what, fmt, layer, xf, idx, w, routed, out, y, n_experts, rows_of=None, addend=None):
    """y [T, k, D] terms: the oracle per expert (all rows, or the rows `rows_of[e]`
    selects), the combine over every token bit for bit."""
    raw_fn = _fp4_expert_raw if fmt.kind == "fp4" else _q2_expert_raw
    if rows_of is None:
        experts = np.unique(idx[(idx >= 0) & (idx < n_experts)])
    else:
        experts = np.asarray(sorted(rows_of))
    tot = {"exact": 0, "flips": 0, "moved": 0, "n": 0}
    worst = 0.0
    for e in experts:
        rows = np.argwhere(idx == e)
        if rows_of is not None:
            rows = rows[rows_of[int(e)]]
        _, raw = raw_fn(fmt, layer, int(e), xf[rows[:, 0]], w[rows[:, 0], rows[:, 1]])
        st = term_flips(y[rows[:, 0], rows[:, 1]], raw, TERM_TOL, f"{what} expert {e}")
        for key in tot:
            tot[key] += st[key]
        worst = max(worst, st["err"])
    want_sum = route_order_sum(np.moveaxis(y, 1, 0))
    assert np.array_equal(routed.view(np.uint32), want_sum.view(np.uint32)), (what, "route-order sum")
    total = routed if addend is None else routed + addend
    assert np.array_equal(out, round_bf16(total)), (what, "output cast")
    report(what, experts=len(experts), terms=tot["n"], exact=tot["exact"], flips=tot["flips"], moved=tot["moved"],
           term_err=f"{worst:.2e}")


@pytest.mark.parametrize("kind", ["fp4", "affine"])
def test_grouped_experts_span_many_tiles(cuda, kind, prefill_path):
    """One expert with 3 x 128 + 37 rows and several with more than 128 (ragged
    last tiles), T = 600, k = 2, E = 8, at the layer's shape."""
    from cachalot_amd.moe_prefill import grouped_experts
    from cachalot_amd.storage.index import affine_format, fp4_format

    fmt = affine_format(4096, 2880) if kind == "affine" else fp4_format(4096, 2880)
    E, t, k = 8, 600, 2
    store = make_store(fmt, n_layers=1, n_experts=E)
    rng = np.random.default_rng(31)
    idx = np.zeros((t, k), np.int32)
    idx[:421, 0] = 0                                       # expert 0: 421 rows = 3 x 128 + 37
    idx[421:, 0] = rng.integers(1, 4, size=t - 421)
    idx[:, 1] = rng.integers(4, 8, size=t)                 # experts 4..7: ~150 rows each
    w = rng.dirichlet(np.ones(k), size=t).astype(np.float32)
    counts = np.bincount(idx.reshape(-1), minlength=E)
    assert counts[0] == 421 and (counts[4:] > 128).all()
    xb = osynth.activations(SEED, 310, t, 4096)
    ab = osynth.activations(SEED, 311, t, 4096)
    routed, out, y = grouped_experts(_bf16(xb, cuda), torch.from_numpy(idx).to(cuda), torch.from_numpy(w).to(cuda),
                                     store.pool, store.layer_table(0), addend=_bf16(ab, cuda), want_routed=True,
                                     want_terms=True)
    _grouped_check(f"grouped many tiles {kind} {prefill_path}", fmt, 0, bf16_bits_to_f32(xb), idx, w, _np(routed), _f32(out),
                   _f32(y), E, addend=bf16_bits_to_f32(ab))


@pytest.mark.parametrize("t", [5, 300])
def test_grouped_out_of_range_ids_contribute_zero(cuda, t):
    """Route ids outside [0, E) are dropped routes: zero terms, the rest exact
    (the batched matrix-core path at T = 5, 64-row tiles at T = 300)."""
    from cachalot_amd.moe_prefill import grouped_experts, permute
    from cachalot_amd.storage.index import affine_format

    fmt = affine_format(4096, 2880)
    E, k = 16, 6
    store = make_store(fmt, n_layers=1, n_experts=E)
    rng = np.random.default_rng(41 + t)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(t)]).astype(np.int32)
    idx[0, 2] = -1
    idx[t - 1, 5] = E + 5
    idx[t // 2, 0] = 1 << 30
    w = rng.dirichlet(np.ones(k), size=t).astype(np.float32)
    di, dw = torch.from_numpy(idx).to(cuda), torch.from_numpy(w).to(cuda)
    offs, tok, slot, rw = permute(di, dw, E)
    p = odispatch.permute(idx, E)
    assert np.array_equal(_np(offs), p["offsets"])
    assert np.array_equal(_np(tok), p["token"]) and np.array_equal(_np(slot), p["slot"])
    assert int(_np(offs)[E]) == t * k - 3 and (_np(rw)[t * k - 3:] == 0).all()
    xb = osynth.activations(SEED, 320 + t, t, 4096)
    for _ in range(2):                                     # y reused from a previous call must not leak in
        routed, out, y = grouped_experts(_bf16(xb, cuda), di, dw, store.pool, store.layer_table(0), want_routed=True,
                                         want_terms=True)
        yf = _f32(y)
        assert not yf[0, 2].any() and not yf[t - 1, 5].any() and not yf[t // 2, 0].any()
        _grouped_check(f"grouped dropped ids T={t}", fmt, 0, bf16_bits_to_f32(xb), idx, w, _np(routed), _f32(out),
                       yf, E)


def test_config3_prefill_workload(cuda, prefill_path):
    """Config 3 itself: 4096 tokens, D 4096, F 2880, 384 FP4 experts, the Zipf
    router bias.  Router ids, weights and scores bit-exact for all 4096 tokens
    (the tiled router kernel at E = 384); the three heaviest experts' rows
    (hundreds to thousands each: many 128-row tiles, many XCD groups) and every
    route of 16 random tokens against the oracle; the combine of all tokens bit
    for bit over the GPU's terms."""
    from cachalot_amd import synth
    from cachalot_amd.moe_prefill import grouped_experts
    from cachalot_amd.router import route_topk_rows
    from cachalot_amd.storage.index import fp4_format

    D, F, E, K, T = 4096, 2880, 384, 6, 4096
    fmt = fp4_format(D, F)
    store = make_store(fmt, n_layers=1, n_experts=E)
    w, b = synth.router_weights(SEED + 3, 0, E, D, cuda)
    b = b + torch.tensor(synth.zipf_bias(E, seed=SEED), dtype=torch.float32, device=cuda)
    x = synth.activations(SEED + 3, 0, T, D, cuda)
    idx, wt, sc = route_topk_rows(x, w, b, topk=K, route_scale=1.0, score_fn="sigmoid")
    xf = _f32(x)
    oi, ow, osc = orouter.route(xf, _f32(w), _np(b), topk=K, route_scale=1.0, score=orouter.SCORE_SIGMOID,
                                workers=WORKERS)
    assert np.array_equal(_np(sc).view(np.uint32), osc.view(np.uint32)), "scores"
    assert np.array_equal(_np(idx), oi), "indices"
    assert np.array_equal(_np(wt).view(np.uint32), ow.view(np.uint32)), "weights"
    counts = np.bincount(oi.reshape(-1), minlength=E)
    heavy = np.argsort(counts, kind="stable")[-3:]
    assert counts[heavy].min() > 256, counts[heavy]
    routed, out, y = grouped_experts(x, idx, wt, store.pool, store.layer_table(0), want_routed=True, want_terms=True)
    rng = np.random.default_rng(5)
    toks = rng.choice(T, size=16, replace=False)
    rows_of = {int(e): slice(None) for e in heavy}
    sample = {}
    for tk in toks:
        for s in range(K):
            sample.setdefault(int(oi[tk, s]), []).append((tk, s))
    yf = _f32(y)
    # every route of the sampled tokens: per expert, the rows of those (token, slot) pairs
    for e, pairs in sample.items():
        if e in rows_of:
            continue
        want = set(pairs)
        rows = np.argwhere(oi == e)
        rows_of[e] = np.asarray([i for i, (a, c) in enumerate(rows.tolist()) if (a, c) in want])
    _grouped_check(f"config3 prefill fp4 {prefill_path}", fmt, 0, xf, oi, ow, _np(routed), _f32(out), yf, E,
                   rows_of=rows_of)
    report(f"config3 prefill fp4 {prefill_path}", rows_per_heavy_expert=counts[heavy].tolist(), max_rows=int(counts.max()),
           experts_touched=int((counts > 0).sum()))


@pytest.mark.parametrize("B", [16, 32])
def test_config2_batched_decode_router_union(cuda, B):
    """Config 2 itself: B tokens through the seeded router over 384 experts (the
    union of their routes, ~85 / ~150 experts, about 1.3-1.6 rows each), then the
    grouped 2-bit decode over that union.  Ids and weights bit-exact for every
    token; every route of 8 sampled experts against the oracle term by term; the
    combine of all B tokens bit for bit over the GPU's terms."""
    from cachalot_amd import synth
    from cachalot_amd.moe_prefill import grouped_experts
    from cachalot_amd.router import route_topk_rows
    from cachalot_amd.storage.index import affine_format

    D, F, E, K = 4096, 2880, 384, 6
    fmt = affine_format(D, F)
    store = make_store(fmt, n_layers=1, n_experts=E)
    w, b = synth.router_weights(SEED, 0, E, D, cuda)
    x = synth.activations(SEED, 2000 + B, B, D, cuda)
    a = synth.activations(SEED, 2100 + B, B, D, cuda)
    idx, wt, _ = route_topk_rows(x, w, b, topk=K, route_scale=1.0, score_fn="sigmoid")
    xf = _f32(x)
    oi, ow, _ = orouter.route(xf, _f32(w), _np(b), topk=K, route_scale=1.0, score=orouter.SCORE_SIGMOID)
    assert np.array_equal(_np(idx), oi) and np.array_equal(_np(wt).view(np.uint32), ow.view(np.uint32))
    union = np.unique(oi)
    assert len(union) > 3 * B // 2, len(union)
    routed, out, y = grouped_experts(x, idx, wt, store.pool, store.layer_table(0), addend=a, want_routed=True,
                                     want_terms=True)
    rng = np.random.default_rng(B)
    sample = rng.choice(union, size=8, replace=False)
    _grouped_check(f"config2 B={B} union {len(union)}", fmt, 0, xf, oi, ow, _np(routed), _f32(out), _f32(y), E,
                   rows_of={int(e): slice(None) for e in sample}, addend=_f32(a))


def test_config4_full_residency_chain(cuda):
    """Config 4 at full residency: 40 x 384 2-bit experts (154 GB) in HBM, one
    token through all 40 layers (device routing, residual as the addend).  Ids
    bit-exact at every layer against the oracle router fed the GPU's own input;
    two sampled layers' outputs term by term; a captured 40-layer graph replays
    identically to the eager chain, three times, with eager work between."""
    from cachalot_amd import synth
    from cachalot_amd.moe_decode import moe_layer_decode
    from cachalot_amd.storage.index import affine_format

    L, E = 40, 384
    fmt = affine_format(4096, 2880)
    store = make_store(fmt, n_layers=L, n_experts=E)
    table = store.track_slots()
    gates = [synth.router_weights(SEED, la, E, 4096, cuda) for la in range(L)]
    x0 = synth.activations(SEED, 4040, 1, 4096, cuda)[0]

    def chain(x, record=None):
        for la in range(L):
            w, bias = gates[la]
            routed, out, route = moe_layer_decode(x, w, bias, store.pool, table[la], topk=6, route_scale=1.0,
                                                  score_fn="sigmoid", addend=x, want_routed=True)
            if record is not None:
                record.append((x, routed, out, route))
            x = out
        return x

    steps = []
    eager = chain(x0, steps)
    torch.cuda.synchronize()
    for la, (x, routed, out, route) in enumerate(steps):
        w, bias = gates[la]
        xf = _f32(x)
        oi, ow, _ = orouter.route(xf[None], _f32(w), _np(bias), topk=6, route_scale=1.0, score=orouter.SCORE_SIGMOID)
        assert np.array_equal(_np(route.indices), oi[0]), la
        assert np.array_equal(_np(route.weights).view(np.uint32), ow[0].view(np.uint32)), la
        if la in (0, 39):
            terms = _decode_terms(cuda, store, la, x, oi[0], ow[0])
            _check_decode(f"config4 full residency layer {la}", fmt, la, xf, oi[0], ow[0], _np(routed), _f32(out),
                          terms, xf)
    xbuf = x0.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = chain(xbuf)
    for _ in range(3):
        xbuf.copy_(x0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
        _ = chain(x0)
        torch.cuda.synchronize()


# ------------------------------------------------------- partial residency ---
def _partial_layer(cuda, resident_of):
    """A 2-bit layer whose store holds only some experts (loader for misses), its router,
    one token, and the router's own ids / weights / scores."""
    from cachalot_amd import synth
    from cachalot_amd.router import route_topk_fused
    from cachalot_amd.storage.index import affine_format

    fmt = affine_format(4096, 2880)
    w, b = synth.router_weights(SEED, 0, 384, 4096, cuda)
    x = synth.activations(SEED, 808, 1, 4096, cuda)[0]
    r = route_topk_fused(x, w, b, topk=6, route_scale=1.0, score_fn="sigmoid")
    ids, wts, scores = [int(e) for e in r.indices.tolist()], r.weights.tolist(), _np(r.scores)
    keys = [(0, e) for e in resident_of(ids, scores + _np(b))]
    store = make_store(fmt, n_layers=1, n_experts=384, keys=keys, n_slots=16, loader=True)
    return fmt, store, x, w, b, ids, wts


def _layer_out(x, w, b, store):
    from cachalot_amd.moe_layer import moe_layer_forward

    out, route = moe_layer_forward(x, layer_id=0, gate_weight=w, gate_bias=b, expert_index=None, expert_store=store,
                                   topk=6, route_scale=1.0, score_fn="sigmoid")
    return _f32(out), route


def _oracle_out(fmt, x, ids, wts):
    _, want_out, ys = oexperts.affine_decode(_f32(x), [q2_mats(fmt, oracle_tensors(fmt, 0, e)) for e in ids],
                                             np.asarray(wts, np.float32), 10.0, terms=True)
    return want_out, ys


def test_decode_miss_budget_drops_and_rescales(cuda):
    """decode_miss_budget = 2 with two of six routed experts resident: the two strongest
    misses load, the other two are dropped and the kept weights rescaled to the
    layer's routing mass (moe_layer_metal.py:286-310)."""
    from cachalot_amd.decode_substitution import rescale_kept

    fmt, store, x, w, b, ids, wts = _partial_layer(cuda, lambda ids, sel: ids[:2])
    store.decode_miss_budget = 2
    got, route = _layer_out(x, w, b, store)
    assert [int(e) for e in route.indices.tolist()] == ids
    miss = sorted(range(2, 6), key=lambda i: -wts[i])[:2]
    kept = sorted([0, 1] + miss)
    want, ys = _oracle_out(fmt, x, [ids[i] for i in kept], rescale_kept(wts, kept))
    assert store.skipped_experts == 2 and store.stats.misses == 2
    ulps = bf16_ulp_dist(got, want)
    report("miss budget", kept=len(kept), out_ulps_max=int(ulps.max()), out_ulps_nonzero=int((ulps > 0).sum()))
    assert np.all(np.abs(got - want) <= 2e-3 * np.abs(want).max() + np.sum(bf16_ulp(ys), 0) + bf16_ulp(want))


def test_decode_substitution_replaces_weak_misses(cuda):
    """decode_substitute_tau: weak non-resident routed experts are replaced by the best
    resident experts ranked just below the top-6 (decode_substitution.py)."""
    from cachalot_amd.decode_substitution import plan_substitution, ranked_candidates

    def resident(ids, sel):
        cand = ranked_candidates(sel, ids, 4)
        return [ids[0], ids[3], cand[0], cand[2]]

    fmt, store, x, w, b, ids, wts = _partial_layer(cuda, resident)
    store.decode_substitute_tau = 0.5
    sel = _np(__import__("cachalot_amd.router", fromlist=["x"]).route_topk_fused(
        x, w, b, topk=6, route_scale=1.0, score_fn="sigmoid").scores) + _np(b)
    want_ids, n = plan_substitution(ids, wts, ranked_candidates(sel, ids, 4),
                                    lambda e: store.is_cached((0, e)), 0.5)
    got, _ = _layer_out(x, w, b, store)
    assert n >= 1 and store.substituted_experts == n
    want, ys = _oracle_out(fmt, x, want_ids, wts)
    report("substitution", replaced=n, ids=want_ids)
    assert np.all(np.abs(got - want) <= 2e-3 * np.abs(want).max() + np.sum(bf16_ulp(ys), 0) + bf16_ulp(want))


def test_routing_prediction_loads_the_next_layer_ahead(cuda):
    """With the next layer's gate in decode_gates, a partially resident layer also
    routes its input through that gate (top-6, moe_layer_metal.py:186-244) and loads
    those experts ahead; the next layer then admits them without a load.  The outputs
    equal those of the same calls without prediction, bit for bit."""
    from cachalot_amd import synth
    from cachalot_amd.moe_layer import moe_layer_forward
    from cachalot_amd.router import route_topk_fused
    from cachalot_amd.storage.index import affine_format

    fmt = affine_format(4096, 2880)
    gates = {la: synth.router_weights(SEED, la, 384, 4096, cuda) for la in range(2)}
    x = synth.activations(SEED, 809, 1, 4096, cuda)[0]
    outs = []
    for predict in (False, True):
        store = make_store(fmt, n_layers=2, n_experts=384, keys=[], n_slots=32, loader=True)
        store.predict_slot_reserve = 0
        loads = []
        inner = store.loader
        store.loader = lambda entry, slot: (loads.append((entry.layer, entry.expert)), inner(entry, slot))
        if predict:
            store.decode_gates = {1: gates[1]}
        got = []
        for la in range(2):
            w, b = gates[la]
            out, route = moe_layer_forward(x, layer_id=la, gate_weight=w, gate_bias=b, expert_index=None,
                                           expert_store=store, topk=6, route_scale=1.0, score_fn="sigmoid")
            got.append((out.clone(), [int(e) for e in route.indices.tolist()]))
        outs.append(got)
        if predict:
            pred = [int(e) for e in route_topk_fused(x, *gates[1], topk=6, route_scale=1.0,
                                                      score_fn="sigmoid").indices.tolist()]
            assert got[1][1] == pred                      # layer 1 routes the same input through the same gate
            assert store.predicted_loads == 6 and store.predicted_used == 6 and store.predicted_expired == 0
            assert loads[6:12] == [(1, e) for e in reversed(pred)]   # strongest first, ascending order
            assert len(loads) == 12                       # layer 1 loaded nothing itself
        else:
            assert len(loads) == 12 and store.predicted_loads == 0
    for (a, ia), (b, ib) in zip(outs[0], outs[1]):
        assert ia == ib and torch.equal(a.view(torch.int16), b.view(torch.int16))
