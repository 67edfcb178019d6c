"""Affine banks of the other widths (3 / 4 bits, groups of 32 / 64, bf16 or fp16
scales): oQ3e is 3-bit g64 with fp16 scales (expert_affine.py:1-10), and the bank
tool writes bits 2/3/4 x groups 32/64/128 (build_affine_bank.py:266-267).

* dequantisation bit-exact against oracle/affine2.py (the MLX bit-stream layout);
* decode at the layer's shape (block-scaled matrix-core kernels for every width,
  and the VALU kernels), per-expert terms against the oracle's rounding points
  (helpers.term_flips), routed = the route-order sum bit for bit,
  out = bf16(routed + addend) bit for bit; the device-routed layer with ids
  bit-exact;
* grouped (prefill / batched) rows against the oracle on the block-scaled prefill kernels,
  the bf16-MFMA grouped kernels and the VALU kernels, dropped ids giving zeros; a small
  layer shape whose K and group counts are ragged on the block-scaled kernels.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import SEED, make_store, oracle_tensors, q2_mats
from oracle import router as orouter
from oracle import synth as osynth
from oracle.affine2 import dequantize_affine
from oracle.bf16 import bf16_bits_to_f32
from test_gpu_workloads import TERM_TOL, _bf16, _check_decode, _decode_terms, _f32, _grouped_check, _np

pytestmark = pytest.mark.gpu

WIDTHS = [(3, 64, "float16"), (4, 32, "bfloat16"), (3, 128, "bfloat16"), (2, 64, "float16")]


def _fmt(bits, group, sd, d=4096, f=2880):
    from cachalot_amd.storage.index import affine_format

    return affine_format(d, f, bits=bits, group_size=group, scale_dtype=sd)


@pytest.mark.parametrize("bits,group,sd", WIDTHS)
def test_affine_dequant_and_fill_bit_exact(cuda, bits, group, sd):
    from cachalot_amd import _lib

    fmt = _fmt(bits, group, sd)
    t = oracle_tensors(fmt, 0, 7)
    for proj, k in (("w1", 4096), ("w2", 2880)):
        w, s, b = t[f"{proj}.weight"], t[f"{proj}.scales"], t[f"{proj}.biases"]
        n, row_words = w.shape
        out = torch.empty((n, k), dtype=torch.float32, device=cuda)
        dw = torch.from_numpy(w.view(np.int32)).to(cuda)
        ds = torch.from_numpy(s.view(np.int16)).to(cuda)
        db = torch.from_numpy(b.view(np.int16)).to(cuda)
        _lib.check(_lib.lib().cachalot_dequant_affine(dw.data_ptr(), ds.data_ptr(), db.data_ptr(), n, k, row_words,
                                                      s.shape[1], group, bits, _lib.scale_dtype_code(sd),
                                                      out.data_ptr(), _lib.stream_handle(cuda)))
        want = dequantize_affine(w, s, b, k=k, group=group, scale_dtype=sd, bits=bits)
        assert np.array_equal(_np(out).view(np.uint32), want.view(np.uint32)), (proj, bits, group)
    store = make_store(fmt, n_layers=1, n_experts=8, keys=[(0, 7)])
    slot = store.pool.slot(store.layer_table(0)[7].item())
    for name, arr in t.items():
        assert np.array_equal(_np(slot.arrays[name]), arr.view(np.uint8).reshape(-1)), name


DECODE_CASES = [(3, 64, "float16", "mx"), (4, 32, "bfloat16", "mx"), (3, 128, "bfloat16", "mx"),
                (2, 64, "float16", "mx"), (4, 128, "float16", "mx"), (2, 32, "bfloat16", "mx"),
                (3, 32, "float16", "mx"), (4, 64, "bfloat16", "mx"),
                (3, 64, "float16", "valu"), (4, 32, "bfloat16", "valu")]


@pytest.mark.parametrize("bits,group,sd,path", DECODE_CASES)
def test_affine_decode_terms(cuda, bits, group, sd, path, monkeypatch):
    """Given experts (two tokens) and the device-routed layer (one token), on the block-scaled
    matrix-core kernels (the default at these shapes) and the VALU kernels
    (CACHALOT_AFFINE_VALU=1)."""
    from cachalot_amd import synth
    from cachalot_amd.moe_decode import decode_experts, moe_layer_decode

    monkeypatch.setenv("CACHALOT_AFFINE_VALU", "1" if path == "valu" else "0")
    monkeypatch.setenv("CACHALOT_PREFILL_BF16", "1" if path == "bf16" else "0")
    fmt = _fmt(bits, group, sd)
    store = make_store(fmt, n_layers=1, n_experts=384)
    rng = np.random.default_rng(bits * 100 + group)
    for tk in range(2):
        idx = rng.choice(384, size=6, replace=False).tolist()
        w = rng.dirichlet(np.ones(6)).astype(np.float32)
        xb = osynth.activations(SEED, 3000 + tk, 1, 4096)[0]
        ab = osynth.activations(SEED, 3100 + tk, 1, 4096)[0]
        x, a = _bf16(xb, cuda), _bf16(ab, cuda)
        routed, out = decode_experts(x, store.pool, store.layer_table(0), torch.tensor(idx, dtype=torch.int32,
                                                                                       device=cuda),
                                     torch.tensor(w, device=cuda), addend=a)
        terms = _decode_terms(cuda, store, 0, x, idx, w)
        _check_decode(f"affine {bits}-bit g{group} {sd} {path} token {tk}", fmt, 0, bf16_bits_to_f32(xb), idx, w,
                      _np(routed), _f32(out), terms, bf16_bits_to_f32(ab))
    gw, gb = synth.router_weights(SEED, 0, 384, 4096, cuda)
    x = synth.activations(SEED, 3200, 1, 4096, cuda)[0]
    routed, out, route = moe_layer_decode(x, gw, gb, store.pool, store.layer_table(0), topk=6, route_scale=1.0,
                                          score_fn="sigmoid", addend=x, want_routed=True)
    xf = _f32(x)
    oi, ow, _ = orouter.route(xf[None], _f32(gw), _np(gb), topk=6, route_scale=1.0, score=orouter.SCORE_SIGMOID)
    assert np.array_equal(_np(route.indices), oi[0])
    assert np.array_equal(_np(route.weights).view(np.uint32), ow[0].view(np.uint32))
    terms = _decode_terms(cuda, store, 0, x, oi[0], ow[0])
    _check_decode(f"affine {bits}-bit g{group} {path} layer", fmt, 0, xf, oi[0], ow[0], _np(routed), _f32(out), terms, xf)


# path: "mfma" = the default kernels (64-row tiles: the block-scaled prefill kernels for
# 2-bit g64 and 3- / 4-bit g64 / g128, the bf16-MFMA grouped kernels for groups of 32;
# 16-row tiles at t = 4), "bf16" = the bf16-MFMA grouped kernels (CACHALOT_PREFILL_BF16=1),
# "valu" = the VALU kernels (CACHALOT_AFFINE_VALU=1)
GROUPED_CASES = [(3, 64, "float16", "mfma", 37, 16), (4, 32, "bfloat16", "mfma", 37, 16),
                 (3, 128, "bfloat16", "mfma", 37, 16), (2, 64, "float16", "mfma", 37, 16),
                 (4, 128, "float16", "mfma", 200, 8), (2, 32, "bfloat16", "mfma", 4, 16),
                 (3, 32, "float16", "mfma", 4, 16), (4, 64, "bfloat16", "mfma", 37, 16),
                 (3, 64, "float16", "mfma", 200, 8), (3, 64, "bfloat16", "bf16", 37, 16),
                 (4, 128, "float16", "bf16", 200, 8),
                 (3, 64, "float16", "valu", 37, 16), (4, 32, "bfloat16", "valu", 37, 16)]


@pytest.mark.parametrize("bits,group,sd,path,t,E", GROUPED_CASES)
def test_affine_grouped_rows(cuda, bits, group, sd, path, t, E, monkeypatch):
    """t tokens x top-6 over E experts (uneven rows), three dropped ids, on each kernel family
    (T = 200 over 8 experts: experts of several tiles)."""
    from cachalot_amd.moe_prefill import grouped_experts

    monkeypatch.setenv("CACHALOT_AFFINE_VALU", "1" if path == "valu" else "0")
    monkeypatch.setenv("CACHALOT_PREFILL_BF16", "1" if path == "bf16" else "0")
    fmt = _fmt(bits, group, sd)
    k = 6
    store = make_store(fmt, n_layers=1, n_experts=E)
    rng = np.random.default_rng(7 + bits + t)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(t)]).astype(np.int32)
    drops = [(0, 1), (t // 2, k - 1), (t - 1, 0)]
    for (r, c), v in zip(drops, (-1, E + 2, 1 << 29)):
        idx[r, c] = v
    w = rng.dirichlet(np.ones(k), size=t).astype(np.float32)
    xb = osynth.activations(SEED, 3300, t, 4096)
    ab = osynth.activations(SEED, 3301, t, 4096)
    for _ in range(2):   # y reused from a previous call must not leak into the dropped rows
        routed, out, y = grouped_experts(_bf16(xb, cuda), torch.from_numpy(idx).to(cuda),
                                         torch.from_numpy(w).to(cuda), store.pool, store.layer_table(0),
                                         addend=_bf16(ab, cuda), want_routed=True, want_terms=True)
        yf = _f32(y)
        assert not any(yf[r, c].any() for r, c in drops)
        _grouped_check(f"grouped affine {bits}-bit g{group} {path} T={t}", fmt, 0, bf16_bits_to_f32(xb), idx, w,
                       _np(routed), _f32(out), yf, E, addend=bf16_bits_to_f32(ab))


def test_affine_missing_slot_and_graph_replays(cuda):
    """oQ3e (3-bit g64 fp16): an expert without a slot contributes exact zeros (routed = the route-order
    sum of the other experts' one-expert terms, bit for bit), and a captured chain of device-routed layer
    decodes replays identically, three times, with eager work and synchronisation between replays."""
    from cachalot_amd import synth
    from cachalot_amd.moe_decode import decode_experts, moe_layer_decode
    from helpers import route_order_sum
    from test_gpu_workloads import _decode_terms

    fmt = _fmt(3, 64, "float16")
    store = make_store(fmt, n_layers=2, n_experts=384)
    idx = [5, 77, 300, 12, 250, 199]
    w = np.full(6, 1 / 6, np.float32)
    x = synth.activations(SEED, 3400, 1, 4096, cuda)[0]
    terms = _decode_terms(cuda, store, 0, x, idx, w)
    store.track_slots()[0, 77] = -1
    routed, _ = decode_experts(x, store.pool, store.layer_table(0), torch.tensor(idx, dtype=torch.int32, device=cuda),
                               torch.from_numpy(w).to(cuda))
    terms[1] = 0.0
    assert np.array_equal(_np(routed).view(np.uint32), route_order_sum(terms).view(np.uint32))
    gates = [synth.router_weights(SEED, la, 384, 4096, cuda) for la in range(2)]

    def chain(x):
        for s in range(4):
            gw, gb = gates[s % 2]
            _, x, _ = moe_layer_decode(x, gw, gb, store.pool, store.layer_table(1), topk=6, route_scale=1.0,
                                       score_fn="sigmoid", addend=x)
        return x

    x0 = synth.activations(SEED, 3401, 1, 4096, cuda)[0]
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
        _ = chain(x0)
        torch.cuda.synchronize()


@pytest.mark.parametrize("bits,group,sd,d,f,k", [(3, 32, "float16", 4096, 2880, 8), (4, 64, "bfloat16", 5120, 2304, 6),
                                                (4, 128, "float16", 5120, 3072, 8), (2, 32, "bfloat16", 1024, 512, 3)])
def test_affine_decode_other_shapes(cuda, bits, group, sd, d, f, k):
    """The matrix-core decode's other register budgets: k = 8 (more down items per wave), D = 5120
    (more gate/up items per wave), F = 3072 (the largest K of the down kernel), a small layer."""
    from cachalot_amd.moe_decode import decode_experts

    fmt = _fmt(bits, group, sd, d=d, f=f)
    store = make_store(fmt, n_layers=1, n_experts=64)
    rng = np.random.default_rng(bits * 1000 + group + d + k)
    idx = rng.choice(64, size=k, replace=False).tolist()
    w = rng.dirichlet(np.ones(k)).astype(np.float32)
    xb = osynth.activations(SEED, 3500 + d, 1, d)[0]
    ab = osynth.activations(SEED, 3600 + d, 1, d)[0]
    x, a = _bf16(xb, cuda), _bf16(ab, cuda)
    routed, out = decode_experts(x, store.pool, store.layer_table(0), torch.tensor(idx, dtype=torch.int32, device=cuda),
                                 torch.tensor(w, device=cuda), addend=a)
    terms = _decode_terms(cuda, store, 0, x, idx, w)
    _check_decode(f"affine {bits}-bit g{group} D={d} F={f} k={k}", fmt, 0, bf16_bits_to_f32(xb), idx, w,
                  _np(routed), _f32(out), terms, bf16_bits_to_f32(ab))


SMALL_PREFILL = [(2, 128, "float16"), (2, 64, "bfloat16"), (3, 64, "float16"), (4, 128, "bfloat16")]


@pytest.mark.parametrize("bits,group,sd", SMALL_PREFILL)
def test_affine_prefill_small_shape(cuda, bits, group, sd, monkeypatch):
    """D = 640, F = 576 on the block-scaled prefill kernels (the 2-bit g128 fp4 path, the 16 x 16 x 128
    fp8-code kernels for groups of 128, the 32 x 32 x 64 kernels for groups of 64): x is five 128-element
    chunks, h four and a half (the last chunk half past F), the rows' group counts (10 / 9 for groups of
    64, 5 for groups of 128) are not multiples of the eight groups a scale load covers, and the weight
    slices run past F and D.  48 tokens x top-6 over 8 experts (64-row tiles, some experts over 64
    rows), three dropped ids; terms against the oracle, the combine bit for bit."""
    from cachalot_amd.moe_prefill import grouped_experts

    monkeypatch.setenv("CACHALOT_AFFINE_VALU", "0")
    monkeypatch.setenv("CACHALOT_PREFILL_BF16", "0")
    D, F, E, k, t = 640, 576, 8, 6, 48
    fmt = _fmt(bits, group, sd, d=D, f=F)
    store = make_store(fmt, n_layers=1, n_experts=E)
    rng = np.random.default_rng(11 + bits + group)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(t)]).astype(np.int32)
    drops = [(0, 2), (t // 2, k - 1), (t - 1, 0)]
    for (r, c), v in zip(drops, (-1, E + 1, 1 << 28)):
        idx[r, c] = v
    w = rng.dirichlet(np.ones(k), size=t).astype(np.float32)
    xb = osynth.activations(SEED, 3400, t, D)
    ab = osynth.activations(SEED, 3401, t, D)
    routed, out, y = grouped_experts(_bf16(xb, cuda), torch.from_numpy(idx).to(cuda), torch.from_numpy(w).to(cuda),
                                     store.pool, store.layer_table(0), addend=_bf16(ab, cuda), want_routed=True,
                                     want_terms=True)
    yf = _f32(y)
    assert not any(yf[r, c].any() for r, c in drops)
    _grouped_check(f"prefill {bits}-bit g{group} {sd} D={D} F={F}", fmt, 0, bf16_bits_to_f32(xb), idx, w,
                   _np(routed), _f32(out), yf, E, addend=bf16_bits_to_f32(ab))


@pytest.mark.parametrize("bits,group", [(2, 128), (3, 64)])
def test_affine_prefill_config3_routing(cuda, bits, group, monkeypatch):
    """Config 3's routing (4096 tokens, D 4096, F 2880, 384 experts, top-6, the Zipf router bias)
    over the 2-bit g128 and oQ3e (3-bit g64) banks with fp16 scales, on the block-scaled prefill
    kernels: 192 sampled rows of each of the three heaviest experts (hundreds to thousands of rows,
    many 64-row tiles) and every route of 16 random tokens against the oracle; the combine of all
    tokens bit for bit over the GPU's terms.  (The router itself is checked bit for bit at this
    shape by test_gpu_workloads.test_config3_prefill_workload.)"""
    from cachalot_amd import synth
    from cachalot_amd.moe_prefill import grouped_experts
    from cachalot_amd.router import route_topk_rows

    monkeypatch.setenv("CACHALOT_AFFINE_VALU", "0")
    monkeypatch.setenv("CACHALOT_PREFILL_BF16", "0")
    D, F, E, K, T = 4096, 2880, 384, 6, 4096
    fmt = _fmt(bits, group, "float16", d=D, f=F)
    store = make_store(fmt, n_layers=1, n_experts=E)
    w, b = synth.router_weights(SEED + 3, 0, E, D, cuda)
    b = b + torch.tensor(synth.zipf_bias(E, seed=SEED), dtype=torch.float32, device=cuda)
    x = synth.activations(SEED + 3, 0, T, D, cuda)
    idx, wt, _ = route_topk_rows(x, w, b, topk=K, route_scale=1.0, score_fn="sigmoid")
    oi, ow = _np(idx), _np(wt)
    counts = np.bincount(oi.reshape(-1), minlength=E)
    heavy = np.argsort(counts, kind="stable")[-3:]
    assert counts[heavy].min() > 256, counts[heavy]
    routed, out, y = grouped_experts(x, idx, wt, store.pool, store.layer_table(0), want_routed=True, want_terms=True)
    rng = np.random.default_rng(9 + bits)
    rows_of = {int(e): np.sort(rng.choice(int(counts[e]), size=192, replace=False)) for e in heavy}
    sample = {}
    for tk in rng.choice(T, size=16, replace=False):
        for s in range(K):
            sample.setdefault(int(oi[tk, s]), []).append((int(tk), s))
    for e, pairs in sample.items():
        if e in rows_of:
            continue
        want = set(pairs)
        rows = np.argwhere(oi == e)
        rows_of[e] = np.asarray([i for i, (a, c) in enumerate(rows.tolist()) if (a, c) in want])
    _grouped_check(f"config3 routing prefill {bits}-bit g{group}", fmt, 0, _f32(x), oi, ow, _np(routed), _f32(out),
                   _f32(y), E, rows_of=rows_of)
