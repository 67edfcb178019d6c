"""GPU parity of the FP8 shared expert against oracle/fp8.py.

Bar: act_quant codes and block exponents bit-exact; the FP8 linear within one
bf16 ulp of the exact block-scaled sum, plus 2^-20 of the sum of the terms'
magnitudes for the fp32 accumulation order (the reference accumulates in fp32
too, in another order); the
shared expert's output within max relative error 2e-3 (max |got - want| /
max |want|) plus one bf16 ulp per element for its final cast.  Weights follow
the reference's own test generator (tests/test_shared_expert_fused.py:31-38:
random E4M3 bytes, E8M0 scales in [120, 130]), NaN codes excluded.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import SEED, bf16_ulp, make_store, rel_err
from oracle import fp8 as ofp8
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _np(t):
    return t.detach().cpu().numpy()


def _bf16_np(t):
    return bf16_bits_to_f32(_np(t.contiguous().view(torch.int16)).view(np.uint16))


def _to_dev_bf16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(f32_to_bf16_bits(np.asarray(a, np.float32)).view(np.int16)).to(dev).view(torch.bfloat16)


def _weights(rng, n, k):
    w = rng.integers(0, 256, size=(n, k), dtype=np.uint8)
    w[(w & 0x7F) == 0x7F] = 0x3F
    s = rng.integers(120, 131, size=(-(-n // 32), k // 32), dtype=np.uint8)
    return w, s


def _expert(rng, d, f):
    return _weights(rng, f, d), _weights(rng, f, d), _weights(rng, d, f)


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_act_quant_bit_exact(cuda):
    from cachalot_amd.shared_expert import quantize_fp8_activation

    rng = np.random.default_rng(SEED)
    m, k = 37, 4096
    x = rng.standard_normal((m, k)) * np.exp2(rng.integers(-30, 30, size=(m, 1)))
    x[0, :32] = 0.0                                               # amax floor 1e-4
    x[1, :32] = -1e-30                                            # negative underflow -> -0 codes
    x[2, :32] = 448.0 * 2.0 ** -5                                 # amax / 448 a power of two
    vals = ofp8.e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = (vals[1:] + vals[:-1]) / 2                             # ties: RNE picks the even code
    x[3, :32] = np.concatenate([[448.0], mids[-31:]]) * 2.0 ** 3
    x[4, :32] = np.concatenate([[448.0], mids[:31]]) * 2.0 ** -2
    x[5, :64] = np.concatenate([[448.0], -mids[40:71]] * 2) * 2.0 ** 7
    x = round_bf16(x.astype(np.float32))
    q = quantize_fp8_activation(_to_dev_bf16(x, cuda))
    wq, we = ofp8.act_quant(x)
    assert np.array_equal(_np(q.values), wq)
    assert np.array_equal(_np(q.scales).astype(np.int32), we + 127)
    # 1-D input (the decode shape)
    q1 = quantize_fp8_activation(_to_dev_bf16(x[7], cuda))
    assert np.array_equal(_np(q1.values), wq[7])


@pytest.mark.parametrize("m,k,n", [(1, 4096, 2880), (3, 2880, 4096), (16, 320, 96), (200, 1024, 640)])
def test_fp8_linear_within_one_bf16_ulp(cuda, m, k, n):
    from cachalot_amd.shared_expert import fp8_linear

    rng = np.random.default_rng(SEED + m)
    w, s = _weights(rng, n, k)
    x = round_bf16(rng.standard_normal((m, k)).astype(np.float32))
    y = fp8_linear(_to_dev_bf16(x, cuda), _dev(w, cuda), _dev(s, cuda))
    torch.cuda.synchronize()
    q, e = ofp8.act_quant(x)
    exact = ofp8.linear(q, e, w, s)
    mag = ofp8.linear(q & 0x7F, e, w & 0x7F, s)                  # sum of |terms|: fp32 summation-order slack
    got = _bf16_np(y)
    assert np.all(np.abs(got - exact) <= bf16_ulp(exact) + 2.0 ** -20 * mag), (m, k, n)
    assert np.mean(got == round_bf16(exact.astype(np.float32))) > 0.99


def _one_ulp_of_exact(got, q, e, w, s):
    """got within one bf16 ulp of the exact block-scaled sum, plus 2^-20 of the sum of the
    terms' magnitudes for the fp32 accumulation order (the bar of the FP8 linear)."""
    exact = ofp8.linear(q, e, w, s)
    mag = ofp8.linear(q & 0x7F, e, w & 0x7F, s)
    return np.all(np.abs(got - exact) <= bf16_ulp(exact) + 2.0 ** -20 * mag)


@pytest.mark.parametrize("m,d,f", [(1, 4096, 2880), (1, 5120, 2304), (3, 4096, 2880), (4, 1024, 2304),
                                   (5, 256, 192), (130, 1024, 640), (200, 4096, 2880)])
def test_shared_expert_matches_oracle(cuda, m, d, f):
    """Decode sizes (M <= 4): the whole expert against the exact oracle, within the 2e-3 bar plus
    one bf16 ulp per element.  Many tokens: stage by stage -- the gate/up products (the FP8 linear,
    the same kernel and the same bits as inside the expert) within one bf16 ulp of the exact sums,
    then y within one ulp of the exact down sum of act_quant(h), h formed from those g and u.
    (End to end against the exact oracle, a g or u one ulp off at a bf16 rounding boundary -- the
    reference's fp32 order is MLX's own -- can move one E4M3 code of h, and with it a row of y by
    a few tenths of a percent: both the 64 x 64 and the 128 x 128 GEMM met that on some shape.)"""
    from cachalot_amd.shared_expert import (fp8_linear_quantized, quantize_fp8_activation, shared_expert_forward,
                                            shared_expert_forward_batched)

    rng = np.random.default_rng(SEED + d + m)
    (w1, s1), (w3, s3), (w2, s2) = _expert(rng, d, f)
    x = round_bf16(rng.standard_normal((m, d)).astype(np.float32))
    dev = {n: _dev(a, cuda) for n, a in dict(w1=w1, w1_scales=s1, w3=w3, w3_scales=s3, w2=w2, w2_scales=s2).items()}
    xd = _to_dev_bf16(x, cuda)
    q, e = ofp8.act_quant(x)
    if m > ofp8_decode_rows():
        qd = quantize_fp8_activation(xd)
        g = _bf16_np(fp8_linear_quantized(qd, dev["w1"], dev["w1_scales"]))
        u = _bf16_np(fp8_linear_quantized(qd, dev["w3"], dev["w3_scales"]))
        assert _one_ulp_of_exact(g, q, e, w1, s1) and _one_ulp_of_exact(u, q, e, w3, s3), (m, d, f)
    for limit in (10.0, 0.25):
        y = shared_expert_forward(xd[0], **dev, swiglu_limit=limit)[None] if m == 1 else \
            shared_expert_forward_batched(xd, **dev, swiglu_limit=limit)
        got = _bf16_np(y)
        want = ofp8.shared_expert(x, w1, s1, w3, s3, w2, s2, limit=limit)
        assert rel_err(got, want) <= TOL + 2.0 ** -8, (m, d, f, limit)
        if m <= ofp8_decode_rows():
            assert np.all(np.abs(got - want) <= TOL * np.abs(want).max() + bf16_ulp(want)), (m, d, f, limit)
            continue
        gg, uu = g.astype(np.float64), u.astype(np.float64)
        uu, gg = np.clip(uu, -limit, limit), np.minimum(gg, limit)
        with np.errstate(over="ignore"):
            hv = gg / (1.0 + np.exp(-gg)) * uu
        h = round_bf16(hv.astype(np.float32))
        # the kernel forms h in fp32 (hardware exp): where hv lies within 2^-21 of a bf16
        # rounding boundary either neighbour may come out; those elements' E4M3 codes (and
        # their blocks' scales) are requantized with the other neighbour, and y's bar widens
        # by exactly the change they can make
        h_lo = round_bf16((hv * (1.0 - 2.0 ** -21)).astype(np.float32))
        h_hi = round_bf16((hv * (1.0 + 2.0 ** -21)).astype(np.float32))
        h_alt = np.where(h_lo != h, h_lo, np.where(h_hi != h, h_hi, h))
        qh, eh = ofp8.act_quant(h)
        qa, ea = ofp8.act_quant(h_alt)
        deq = lambda q_, e_: ofp8.e4m3_decode(q_).astype(np.float64) * np.exp2(np.repeat(e_, 32, axis=-1))
        dh = np.abs(deq(qa, ea) - deq(qh, eh))                                # [M, F]
        w2v = np.abs(ofp8.e4m3_decode(w2).astype(np.float64)) * np.exp2(
            np.repeat(s2.astype(np.float64) - 127.0, 32, axis=1)[np.arange(d) // 32][:, :f])
        slack = dh @ w2v.T                                                    # [M, D]
        exact = ofp8.linear(qh, eh, w2, s2)
        mag = ofp8.linear(qh & 0x7F, eh, w2 & 0x7F, s2)
        bad = np.abs(got - exact) > bf16_ulp(exact) + 2.0 ** -20 * mag + slack
        assert not bad.any(), (m, d, f, limit, int(bad.sum()), int((dh > 0).sum()))


def ofp8_decode_rows():
    """Tokens up to which the expert runs its decode tiles (quantizing x itself)."""
    return 4


def test_shared_expert_fused_w13_is_identical(cuda):
    from cachalot_amd.shared_expert import shared_expert_forward, shared_expert_forward_fused

    rng = np.random.default_rng(SEED + 1)
    (w1, s1), (w3, s3), (w2, s2) = _expert(rng, 1024, 640)
    x = _to_dev_bf16(round_bf16(rng.standard_normal(1024).astype(np.float32)), cuda)
    a = shared_expert_forward(x, w1=_dev(w1, cuda), w1_scales=_dev(s1, cuda), w3=_dev(w3, cuda),
                              w3_scales=_dev(s3, cuda), w2=_dev(w2, cuda), w2_scales=_dev(s2, cuda))
    b = shared_expert_forward_fused(x, w13=_dev(np.concatenate([w1, w3]), cuda),
                                    w13_scales=_dev(np.concatenate([s1, s3]), cuda), w2=_dev(w2, cuda),
                                    w2_scales=_dev(s2, cuda))
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_layer_entries_add_the_shared_expert(cuda):
    """moe_layer_forward / moe_prefill_grouped with shared_* give exactly the
    output of the same call with the shared expert's output as the addend, the
    reference's bf16(routed + shared) (moe_layer_metal.py:381-397,
    moe_prefill_grouped.py:532-545)."""
    from cachalot_amd import synth
    from cachalot_amd.moe_layer import moe_layer_forward
    from cachalot_amd.moe_prefill import moe_prefill_grouped
    from cachalot_amd.shared_expert import shared_expert_forward, shared_expert_forward_batched
    from cachalot_amd.storage.index import affine_format

    d, f, e = 4096, 2880, 16
    store = make_store(affine_format(d, f), n_layers=1, n_experts=e)
    w, b = synth.router_weights(SEED, 0, e, d, cuda)
    rng = np.random.default_rng(SEED + 2)
    (w1, s1), (w3, s3), (w2, s2) = _expert(rng, d, 2304)
    shared = dict(shared_w1=_dev(w1, cuda), shared_w1_scales=_dev(s1, cuda), shared_w2=_dev(w2, cuda),
                  shared_w2_scales=_dev(s2, cuda), shared_w3=_dev(w3, cuda), shared_w3_scales=_dev(s3, cuda))
    plain = {k[len("shared_"):]: v for k, v in shared.items()}
    kw = dict(layer_id=0, gate_weight=w, gate_bias=b, expert_index=None, expert_store=store, topk=6,
              route_scale=1.0, score_fn="sigmoid")
    x = synth.activations(SEED, 90, 8, d, cuda)
    out, route = moe_layer_forward(x[0], **kw, **shared)
    ref, route2 = moe_layer_forward(x[0], **kw, addend=shared_expert_forward(x[0], **plain))
    assert torch.equal(route.indices, route2.indices)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    outp, _ = moe_prefill_grouped(x, **kw, **shared)
    refp, _ = moe_prefill_grouped(x, **kw, addend=shared_expert_forward_batched(x, **plain))
    assert torch.equal(outp.view(torch.int16), refp.view(torch.int16))
    # from SIDE_STREAM_MIN_TOKENS tokens on the shared expert runs on a second stream
    xl = synth.activations(SEED, 91, 300, d, cuda)
    refl, _ = moe_prefill_grouped(xl, **kw, addend=shared_expert_forward_batched(xl, **plain))
    for _ in range(3):
        outl, _ = moe_prefill_grouped(xl, **kw, **shared)
        assert torch.equal(outl.view(torch.int16), refl.view(torch.int16))
    with pytest.raises(ValueError):
        moe_layer_forward(x[0], **kw, **shared, addend=refp[0])


def test_shared_expert_argument_errors_and_no_limit(cuda):
    """Contract errors (the reference's ValueErrors for shapes, fp8_ref.py:48-58,140-170) and
    swiglu_limit <= 0 (no clamp, shared_expert_metal.py:99-108)."""
    from cachalot_amd.shared_expert import fp8_linear, quantize_fp8_activation, shared_expert_forward

    rng = np.random.default_rng(SEED + 7)
    (w1, s1), (w3, s3), (w2, s2) = _expert(rng, 256, 192)
    dev = {n: _dev(a, cuda) for n, a in dict(w1=w1, w1_scales=s1, w3=w3, w3_scales=s3, w2=w2, w2_scales=s2).items()}
    x = round_bf16((rng.standard_normal(256) * 4).astype(np.float32))
    got = _bf16_np(shared_expert_forward(_to_dev_bf16(x, cuda), **dev, swiglu_limit=0.0))
    want = ofp8.shared_expert(x[None], w1, s1, w3, s3, w2, s2, limit=0.0)[0]
    assert np.all(np.abs(got - want) <= TOL * np.abs(want).max() + bf16_ulp(want))
    with pytest.raises(ValueError):
        quantize_fp8_activation(_to_dev_bf16(np.zeros(40, np.float32), cuda))          # K not a multiple of 32
    with pytest.raises(ValueError):
        fp8_linear(_to_dev_bf16(x, cuda), dev["w1"], dev["w1_scales"][:-1])            # scale shape
    with pytest.raises(ValueError):
        fp8_linear(_to_dev_bf16(x[:128], cuda), dev["w1"], dev["w1_scales"])           # K mismatch
    with pytest.raises(ValueError):
        shared_expert_forward(_to_dev_bf16(x, cuda)[None], **dev)                       # decode takes 1-D x
    with pytest.raises(ValueError):
        shared_expert_forward(_to_dev_bf16(x, cuda), **{**dev, "w2": dev["w1"]})       # w2 shape


@pytest.mark.parametrize("kind,d,f_sh,k,limit", [
    ("affine", 4096, 2880, 6, 10.0), ("affine", 4096, 2880, 8, 0.25), ("affine", 2048, 4096, 6, 0.0),
    ("affine", 1024, 640, 3, 10.0), ("affine", 5120, 2880, 6, 10.0), ("affine", 4096, 4608, 6, 10.0),
    ("fp4", 4096, 2880, 6, 10.0), ("fp4", 2048, 3072, 3, 0.25), ("fp4", 4096, 2880, 8, 10.0),
    ("fp4", 1024, 640, 2, 0.0)])
def test_layer_decode_carries_the_shared_expert(cuda, kind, d, f_sh, k, limit):
    """cachalot_moe_layer_decode_{q2,fp4}_shared equal, bit for bit, the shared expert's
    own call followed by the layer decode with its output as addend -- where the routed
    launches carry the shared tiles (2-bit: D, F_sh <= 4096; FP4: also 3 <= k <= 6) and
    where the shared expert runs first (D = 5120, F_sh = 4608, FP4 at k = 8 and 2);
    routing and the fp32 routed sum unchanged."""
    from cachalot_amd import synth
    from cachalot_amd.moe_decode import moe_layer_decode
    from cachalot_amd.shared_expert import shared_expert_forward
    from cachalot_amd.storage.index import affine_format, fp4_format

    f, e = 2880, 24
    fmt = affine_format(d, f) if kind == "affine" else fp4_format(d, f)
    store = make_store(fmt, n_layers=1, n_experts=e)
    w, b = synth.router_weights(SEED, 3, e, d, cuda)
    rng = np.random.default_rng(SEED + d + f_sh + k)
    (w1, s1), (w3, s3), (w2, s2) = _expert(rng, d, f_sh)
    plain = dict(w1=_dev(w1, cuda), w1_scales=_dev(s1, cuda), w2=_dev(w2, cuda), w2_scales=_dev(s2, cuda),
                 w3=_dev(w3, cuda), w3_scales=_dev(s3, cuda))
    kw = dict(topk=k, route_scale=1.0, score_fn="sigmoid", swiglu_limit=limit, want_routed=True)
    xs = synth.activations(SEED, 91, 3, d, cuda)
    for t in range(3):
        args = (xs[t], w, b, store.pool, store.layer_table(0))
        r1, o1, rt1 = moe_layer_decode(*args, **kw, shared=plain)
        r2, o2, rt2 = moe_layer_decode(*args, **kw, addend=shared_expert_forward(xs[t], **plain, swiglu_limit=limit))
        assert torch.equal(rt1.indices, rt2.indices) and torch.equal(rt1.weights, rt2.weights), (kind, d, f_sh, k, t)
        assert torch.equal(r1, r2), (kind, d, f_sh, k, t)
        assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), (kind, d, f_sh, k, t)
    # a captured step replays to the eager result (the workspace exists from the eager calls)
    x = xs[0].clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _, og, _ = moe_layer_decode(x, w, b, store.pool, store.layer_table(0), **kw, shared=plain)
    _, want, _ = moe_layer_decode(xs[0], w, b, store.pool, store.layer_table(0), **kw, shared=plain)
    for t in (1, 0, 2, 0):
        x.copy_(xs[t])
        g.replay()
        torch.cuda.synchronize()
        _, eager, _ = moe_layer_decode(xs[t], w, b, store.pool, store.layer_table(0), **kw, shared=plain)
        assert torch.equal(og.view(torch.int16), eager.view(torch.int16)), t
    with pytest.raises(ValueError):
        moe_layer_decode(xs[0], w, b, store.pool, store.layer_table(0), **kw, shared=plain, addend=xs[1])


def test_fp8_row_helpers_match_oracle(cuda):
    """quantize_activation_fp8_rows / dequantize_fp8_weight (moe_prefill_batched.py:62-84):
    exact dequantized values, bit for bit against oracle.fp8 (act_quant codes times 2^e,
    E4M3 times E8M0 with N not a multiple of 32 and edge scale bytes); fp8_linear_rows
    is fp8_linear on rows."""
    from cachalot_amd.shared_expert import (dequantize_fp8_weight, fp8_linear, fp8_linear_rows, gemm_dtype,
                                            quantize_activation_fp8_rows)

    rng = np.random.default_rng(SEED + 31)
    x = rng.standard_normal((7, 256)).astype(np.float32) * np.float32(3.0)
    x[1, :32] = 0.0                                  # an all-zero block (the amax floor)
    x[2, 32:64] *= np.float32(1e-6)                  # a tiny block
    x = round_bf16(x)
    xd = _to_dev_bf16(x, cuda)
    q, e = ofp8.act_quant(x)
    want = (ofp8.e4m3_decode(q).reshape(7, 8, 32) * np.exp2(e.astype(np.float64))[..., None]).reshape(7, 256)
    got = _np(quantize_activation_fp8_rows(xd))
    assert got.dtype == np.float32 and np.array_equal(got, want.astype(np.float32))
    got_bf = quantize_activation_fp8_rows(xd, torch.bfloat16)
    assert got_bf.dtype == torch.bfloat16 and np.array_equal(_np(got_bf.float()), want.astype(np.float32))

    w = rng.integers(0, 256, size=(80, 256), dtype=np.uint8)
    w[(w & 0x7F) == 0x7F] = 0x3F
    s = rng.integers(100, 140, size=(3, 8), dtype=np.uint8)
    s[0, 0], s[2, 7] = 10, 240                       # the smallest products stay normal; 2^113
    rows = np.arange(80) // 32
    want_w = ofp8.e4m3_decode(w).astype(np.float64) * np.exp2(s.astype(np.float64) - 127.0)[rows][:, np.arange(256) // 32]
    got_w = _np(dequantize_fp8_weight(_dev(w, cuda), _dev(s, cuda)))
    assert np.array_equal(got_w, want_w.astype(np.float32))
    with pytest.raises(ValueError):
        dequantize_fp8_weight(_dev(w, cuda), _dev(s[:2], cuda))

    wd, sd = _dev(w[:64], cuda), _dev(s[:2], cuda)
    assert torch.equal(fp8_linear_rows(xd, wd, sd).view(torch.int16), fp8_linear(xd, wd, sd).view(torch.int16))
    with pytest.raises(ValueError):
        fp8_linear_rows(xd[0], wd, sd)
    assert gemm_dtype() in (torch.bfloat16, torch.float32)
    from cachalot_amd.shared_expert import _e8m0_values

    sv = _np(_e8m0_values(torch.tensor([0, 1, 127, 254, 255], dtype=torch.uint8, device=cuda)))
    assert sv[0] == np.float32(2.0 ** -127) and sv[1] == np.float32(2.0 ** -126)
    assert sv[2] == 1.0 and sv[3] == np.float32(2.0 ** 127) and np.isnan(sv[4])
