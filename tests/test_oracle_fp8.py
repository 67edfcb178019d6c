"""Pins for the FP8 (E4M3FN + E8M0) restatement in oracle/fp8.py.

Independent checks: torch's own float8_e4m3fn dtype (bit decode of all 256 codes
and its round-to-nearest-even cast), the definition of the act_quant exponent as
the smallest power of two that maps the block maximum into [-448, 448], a
fully dequantized float64 matmul (one sum over K instead of per-block partials
scaled afterwards) for the block-scaled linear, and the shared expert rebuilt
from torch primitives (float8 cast, silu, bf16 casts).  The reference's own
shared-expert tests (tests/test_shared_expert_fused.py) need MLX and hold no
vectors; their weight generator (random bytes, E8M0 scales in [120, 130]) is the
input distribution used here.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import fp8
from oracle.bf16 import round_bf16

F8 = torch.float8_e4m3fn


def _torch_encode(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(F8).view(torch.uint8).numpy()


def _weights(rng, n, k):
    w = rng.integers(0, 256, size=(n, k), dtype=np.uint8)
    w[(w & 0x7F) == 0x7F] = 0x3F          # no NaN codes in a real checkpoint
    s = rng.integers(120, 131, size=(-(-n // 32), k // 32), dtype=np.uint8)
    return w, s


def test_decode_all_codes_match_torch():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(F8).float().numpy()
    got = fp8.e4m3_decode(codes)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def test_encode_matches_torch_rne():
    rng = np.random.default_rng(1)
    x = np.clip(rng.standard_normal(200_000).astype(np.float32) * 60.0, -448, 448)
    assert np.array_equal(fp8.e4m3_encode(x), _torch_encode(x))
    # every code round-trips; exact midpoints between neighbours go to the even code
    vals = fp8.e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = ((vals[1:] + vals[:-1]) / 2).astype(np.float32)
    for v in (vals.astype(np.float32), -vals.astype(np.float32), mids, -mids):
        assert np.array_equal(fp8.e4m3_encode(v), _torch_encode(v))
    assert np.all(fp8.e4m3_encode(mids) % 2 == 0)


def test_act_quant_exponent_is_the_smallest_fitting_power_of_two():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((64, 256)) * np.exp2(rng.integers(-20, 12, size=(64, 1)))).astype(np.float32)
    x[0, :32] = 0.0                                   # all-zero block: amax floor 1e-4
    x[1, :32] = 448.0 * 2.0 ** -3                     # amax / 448 exactly a power of two
    x[2, 32:64] = np.float32(448.0 * 2.0 ** 5) * np.float32(1 + 2 ** -23)   # one ulp above
    q, e = fp8.act_quant(x)
    blocks = x.reshape(64, 8, 32).astype(np.float64)
    amax = np.maximum(np.abs(blocks).max(-1), np.float64(np.float32(1e-4)))
    r = (amax.astype(np.float32) / np.float32(448.0)).astype(np.float64)
    for (i, j), rv in np.ndenumerate(r):
        assert 2.0 ** e[i, j] >= rv > 2.0 ** (e[i, j] - 1)
    assert e[1, 0] == -3 and e[2, 1] == 6
    want = _torch_encode(np.clip(blocks * np.exp2(-e.astype(np.float64))[..., None], -448, 448).astype(np.float32))
    assert np.array_equal(q, want.reshape(64, 256))
    assert np.all(q[0, :32] == 0)


def test_linear_matches_dequantized_matmul():
    rng = np.random.default_rng(3)
    m, n, k = 3, 80, 320                               # n not a multiple of 32 rows per scale block
    w, s = _weights(rng, n, k)
    x = round_bf16(rng.standard_normal((m, k)).astype(np.float32))
    q, e = fp8.act_quant(x)
    wd = torch.from_numpy(w).view(F8).double() * torch.from_numpy(
        np.exp2(s.astype(np.float64) - 127)).repeat_interleave(32, 0)[:n].repeat_interleave(32, 1)
    xd = torch.from_numpy(q).view(F8).double() * torch.from_numpy(np.exp2(e.astype(np.float64))).repeat_interleave(32, 1)
    want = (xd @ wd.T).numpy()
    got = fp8.linear(q, e, w, s)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())
    # the quantized product tracks the unquantized one to fp8 precision
    full = x.astype(np.float64) @ (torch.from_numpy(w).view(F8).double().numpy() * np.exp2(
        np.repeat(np.repeat(s.astype(np.float64) - 127, 32, 0)[:n], 32, 1))).T
    assert np.abs(got - full).max() < 0.1 * np.abs(full).max()


def _torch_shared(x, w1, s1, w3, s3, w2, s2, limit):
    def quant(v):
        v = torch.from_numpy(np.asarray(v, np.float32))
        b = v.reshape(v.shape[0], -1, 32)
        amax = b.abs().amax(-1).clamp_min(torch.tensor(1e-4, dtype=torch.float32))
        r = (amax / 448.0).double()
        e = torch.ceil(torch.log2(r))
        e = torch.where(torch.exp2(e - 1) >= r, e - 1, e)          # guard log2 rounding
        qv = (b.double() * torch.exp2(-e)[..., None]).clamp(-448, 448).float().to(F8)
        return qv.double().reshape(v.shape) * torch.exp2(e).repeat_interleave(32, 1)

    def deq(w, s):
        n = w.shape[0]
        sc = torch.exp2(torch.from_numpy(s.astype(np.float64)) - 127).repeat_interleave(32, 0)[:n]
        return torch.from_numpy(w).view(F8).double() * sc.repeat_interleave(32, 1)

    xq = quant(x)
    g = (xq @ deq(w1, s1).T).float().bfloat16().double()
    u = (xq @ deq(w3, s3).T).float().bfloat16().double()
    u = u.clamp(-limit, limit)
    g = g.clamp(max=limit)
    h = (torch.nn.functional.silu(g) * u).float().bfloat16().float()
    y = (quant(h.numpy()) @ deq(w2, s2).T).float().bfloat16().float()
    return y.numpy()


def test_shared_expert_matches_torch_composition():
    rng = np.random.default_rng(4)
    d, f = 256, 192
    w1, s1 = _weights(rng, f, d)
    w3, s3 = _weights(rng, f, d)
    w2, s2 = _weights(rng, d, f)
    x = round_bf16(rng.standard_normal((4, d)).astype(np.float32))
    for limit in (10.0, 0.5):
        got = fp8.shared_expert(x, w1, s1, w3, s3, w2, s2, limit=limit)
        want = _torch_shared(x, w1, s1, w3, s3, w2, s2, limit)
        # one bf16 ulp where float64 silu and torch's differ at a rounding boundary
        close = np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-30
        assert close.mean() > 0.999 and np.array_equal(got, round_bf16(got))
