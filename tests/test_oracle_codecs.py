"""Pins for the oracle's codecs: FP4 E2M1/E8M0, the MLX 2-bit affine layout, bf16.

Each check comes from a source independent of the oracle's own code: the
E2M1 bit-field definition (OCP Microscaling spec), hand-worked bytes and
words, and torch's own bf16 conversion.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.affine2 import dequantize_affine, dequantize_affine64, pack_2bit, qmv64, unpack_2bit
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16
from oracle.fp4 import FP4_E2M1_TABLE, decode_e8m0, dequantize_fp4_weight, unpack_fp4_e2m1


def e2m1_from_bits(code: int) -> float:
    s, e, m = code >> 3, (code >> 1) & 3, code & 1
    mag = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1.0 + m / 2.0)
    return -mag if s else mag


def test_fp4_table_matches_e2m1_bitfield():
    for code in range(16):
        assert FP4_E2M1_TABLE[code] == e2m1_from_bits(code), code


def test_e8m0_known_values():
    got = decode_e8m0(np.array([127, 119, 128, 0, 254], np.uint8))
    assert got.tolist() == [1.0, 2.0 ** -8, 2.0, 2.0 ** -127, 2.0 ** 127]


def test_unpack_low_nibble_first():
    got = unpack_fp4_e2m1(np.array([[0x21, 0xF9, 0x7A]], np.uint8))
    # 0x21: low 1 -> 0.5, high 2 -> 1.0; 0xF9: low 9 -> -0.5, high 15 -> -6; 0x7A: low 10 -> -1, high 7 -> 6
    assert got.tolist() == [[0.5, 1.0, -0.5, -6.0, -1.0, 6.0]]


def test_dequantize_fp4_block_scales_and_errors():
    packed = np.full((2, 32), 0x75, np.uint8)          # low 5 -> 3.0, high 7 -> 6.0
    scales = np.array([[126, 127], [120, 130]], np.uint8)
    w = dequantize_fp4_weight(packed, scales)
    assert w.shape == (2, 64)
    assert w[0, :32].tolist() == [1.5, 3.0] * 16 and w[0, 32:].tolist() == [3.0, 6.0] * 16
    assert w[1, 0] == 3.0 * 2.0 ** -7 and w[1, 63] == 6.0 * 8.0
    with pytest.raises(ValueError):
        dequantize_fp4_weight(packed, scales[:, :1])
    with pytest.raises(ValueError):
        dequantize_fp4_weight(np.zeros((1, 8), np.uint8), np.zeros((1, 1), np.uint8))


def test_pack_2bit_known_words():
    q = np.zeros(16, np.uint8)
    q[0] = 1
    assert pack_2bit(q).tolist() == [1]
    q = np.zeros(16, np.uint8)
    q[15] = 3
    assert pack_2bit(q).tolist() == [3 << 30]
    q = np.array([0, 1, 2, 3] * 4, np.uint8)
    # fields 2i hold q_i: 0b11100100 repeated per byte
    assert pack_2bit(q).tolist() == [0xE4E4E4E4]
    with pytest.raises(ValueError):
        pack_2bit(np.zeros(10, np.uint8))


def test_unpack_2bit_roundtrip():
    rng = np.random.default_rng(3)
    q = rng.integers(0, 4, size=(5, 64), dtype=np.uint8)
    assert np.array_equal(unpack_2bit(pack_2bit(q)), q)
    assert np.array_equal(unpack_2bit(pack_2bit(q), 40), q[:, :40])


def test_dequantize_affine_elementwise():
    rng = np.random.default_rng(4)
    q = rng.integers(0, 4, size=(3, 48), dtype=np.uint8)
    s = f32_to_bf16_bits(rng.uniform(0.005, 0.05, size=(3, 3)).astype(np.float32))
    b = f32_to_bf16_bits(rng.normal(0, 0.02, size=(3, 3)).astype(np.float32))
    w = pack_2bit(q)
    got = dequantize_affine(w, s, b, k=40, group=16)
    sf, bf = bf16_bits_to_f32(s), bf16_bits_to_f32(b)
    for n in range(3):
        for k in range(40):
            want = np.float32(np.float32(sf[n, k // 16] * np.float32(q[n, k])) + bf[n, k // 16])
            assert got[n, k] == want
    # the float64 form equals the exact value of s*q+b
    got64 = dequantize_affine64(w, s, b, k=40, group=16)
    assert got64[1, 17] == float(sf[1, 1]) * int(q[1, 17]) + float(bf[1, 1])


def test_qmv64_group_formula_with_partial_last_group():
    """sum_g s_g * sum(x q) + b_g * sum(x) over a K that ends mid-group."""
    rng = np.random.default_rng(5)
    n, k, group = 4, 40, 16
    q = rng.integers(0, 4, size=(n, 48), dtype=np.uint8)
    q[:, k:] = 0
    s = f32_to_bf16_bits(rng.uniform(0.005, 0.05, size=(n, 3)).astype(np.float32))
    b = f32_to_bf16_bits(rng.normal(0, 0.02, size=(n, 3)).astype(np.float32))
    x = round_bf16(rng.normal(size=(2, k)).astype(np.float32))
    got = qmv64(x, pack_2bit(q), s, b, k=k, group=group)
    sf, bf = bf16_bits_to_f32(s).astype(float), bf16_bits_to_f32(b).astype(float)
    for m in range(2):
        for r in range(n):
            total = 0.0
            for g in range(3):
                lo, hi = g * group, min(k, (g + 1) * group)
                xq = sum(float(x[m, i]) * int(q[r, i]) for i in range(lo, hi))
                xs = sum(float(x[m, i]) for i in range(lo, hi))
                total += sf[r, g] * xq + bf[r, g] * xs
            assert abs(got[m, r] - total) <= 1e-12 * max(1.0, abs(total))


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(6)
    vals = np.concatenate([
        rng.normal(size=20000).astype(np.float32),
        (rng.normal(size=2000) * 1e-30).astype(np.float32),
        # exact ties: mantissa ends in 0x8000
        (np.arange(1, 2001, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38], np.float32),
    ])
    want = torch.from_numpy(vals).to(torch.bfloat16).float().numpy()
    got = round_bf16(vals)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_fp16_scale_values_known_bits():
    """fp16 scale / bias storage (the oQ3e banks): IEEE half bits,
    subnormals included; bf16 bits are the high half of an fp32."""
    from oracle.affine2 import scale_values

    got = scale_values(np.array([0x3C00, 0xC000, 0x0001, 0x3555, 0x7BFF], np.uint16), "float16")
    assert got.tolist() == [1.0, -2.0, 2.0 ** -24, 0.333251953125, 65504.0]
    assert scale_values(np.array([0x3F80, 0xBF00], np.uint16)).tolist() == [1.0, -0.5]
    with pytest.raises(ValueError):
        scale_values(np.array([0], np.uint16), "float32")


def test_dequantize_affine_fp16_known_words():
    from oracle.affine2 import dequantize_affine, pack_2bit

    q = np.tile(np.arange(4, dtype=np.uint8), 4)[None, :]          # 0 1 2 3 0 1 2 3 ...
    w = pack_2bit(q)
    s = np.array([[0x3800]], np.uint16)                              # 0.5
    b = np.array([[0xBC00]], np.uint16)                              # -1.0
    got = dequantize_affine(w, s, b, k=16, group=16, scale_dtype="float16")
    assert got[0, :4].tolist() == [-1.0, -0.5, 0.0, 0.5]


def test_requant_fp16_rounds_the_same_fit():
    """The fp16 bank's (scale, bias) are the RNE-to-fp16 of the searched fit the bf16
    bank rounds to bf16; codes follow the rounded pair; a constant group's fp16 scale
    rounds to zero and its codes are 0 (its bias then equals the constant)."""
    from oracle import requant as orq
    from oracle.affine2 import dequantize_affine

    rng = np.random.default_rng(3)
    dense = (rng.standard_normal((6, 256)) * 0.05).astype(np.float32)
    dense[5, 128:] = 0.25                                             # one constant group
    g = dense.reshape(-1, 128)
    s, b = orq.fit_search(g, np.ones_like(g, bool))
    q16, s16, b16 = orq.requantize(dense, scale_dtype="float16")
    assert np.array_equal(s16.reshape(-1), s.reshape(-1).astype(np.float16).view(np.uint16))
    assert np.array_equal(b16.reshape(-1), b.reshape(-1).astype(np.float16).view(np.uint16))
    assert s16.reshape(-1)[-1] == 0 and not (q16.reshape(6, -1)[5, 8:]).any()
    back = dequantize_affine(q16, s16, b16, k=256, group=128, scale_dtype="float16")
    assert np.array_equal(back[5, 128:], dense[5, 128:])
    # fp16 keeps 3 more significand bits than bf16: the fit's error is no larger on average
    qb, sb, bb = orq.requantize(dense)
    err16 = np.abs(back - dense).mean()
    errb = np.abs(dequantize_affine(qb, sb, bb, k=256, group=128) - dense).mean()
    assert err16 <= errb * 1.01


def test_fp16_synthetic_kinds_follow_the_bf16_stream():
    """The fp16 fill kinds draw the same fp32 values as the bf16 kinds and round them
    to half precision: each pair lies within one bf16 step of each other."""
    from oracle import synth as osynth
    from oracle.affine2 import scale_values

    key = osynth.stream_key(5, 1, 2, 3)
    for kb, kf, p0, p1 in ((osynth.KIND_BF16_UNIFORM, osynth.KIND_F16_UNIFORM, 0.005, 0.045),
                           (osynth.KIND_BF16_NORMAL, osynth.KIND_F16_NORMAL, 0.02, 0.0)):
        vb = scale_values(osynth.fill(kb, 4000, key, p0, p1))
        vf = scale_values(osynth.fill(kf, 4000, key, p0, p1), "float16")
        assert np.all(np.abs(vb - vf) <= np.abs(vb) * 2.0 ** -8 + 2.0 ** -24)
        assert not np.array_equal(vb, vf)


def test_pack_bits_3bit_known_words():
    """MLX's 3-bit layout (quant_affine.py:69-105): one little-endian bit stream, code i
    at bits [3i, 3i+3); code 10 straddles words 0 and 1 (bits 30..32)."""
    from oracle.affine2 import pack_bits, unpack_bits

    q = np.zeros(32, np.uint8)
    q[0], q[1], q[10], q[11], q[31] = 7, 5, 6, 1, 3
    w = pack_bits(q, 3)
    assert w.shape == (3,)
    # word 0: 7 | 5 << 3 | (6 & 3) << 30 ; word 1: 6 >> 2 = 1 in bit 0, code 11 at bits 1..3
    assert int(w[0]) == (7 | (5 << 3) | ((6 & 3) << 30))
    assert int(w[1]) == (1 | (1 << 1))
    assert int(w[2]) == 3 << 29                     # code 31 at stream bits 93..95
    assert np.array_equal(unpack_bits(w, 3), q)


def test_pack_bits_round_trip_and_2bit_agreement():
    from oracle.affine2 import pack_2bit, pack_bits, unpack_bits

    rng = np.random.default_rng(4)
    for bits in (2, 3, 4):
        q = rng.integers(0, 1 << bits, size=(5, 256), dtype=np.uint8)
        w = pack_bits(q, bits)
        assert w.shape == (5, 256 * bits // 32)
        assert np.array_equal(unpack_bits(w, bits), q)
    q = rng.integers(0, 4, size=(3, 128), dtype=np.uint8)
    assert np.array_equal(pack_bits(q, 2), pack_2bit(q))
    # 4-bit: eight codes per word, low nibble first (byte-aligned, so also the nibble order)
    q = np.arange(8, dtype=np.uint8)
    assert int(pack_bits(q, 4)[0]) == 0x76543210


def test_affine_widths_qmv_equals_dense_product():
    """3-bit g64 with fp16 scales (oQ3e) and 4-bit g32: the group formula equals the
    dense product of the dequantised matrix."""
    from oracle.affine2 import dequantize_affine, dequantize_affine64, pack_bits, qmv64

    rng = np.random.default_rng(5)
    for bits, group, sd in ((3, 64, "float16"), (4, 32, "bfloat16")):
        n, k = 12, 160                                  # 2.5 groups of 64, 5 of 32
        kp = -(-k // group) * group
        q = rng.integers(0, 1 << bits, size=(n, kp), dtype=np.uint8)
        q[:, k:] = 0
        w = pack_bits(q, bits)
        s = rng.uniform(0.005, 0.05, size=(n, kp // group)).astype(np.float32)
        b = rng.normal(0, 0.02, size=(n, kp // group)).astype(np.float32)
        if sd == "float16":
            sb, bb = s.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
            sv, bv = sb.view(np.float16).astype(np.float64), bb.view(np.float16).astype(np.float64)
        else:
            sb, bb = f32_to_bf16_bits(s), f32_to_bf16_bits(b)
            sv, bv = bf16_bits_to_f32(sb).astype(np.float64), bf16_bits_to_f32(bb).astype(np.float64)
        dense = q[:, :k] * np.repeat(sv, group, axis=1)[:, :k] + np.repeat(bv, group, axis=1)[:, :k]
        assert np.array_equal(dequantize_affine64(w, sb, bb, k=k, group=group, scale_dtype=sd, bits=bits), dense)
        x = rng.normal(size=(3, k))
        assert np.allclose(qmv64(x, w, sb, bb, k=k, group=group, scale_dtype=sd, bits=bits), x @ dense.T,
                           rtol=1e-12, atol=1e-12)
        f32 = dequantize_affine(w, sb, bb, k=k, group=group, scale_dtype=sd, bits=bits)
        assert np.array_equal(f32, (q[:, :k].astype(np.float32) * np.repeat(sv, group, axis=1)[:, :k].astype(
            np.float32)) + np.repeat(bv, group, axis=1)[:, :k].astype(np.float32))
