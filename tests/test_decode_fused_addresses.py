"""Bounds of every global address the one-launch 2-bit decode kernel forms.

A CPU mirror of the index arithmetic of ``q2_decode_fused_kernel``
(cachalot_amd/csrc/decode_q2_fused.hip) and of its host envelope
(``q2_fused_grid``): for every shape the envelope accepts at 256 workgroups, every
workgroup / wave / lane / item must address inside its tensor.  Workgroups without
gate/up or down items are the case that once read uninitialised item tables."""
from __future__ import annotations

import pytest

WAVES, PUB, DN_WAVES = 16, 15, 15
MAX_T, MAX_TD, MAX_GU, MAX_DN = 6, 2, 48, 60


def _envelope(D, F, k, G):
    TT, TD = k * (F // 16), D // 16
    max_t, max_td = -(-TT // G), -(-TD // G)
    NQ, NQ2 = D // 512, (-(-F // 128) + 3) // 4
    return (D % 1024 == 0 and D <= 5120 and F % 64 == 0 and F <= 3072 and 1 <= k <= 8 and max_t <= MAX_T
            and max_td <= MAX_TD and -(-max_t * NQ // WAVES) <= 3 and -(-max_td * k * NQ2 // DN_WAVES) <= 4)


def _out_of_bounds(D, F, k, G, eslot):
    GT, GK = D // 128, -(-F // 128)
    NQ, NQ2, FT = GT // 4, (GK + 3) // 4, F // 16
    size = {0: F * GT * 32, 1: F * GT * 2, 2: F * GT * 2, 3: D * GK * 32, 4: D * GK * 2, 5: D * GK * 2,
            6: F * GT * 32, 7: F * GT * 2, 8: F * GT * 2}
    TT, TD = k * FT, D // 16
    tpw = -(-TT // G)
    MAXGU, MAXDN = -(-tpw * NQ // WAVES), -(-(-(-TD // G)) * k * NQ2 // DN_WAVES)
    bad = 0
    for b in range(G):
        t0 = min(b * tpw, TT)
        nt = min(t0 + tpw, TT) - t0
        d0, d1 = TD * b // G, TD * (b + 1) // G
        ntd = d1 - d0
        n_gu, n_dn = nt * NQ, ntd * k * NQ2
        assert nt <= MAX_T and ntd <= MAX_TD and n_gu <= MAX_GU and n_dn <= MAX_DN
        gu_tl = [t // NQ if t < n_gu else 0 for t in range(MAX_GU)]
        gu_q = [t % NQ if t < n_gu else 0 for t in range(MAX_GU)]
        t_e = [(t0 + t) // FT if t < nt else 0 for t in range(MAX_T)]
        t_p = [(t0 + t) % FT if t < nt else 0 for t in range(MAX_T)]
        dn_tdl = [t // (k * NQ2) if t < n_dn else 0 for t in range(MAX_DN)]
        dn_e = [(t // NQ2) % k if t < n_dn else 0 for t in range(MAX_DN)]
        dn_q2 = [t % NQ2 if t < n_dn else 0 for t in range(MAX_DN)]
        for wave in range(WAVES):
            if n_gu > 0:
                for m in range(MAXGU):
                    it = min(wave + WAVES * m, n_gu - 1)
                    tl, q = gu_tl[it], gu_q[it]
                    row0 = t_p[tl] * 16
                    for lane in range(64):
                        j, kg = lane & 15, lane >> 4
                        o = ((row0 + (lane & 15)) * GT + 4 * q) * 2
                        bad += (o & ~15) + 16 > size[(1, 2, 7, 8)[lane >> 4]]
                        bad += (row0 + j) * (D // 4) + (4 * q + kg) * 32 + 32 > size[0]
            if wave != PUB and n_dn > 0:
                for m in range(MAXDN):
                    it = min(wave + DN_WAVES * m, n_dn - 1)
                    tdl, q2 = dn_tdl[it], dn_q2[it]
                    for lane in range(64):
                        j, kg = lane & 15, lane >> 4
                        g2 = min(4 * q2 + kg, GK - 1)
                        n = min(d0 + tdl, TD - 1) * 16 + j
                        bad += n * GK * 32 + g2 * 32 + 32 > size[3]
                        bad += (n * GK + g2) * 2 + 2 > size[4]
        for tl in range(nt):   # publication: plane blocks of the tile's group, zero pieces included
            bad += (t_e[tl] * GK + (t_p[tl] >> 3) + 1) * 320 > k * GK * 320
        bad += any((d0 + t // 16) * 16 + (t & 15) >= D for t in range(ntd * 16))
    return bad


@pytest.mark.parametrize("D,F", [(4096, 2880), (5120, 2304), (4096, 3072), (2048, 1408), (1024, 512)])
@pytest.mark.parametrize("k", [1, 2, 3, 6, 8])
def test_fused_decode_addresses_in_bounds(D, F, k):
    G = 256
    if not _envelope(D, F, k, G):
        pytest.skip("outside the one-launch envelope (two-kernel path)")
    assert _out_of_bounds(D, F, k, G, [0] * k) == 0
