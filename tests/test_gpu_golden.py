"""The HIP library against the committed golden vectors (tests/golden/*.npz).

Bit-exact: router ids, scores and weights, FP4 and 2-bit dequantization,
act_quant codes and exponents, requantized codes, scales and biases.  The
shared expert within the parity bar (2e-3 of max |want| plus one bf16 ulp).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import bf16_ulp
from oracle.bf16 import bf16_bits_to_f32

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _np(t):
    return t.detach().cpu().numpy()


def _bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)


@pytest.mark.parametrize("variant", ["softplus_asc", "sigmoid_rank"])
def test_router_golden(cuda, variant):
    from cachalot_amd.router import route_topk_rows

    g = _load("router")
    score, order = ("sqrt_softplus", "ascending") if variant == "softplus_asc" else ("sigmoid", "rank")
    idx, w, sc = route_topk_rows(_bf16(g["x"], cuda), _bf16(g["w"], cuda), torch.from_numpy(g["bias"]).to(cuda),
                                 topk=6, route_scale=1.5, score_fn=score, order=order)
    assert np.array_equal(_np(idx), g[f"{variant}_idx"])
    assert np.array_equal(_np(w).view(np.uint32), g[f"{variant}_w"].view(np.uint32))
    assert np.array_equal(_np(sc).view(np.uint32), g[f"{variant}_scores"].view(np.uint32))


def test_dequant_golden(cuda):
    from cachalot_amd import _lib

    g = _load("fp4_dequant")
    n, k = g["packed"].shape[0], g["packed"].shape[1] * 2
    out = torch.empty((n, k), dtype=torch.float32, device=cuda)
    dp, dsc = torch.from_numpy(g["packed"]).to(cuda), torch.from_numpy(g["scales"]).to(cuda)   # held: in use
    _lib.check(_lib.lib().cachalot_dequant_fp4(dp.data_ptr(), dsc.data_ptr(), n, k, 0, out.data_ptr(),
                                               _lib.stream_handle(cuda)))
    assert np.array_equal(_np(out), g["dense"])
    g = _load("q2_dequant")
    k = int(g["k"][0])
    n, row_words = g["w"].shape
    out = torch.empty((n, k), dtype=torch.float32, device=cuda)
    dw = torch.from_numpy(g["w"].view(np.int32)).to(cuda)
    ds = torch.from_numpy(g["scales"].view(np.int16)).to(cuda)
    db = torch.from_numpy(g["biases"].view(np.int16)).to(cuda)
    _lib.check(_lib.lib().cachalot_dequant_q2(dw.data_ptr(), ds.data_ptr(), db.data_ptr(), n, k, row_words,
                                              g["scales"].shape[1], 128, 0, out.data_ptr(), _lib.stream_handle(cuda)))
    assert np.array_equal(_np(out).view(np.uint32), g["dense"].view(np.uint32))


def test_fp8_golden(cuda):
    from cachalot_amd.shared_expert import quantize_fp8_activation, shared_expert_forward_batched

    g = _load("fp8")
    q = quantize_fp8_activation(_bf16(g["x"], cuda))
    assert np.array_equal(_np(q.values), g["q"]) and np.array_equal(_np(q.scales), g["e"])
    dev = {k: torch.from_numpy(g[s]).to(cuda) for k, s in
           (("w1", "w1"), ("w1_scales", "s1"), ("w3", "w3"), ("w3_scales", "s3"), ("w2", "w2"), ("w2_scales", "s2"))}
    y = bf16_bits_to_f32(_np(shared_expert_forward_batched(_bf16(g["xs"], cuda), **dev).view(torch.int16)).view(np.uint16))
    want = bf16_bits_to_f32(g["y"])
    assert np.all(np.abs(y - want) <= 2e-3 * np.abs(want).max() + bf16_ulp(want))


def test_requant_golden(cuda):
    from cachalot_amd.requant import requantize_fp4_matrix

    g = _load("requant")
    q, s, b = requantize_fp4_matrix(torch.from_numpy(g["packed"]).to(cuda), torch.from_numpy(g["scales"]).to(cuda),
                                    g["packed"].shape[1] * 2)
    assert np.array_equal(_np(q).view(np.uint32), g["q"])
    assert np.array_equal(_np(s).view(np.uint16), g["q_scales"])
    assert np.array_equal(_np(b).view(np.uint16), g["q_biases"])
