"""GPU requantizer (FP4 -> affine at every width and fit of the bank tool) against oracle/requant.py.

The oracle evaluates the fit in float32 with the error summed in index order,
the order the kernel uses, so codes, scales and biases must match bit for bit.
Sources are the seeded synthetic FP4 experts (uniform nibbles, many exact ties
between candidates) and FP4-rounded Gaussian weights.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import oracle_tensors
from oracle import requant as orq
from oracle.fp4 import dequantize_fp4_weight
from cachalot_amd.storage import index as I

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _check_matrix(cuda, w, s, scale_dtype="bfloat16"):
    from cachalot_amd.requant import requantize_fp4_matrix

    k = w.shape[1] * 2
    q, sc, bi = requantize_fp4_matrix(torch.from_numpy(w).to(cuda), torch.from_numpy(s).to(cuda), k,
                                      scale_dtype=scale_dtype)
    wq, ws, wb = orq.requantize(dequantize_fp4_weight(w, s).astype(np.float32), scale_dtype=scale_dtype)
    assert np.array_equal(_np(q).view(np.uint32), wq)
    assert np.array_equal(_np(sc).view(np.uint16), ws)
    assert np.array_equal(_np(bi).view(np.uint16), wb)


@pytest.mark.parametrize("proj,scale_dtype", [("w1", "bfloat16"), ("w2", "bfloat16"), ("w2", "float16")])
def test_requant_matrix_bit_exact_synthetic(cuda, proj, scale_dtype):
    fmt = I.fp4_format(1024, 2880)                   # w2: K = 2880, a partial last group
    t = oracle_tensors(fmt, 0, 3)
    rows = 640 if proj == "w1" else 512
    _check_matrix(cuda, t[f"{proj}.weight"][:rows], t[f"{proj}.scale"][:rows], scale_dtype)


def _gaussian_fp4(rng, n, k):
    """FP4-encode Gaussian weights: per 32-block scale 2^ceil(log2(amax/6)), nearest E2M1 code."""
    dense = rng.standard_normal((n, k)) * rng.uniform(0.01, 1.0, size=(n, 1))
    blocks = dense.reshape(n, k // 32, 32)
    e = np.ceil(np.log2(np.abs(blocks).max(-1) / 6.0)).astype(np.int32)
    grid = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6])
    mag = np.abs(blocks) / np.exp2(e)[..., None]
    code = np.abs(mag[..., None] - grid).argmin(-1) | (np.signbit(blocks) << 3)
    code = code.reshape(n, k).astype(np.uint8)
    w = (code[:, 0::2] | (code[:, 1::2] << 4)).astype(np.uint8)
    s = (e + 127).astype(np.uint8)
    return w, s


def test_requant_matrix_bit_exact_gaussian(cuda):
    w, s = _gaussian_fp4(np.random.default_rng(9), 256, 1024)
    _check_matrix(cuda, w, s)
    _check_matrix(cuda, w, s, "float16")
    w[:4] = 0                                        # constant groups: the fp16 scale rounds to zero, codes 0
    _check_matrix(cuda, w, s, "float16")


_WIDTHS = [(b, g, f) for b in (2, 3, 4) for g in (32, 64, 128) for f in orq.FITS]


@pytest.mark.parametrize("bits,group,fit", _WIDTHS)
def test_requant_widths_and_fits_bit_exact(cuda, bits, group, fit):
    """Every width x group x fit of the bank tool, bit for bit; K = 1056 leaves a partial last group at
    g64 and g128.  Cases alternate the scale dtype and the importance weighting (zero over the first
    32 columns -- a whole g32 group with a zero weight total -- and over every seventh column)."""
    from cachalot_amd.requant import requantize_fp4_matrix

    i = _WIDTHS.index((bits, group, fit))
    rng = np.random.default_rng(100 + i)
    n, k = 96, 1056
    w, s = _gaussian_fp4(rng, n, k)
    scale_dtype = "float16" if i % 2 else "bfloat16"
    imp = None
    if i % 3 != 2:
        imp = rng.uniform(0.05, 4.0, k).astype(np.float32)
        imp[:32] = 0.0
        imp[::7] = 0.0
    print(f"requant case bits={bits} group={group} fit={fit} {scale_dtype} importance={imp is not None}", flush=True)
    q, sc, bi = requantize_fp4_matrix(torch.from_numpy(w).to(cuda), torch.from_numpy(s).to(cuda), k, bits=bits,
                                      group_size=group, fit=fit, scale_dtype=scale_dtype,
                                      importance=None if imp is None else torch.from_numpy(imp).to(cuda))
    wq, ws, wb = orq.requantize(dequantize_fp4_weight(w, s).astype(np.float32), group, scale_dtype, bits=bits,
                                fit_name=fit, importance=imp)
    assert np.array_equal(_np(sc).view(np.uint16), ws)
    assert np.array_equal(_np(bi).view(np.uint16), wb)
    assert np.array_equal(_np(q).view(np.uint32), wq)


def test_requant_rejects_bad_arguments(cuda):
    from cachalot_amd.requant import requantize_fp4_matrix

    w, s = _gaussian_fp4(np.random.default_rng(1), 8, 256)
    wt, st = torch.from_numpy(w).to(cuda), torch.from_numpy(s).to(cuda)
    with pytest.raises(ValueError):
        requantize_fp4_matrix(wt, st, 256, bits=5)
    with pytest.raises(ValueError):
        requantize_fp4_matrix(wt, st, 256, fit="mlx")
    with pytest.raises(ValueError):
        requantize_fp4_matrix(wt, st, 256, importance=torch.ones(128, device=cuda))


def test_build_affine_bank_other_width(cuda, tmp_path):
    """build_affine_bank at 3-bit g64 fp16 with the wide-lsq fit and importance reads back as that bank."""
    from cachalot_amd.requant import build_affine_bank
    from cachalot_amd.storage.reader import preload_bank
    from cachalot_amd.storage.writer import write_fp4_shard
    from cachalot_amd.cache.resident_store import ResidentExpertStore

    src_fmt = I.fp4_format(512, 320)
    (tmp_path / "fp4").mkdir()
    write_fp4_shard(tmp_path / "fp4" / "model-00001-of-00001.safetensors",
                    {(0, e): oracle_tensors(src_fmt, 0, e) for e in range(2)})
    rng = np.random.default_rng(5)
    imps = {(0, e): {p: rng.uniform(0.1, 2.0, 512 if p != "w2" else 320).astype(np.float32)
                     for p in ("w1", "w2", "w3")} for e in range(2)}
    build_affine_bank(tmp_path / "fp4", tmp_path / "q3", bits=3, group_size=64, fit="wide-lsq",
                      scale_dtype="float16", device=cuda,
                      importance=lambda la, e: {p: torch.from_numpy(v).to(cuda) for p, v in imps[(la, e)].items()})
    fmt, index = I.detect_expert_bank(tmp_path / "q3")
    assert (fmt.bits, fmt.group_size, fmt.dtypes["w1.scales"]) == (3, 64, "float16")
    store = ResidentExpertStore(fmt=fmt, n_slots=2, n_layers=1, n_experts=2, device=cuda)
    preload_bank(store, index)
    for e in range(2):
        t = oracle_tensors(src_fmt, 0, e)
        slot = store.pool.slot(store.layer_table(0)[e].item())
        for p in ("w1", "w2", "w3"):
            q, sb, bb = orq.requantize(dequantize_fp4_weight(t[f"{p}.weight"], t[f"{p}.scale"]).astype(np.float32),
                                       64, "float16", bits=3, fit_name="wide-lsq", importance=imps[(0, e)][p])
            for name, arr in ((f"{p}.weight", q), (f"{p}.scales", sb), (f"{p}.biases", bb)):
                assert np.array_equal(_np(slot.arrays[name]), arr.view(np.uint8).reshape(-1)), (e, name)


def test_requantize_store_and_bank_file(cuda, tmp_path):
    from cachalot_amd.requant import build_affine_bank, requantize_store
    from cachalot_amd.storage.reader import preload_bank
    from cachalot_amd.storage.writer import write_fp4_shard
    from cachalot_amd.cache.resident_store import ResidentExpertStore
    from helpers import make_store

    src_fmt = I.fp4_format(1024, 640)
    src = make_store(src_fmt, n_layers=1, n_experts=4)
    dst = ResidentExpertStore(fmt=I.affine_format(1024, 640), n_slots=4, n_layers=1, n_experts=4, device=cuda)
    requantize_store(src, dst)
    torch.cuda.synchronize()
    want = {}
    for e in range(4):
        t = oracle_tensors(src_fmt, 0, e)
        want[e] = {}
        for p in ("w1", "w2", "w3"):
            q, sb, bb = orq.requantize(dequantize_fp4_weight(t[f"{p}.weight"], t[f"{p}.scale"]).astype(np.float32))
            want[e].update({f"{p}.weight": q, f"{p}.scales": sb, f"{p}.biases": bb})
        slot = dst.pool.slot(dst.layer_table(0)[e].item())
        for name, arr in want[e].items():
            assert np.array_equal(_np(slot.arrays[name]), arr.view(np.uint8).reshape(-1)), (e, name)
    # the same through files: FP4 shard -> build_affine_bank -> detect -> preload
    (tmp_path / "fp4").mkdir()
    write_fp4_shard(tmp_path / "fp4" / "model-00001-of-00001.safetensors",
                    {(0, e): oracle_tensors(src_fmt, 0, e) for e in range(4)})
    build_affine_bank(tmp_path / "fp4", tmp_path / "q2", device=cuda)
    fmt, index = I.detect_expert_bank(tmp_path / "q2")
    store = ResidentExpertStore(fmt=fmt, n_slots=4, n_layers=1, n_experts=4, device=cuda)
    preload_bank(store, index)
    for e in range(4):
        slot = store.pool.slot(store.layer_table(0)[e].item())
        for name, arr in want[e].items():
            assert np.array_equal(_np(slot.arrays[name]), arr.view(np.uint8).reshape(-1)), (e, name)
