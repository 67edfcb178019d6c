"""Shared helpers for the GPU parity tests: synthetic banks in HBM and their
oracle twins on the host."""
from __future__ import annotations

import numpy as np

from oracle import synth as osynth
from oracle.affine2 import qmv64
from oracle.fp4 import dequantize_fp4_weight

SEED = 20260917


def make_store(fmt, *, n_layers=1, n_experts=384, keys=None, seed=SEED, n_slots=None, loader=False):
    """A ResidentExpertStore with `keys` (default: every expert) preloaded from the synthetic generator."""
    import torch

    from cachalot_amd.cache.resident_store import ResidentExpertStore, SyntheticLoader

    syn = SyntheticLoader(fmt, seed)
    store = ResidentExpertStore(fmt=fmt, n_slots=n_slots or n_layers * n_experts, n_layers=n_layers,
                                n_experts=n_experts, device="cuda:0", loader=syn if loader else None)
    if keys is None:
        keys = [(la, e) for la in range(n_layers) for e in range(n_experts)]
    store.preload(keys, syn.fill_key)
    store.track_slots()
    torch.cuda.synchronize()
    return store


def oracle_tensors(fmt, layer, expert, seed=SEED):
    if fmt.kind == "fp4":
        specs = osynth.fp4_tensor_specs(fmt.d_model, fmt.d_ff)
    else:
        specs = osynth.q2_tensor_specs(fmt.d_model, fmt.d_ff, fmt.group_size,
                                       scale_dtype=fmt.dtypes.get("w1.scales", "bfloat16"), bits=fmt.bits)
    return osynth.expert_tensors(seed, layer, expert, specs)


def q2_mats(fmt, tensors):
    """(mm1, mm3, mm2): float64 products with W1^T, W3^T, W2^T of one 2-bit expert."""
    g = fmt.group_size
    sd = fmt.dtypes.get("w1.scales", "bfloat16")

    def mm(proj, k):
        w, s, b = tensors[f"{proj}.weight"], tensors[f"{proj}.scales"], tensors[f"{proj}.biases"]
        return lambda x: qmv64(x, w, s, b, k=k, group=g, scale_dtype=sd, bits=fmt.bits)

    return mm("w1", fmt.d_model), mm("w3", fmt.d_model), mm("w2", fmt.d_ff)


def fp4_dense(tensors):
    return tuple(dequantize_fp4_weight(tensors[f"{p}.weight"], tensors[f"{p}.scale"]) for p in ("w1", "w3", "w2"))


def rel_err(got, want) -> float:
    """max |got - want| / max |want|: the relative error the parity bar is stated in."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def bf16_ulp(v) -> np.ndarray:
    """Spacing of bf16 numbers at |v| (8 significant bits)."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def bf16_out_ok(got_bf16, want_total_f32, tol: float) -> bool:
    """A bf16 output against the oracle's fp32 value before the cast: the bar plus
    the cast's own half-ulp rounding, per element."""
    got = np.asarray(got_bf16, np.float64)
    want = np.asarray(want_total_f32, np.float64)
    bound = tol * np.abs(want).max() + 0.5 * bf16_ulp(want)
    return bool(np.all(np.abs(got - want) <= bound))


def bf16_terms_ok(got, want, terms, tol: float) -> bool:
    """Outputs that sum per-expert bf16 casts (the 2-bit path rounds every expert's
    y_e to bf16, ``expert_affine.py:81,149-151``): the bar plus one bf16 ulp per
    expert term, since a different fp32 summation order may move a y_e across a
    rounding boundary."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    slack = np.sum(bf16_ulp(np.asarray(terms, np.float64)), axis=0)
    return bool(np.all(np.abs(got - want) <= tol * np.abs(want).max() + slack))


def term_flips(got, raw, tol: float = 2e-3, what: str = "") -> dict:
    """Per-expert outputs y_e (bf16 values) against the oracle's float64 value of
    the same product before its casts (``swiglu_rows(raw=True)``).

    The reference rounds g, u, h and every y_e to bf16 (``expert_affine.py:65-81,
    149-151``).  A different fp32 summation order can move a value across a
    rounding boundary at any of those points: at y_e itself that is a one-step
    "flip"; at g, u or h it moves every y_e of that expert by a fraction of a
    step.  So each GPU term must lie within half a bf16 step of the raw value
    (its own cast) plus ``tol`` * max|raw|.  Returned: how many terms equal the
    oracle's cast exactly, how many are the adjacent bf16 value ("flips"), how
    many are further ("moved"), and the largest excess over the half step in
    units of max|raw| (``err``: the expert-output error the reference's own
    bf16 cast does not explain)."""
    from oracle.bf16 import round_bf16

    got = np.asarray(got, np.float64)
    raw = np.asarray(raw, np.float64)
    want = round_bf16(raw.astype(np.float32)).astype(np.float64)
    scale = max(float(np.abs(raw).max()), 1e-30)
    excess = np.maximum(np.abs(got - raw) - 0.5 * bf16_ulp(raw), 0.0) / scale
    diff = got != want
    adjacent = np.abs(got - want) <= bf16_ulp(np.maximum(np.abs(got), np.abs(want))) * (1 + 1e-9)
    bad = excess > tol
    assert not bad.any(), (what, f"{int(bad.sum())} terms beyond half a step + {tol} of max|y|",
                           float(excess.max()), got[bad][:4].tolist(), raw[bad][:4].tolist())
    return {"exact": int((~diff).sum()), "flips": int((diff & adjacent).sum()), "moved": int((diff & ~adjacent).sum()),
            "n": int(got.size), "err": float(excess.max())}


def route_order_sum(terms) -> np.ndarray:
    """0 + y_0 + ... + y_{k-1} in fp32 over the first axis (the reference's combine order)."""
    terms = np.asarray(terms, np.float32)
    acc = np.float32(0.0) + terms[0]
    for t in terms[1:]:
        acc = (acc + t).astype(np.float32)
    return acc.astype(np.float32)


def bf16_ulp_dist(a_bf16, b_bf16) -> np.ndarray:
    """Distance in bf16 steps between two arrays of bf16 values (ordered-integer difference)."""
    from oracle.bf16 import f32_to_bf16_bits

    def key(v):
        u = f32_to_bf16_bits(np.asarray(v, np.float32)).astype(np.int32)
        return np.where(u & 0x8000, 0x8000 - (u & 0x7FFF), 0x8000 + u)

    return np.abs(key(a_bf16) - key(b_bf16))


def report(what: str, **fields) -> None:
    """One parity line on stdout (seen with pytest -s and in the smoke output)."""
    print(f"[parity] {what}: " + ", ".join(f"{k}={v}" for k, v in fields.items()), flush=True)
