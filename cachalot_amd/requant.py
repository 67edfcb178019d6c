"""FP4 -> 2-bit affine g128 requantizer on the GPU (the searched fit).

Mirrors ``benchmarks/quant_affine.py``'s ``quantize_affine(w, group_size=128,
bits=2, fit=fit_search)`` (:177-205, :330-359) applied to the FP4 checkpoint's
dequantized experts, which is what ``benchmarks/build_affine_bank.py`` does for
every expert of the bank (:165-189, default fit "search").  The fit runs in
``cachalot_requant_fp4_to_q2`` (one GPU thread per 128-element group); this
module moves experts between slots, stores and shard files.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from . import _lib
from .storage.index import ExpertFormat, affine_format, detect_expert_bank

PROJS = ("w1", "w2", "w3")


def requantize_fp4_matrix(w_fp4: torch.Tensor, s_fp4: torch.Tensor, k: int, *, group_size: int = 128,
                          scale_dtype: str = "bfloat16"):
    """w_fp4 uint8 [N, K/2], s_fp4 uint8 [N, K/32] (device) -> (codes int32 [N, Kp/16] (uint32 bits),
    scales int16 [N, Kp/128] (bf16 or fp16 bits, ``scale_dtype``), biases int16) on the same device."""
    if group_size != 128:
        raise ValueError("the requantizer writes the g128 bank")
    n = w_fp4.shape[0]
    w_fp4 = w_fp4.reshape(n, -1).contiguous()
    s_fp4 = s_fp4.reshape(n, -1).contiguous()
    if w_fp4.shape[1] * 2 != k or s_fp4.shape[1] * 32 != k:
        raise ValueError(f"FP4 tensors {tuple(w_fp4.shape)} / {tuple(s_fp4.shape)} do not hold K={k}")
    _lib.require_cuda(w_fp4, s_fp4)
    g = -(-k // 128)
    dev = w_fp4.device
    q = torch.empty((n, g * 8), dtype=torch.int32, device=dev)
    s = torch.empty((n, g), dtype=torch.int16, device=dev)
    b = torch.empty((n, g), dtype=torch.int16, device=dev)
    rc = _lib.lib().cachalot_requant_fp4_to_q2(w_fp4.data_ptr(), s_fp4.data_ptr(), n, k, q.data_ptr(), s.data_ptr(),
                                               b.data_ptr(), _lib.scale_dtype_code(scale_dtype),
                                               _lib.stream_handle(dev))
    _lib.check(rc, "requant_fp4_to_q2")
    return q, s, b


def requantize_expert(src: dict[str, torch.Tensor], src_fmt: ExpertFormat, dst: dict[str, torch.Tensor],
                      dst_fmt: ExpertFormat) -> None:
    """FP4 slot arrays -> 2-bit slot arrays (uint8 views, e.g. ``slot.arrays``) of one expert."""
    if src_fmt.kind != "fp4" or dst_fmt.kind != "affine" or dst_fmt.bits != 2 or dst_fmt.group_size != 128:
        raise ValueError("requantize_expert maps an FP4 expert to the 2-bit g128 format")
    if (src_fmt.d_model, src_fmt.d_ff) != (dst_fmt.d_model, dst_fmt.d_ff):
        raise ValueError("source and destination shapes differ")
    for proj in PROJS:
        rows, half_k = src_fmt.shapes[f"{proj}.weight"]
        q, s, b = requantize_fp4_matrix(src[f"{proj}.weight"].view(rows, half_k),
                                        src[f"{proj}.scale"].view(rows, -1), 2 * half_k,
                                        scale_dtype=dst_fmt.dtypes[f"{proj}.scales"])
        for name, t in ((f"{proj}.weight", q), (f"{proj}.scales", s), (f"{proj}.biases", b)):
            dst[name].view(torch.uint8).copy_(t.view(torch.uint8).reshape(-1))


def requantize_store(src_store, dst_store, keys=None) -> None:
    """Fill `dst_store` (2-bit) with the requantized experts of `src_store` (FP4), all on the device."""
    keys = keys if keys is not None else sorted(src_store._items)

    def fill(key, slot):
        requantize_expert(src_store._items[key].arrays, src_store.format, slot.arrays, dst_store.format)

    dst_store.preload(keys, fill)


def build_affine_bank(fp4_path: str | Path, out_path: str | Path, *, layers=None, device="cuda") -> ExpertFormat:
    """Read an FP4 checkpoint's routed experts, requantize each on the GPU and write the stacked 2-bit g128
    bank (one shard per layer + config.json) that ``detect_expert_bank`` reads
    (``benchmarks/build_affine_bank.py``'s output layout)."""
    from .storage.reader import ExpertReader
    from .storage.writer import StackedShardWriter, write_stacked_config

    src_fmt, index = detect_expert_bank(fp4_path)
    if src_fmt.kind != "fp4":
        raise ValueError(f"{fp4_path} is not an FP4 expert bank")
    dst_fmt = affine_format(src_fmt.d_model, src_fmt.d_ff)
    out = Path(out_path)
    out.mkdir(parents=True, exist_ok=True)
    all_layers = sorted({k[0] for k in index})
    n_layers = max(all_layers) + 1
    n_experts = max(k[1] for k in index) + 1
    dev = torch.device(device)
    src = {n: torch.empty(src_fmt.tensor_bytes(n), dtype=torch.uint8, device=dev) for n in src_fmt.tensor_names}
    dst = {n: torch.empty(dst_fmt.tensor_bytes(n), dtype=torch.uint8, device=dev) for n in dst_fmt.tensor_names}
    with ExpertReader() as reader:
        for layer in (layers if layers is not None else all_layers):
            w = StackedShardWriter(out, layer, n_layers, n_experts, dst_fmt)
            for e in range(n_experts):
                reader.read_expert_into(index[(layer, e)], src)
                requantize_expert(src, src_fmt, dst, dst_fmt)
                host = {n: t.cpu().numpy() for n, t in dst.items()}
                w.put(e, host)
            w.close()
    write_stacked_config(out, dst_fmt, n_layers, n_experts)
    return dst_fmt
