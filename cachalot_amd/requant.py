"""FP4 -> affine requantizer on the GPU (the bank tool's fits).

Mirrors ``benchmarks/quant_affine.py``'s ``quantize_affine(w, group_size, bits, fit,
importance)`` (:303-329) applied to the FP4 checkpoint's dequantized experts, which
is what ``benchmarks/build_affine_bank.py`` does for every expert of a bank
(``quantize_expert`` :162-189; fits ``FITS`` :74-75 -- all but "mlx", MLX's own
quantizer; widths :266-267).  The fit runs in ``cachalot_requant_fp4_to_affine``
(one GPU thread per group); this module moves experts between slots, stores and
shard files.  Activation importance is taken per projection as given: deriving
it from recorded activations (``benchmarks/activation_importance.py``) is the
calibration step before the bank tool, not part of it.
"""
from __future__ import annotations

from pathlib import Path

import torch

from . import _lib
from .storage.index import ExpertFormat, affine_format, detect_expert_bank

PROJS = ("w1", "w2", "w3")
FITS = {"minmax": 0, "search": 1, "search-lsq": 2, "wide-lsq": 3}     # CACHALOT_FIT_*


def fit_code(name: str) -> int:
    try:
        return FITS[name]
    except KeyError:
        raise ValueError(f"unknown fit {name!r} (one of {tuple(FITS)}; MLX's own 'mlx' fit is not offered)") from None


def requantize_fp4_matrix(w_fp4: torch.Tensor, s_fp4: torch.Tensor, k: int, *, bits: int = 2,
                          group_size: int = 128, fit: str = "search", importance: torch.Tensor | None = None,
                          scale_dtype: str = "bfloat16"):
    """w_fp4 uint8 [N, K/2], s_fp4 uint8 [N, K/32] (device) -> (codes int32 [N, Kp*bits/32] (uint32 bits),
    scales int16 [N, Kp/group] (bf16 or fp16 bits, ``scale_dtype``), biases int16) on the same device;
    ``importance`` float32 [K] (device) weights the fit per column."""
    if bits not in (2, 3, 4) or group_size not in (32, 64, 128):
        raise ValueError(f"affine banks have 2, 3 or 4 bits in groups of 32, 64 or 128 "
                         f"(bits={bits}, group_size={group_size})")
    code = fit_code(fit)
    n = w_fp4.shape[0]
    w_fp4 = w_fp4.reshape(n, -1).contiguous()
    s_fp4 = s_fp4.reshape(n, -1).contiguous()
    if w_fp4.shape[1] * 2 != k or s_fp4.shape[1] * 32 != k:
        raise ValueError(f"FP4 tensors {tuple(w_fp4.shape)} / {tuple(s_fp4.shape)} do not hold K={k}")
    _lib.require_cuda(w_fp4, s_fp4)
    imp_ptr = None
    if importance is not None:
        importance = importance.reshape(-1).contiguous()
        if importance.dtype != torch.float32 or importance.numel() != k:
            raise ValueError(f"importance must be float32 [{k}], got {importance.dtype} {tuple(importance.shape)}")
        _lib.require_cuda(importance)
        imp_ptr = importance.data_ptr()
    g = -(-k // group_size)
    dev = w_fp4.device
    q = torch.empty((n, g * group_size * bits // 32), dtype=torch.int32, device=dev)
    s = torch.empty((n, g), dtype=torch.int16, device=dev)
    b = torch.empty((n, g), dtype=torch.int16, device=dev)
    rc = _lib.lib().cachalot_requant_fp4_to_affine(w_fp4.data_ptr(), s_fp4.data_ptr(), n, k, bits, group_size,
                                                   code, imp_ptr, q.data_ptr(), s.data_ptr(), b.data_ptr(),
                                                   _lib.scale_dtype_code(scale_dtype), _lib.stream_handle(dev))
    _lib.check(rc, "requant_fp4_to_affine")
    return q, s, b


def requantize_expert(src: dict[str, torch.Tensor], src_fmt: ExpertFormat, dst: dict[str, torch.Tensor],
                      dst_fmt: ExpertFormat, *, fit: str = "search",
                      importance: dict[str, torch.Tensor] | None = None) -> None:
    """FP4 slot arrays -> affine slot arrays (uint8 views, e.g. ``slot.arrays``) of one expert, at the
    destination format's width, group and scale dtype; ``importance`` maps w1/w2/w3 to float32 [K]."""
    if src_fmt.kind != "fp4" or dst_fmt.kind != "affine":
        raise ValueError("requantize_expert maps an FP4 expert to an affine format")
    if (src_fmt.d_model, src_fmt.d_ff) != (dst_fmt.d_model, dst_fmt.d_ff):
        raise ValueError("source and destination shapes differ")
    for proj in PROJS:
        rows, half_k = src_fmt.shapes[f"{proj}.weight"]
        q, s, b = requantize_fp4_matrix(src[f"{proj}.weight"].view(rows, half_k),
                                        src[f"{proj}.scale"].view(rows, -1), 2 * half_k,
                                        bits=dst_fmt.bits, group_size=dst_fmt.group_size, fit=fit,
                                        importance=None if importance is None else importance[proj],
                                        scale_dtype=dst_fmt.dtypes[f"{proj}.scales"])
        for name, t in ((f"{proj}.weight", q), (f"{proj}.scales", s), (f"{proj}.biases", b)):
            dst[name].view(torch.uint8).copy_(t.view(torch.uint8).reshape(-1))


def requantize_store(src_store, dst_store, keys=None, *, fit: str = "search") -> None:
    """Fill `dst_store` (affine) with the requantized experts of `src_store` (FP4), all on the device."""
    keys = keys if keys is not None else sorted(src_store._items)

    def fill(key, slot):
        requantize_expert(src_store._items[key].arrays, src_store.format, slot.arrays, dst_store.format, fit=fit)

    dst_store.preload(keys, fill)


def build_affine_bank(fp4_path: str | Path, out_path: str | Path, *, bits: int = 2, group_size: int = 128,
                      fit: str = "search", scale_dtype: str = "bfloat16", importance=None, layers=None,
                      device="cuda") -> ExpertFormat:
    """Read an FP4 checkpoint's routed experts, requantize each on the GPU and write the stacked affine
    bank (one shard per layer + config.json) that ``detect_expert_bank`` reads
    (``benchmarks/build_affine_bank.py``'s output layout and options: --bits, --group, --fit).
    ``importance(layer, expert)``, when given, returns the expert's per-projection weights
    ({"w1": float32 [K], ...}, on the device) -- the --importance weighting."""
    from .storage.reader import ExpertReader
    from .storage.writer import StackedShardWriter, write_stacked_config

    src_fmt, index = detect_expert_bank(fp4_path)
    if src_fmt.kind != "fp4":
        raise ValueError(f"{fp4_path} is not an FP4 expert bank")
    fit_code(fit)
    dst_fmt = affine_format(src_fmt.d_model, src_fmt.d_ff, bits=bits, group_size=group_size,
                            scale_dtype=scale_dtype)
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
                requantize_expert(src, src_fmt, dst, dst_fmt, fit=fit,
                                  importance=None if importance is None else importance(layer, e))
                host = {n: t.cpu().numpy() for n, t in dst.items()}
                w.put(e, host)
            w.close()
    write_stacked_config(out, dst_fmt, n_layers, n_experts)
    return dst_fmt
