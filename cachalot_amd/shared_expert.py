"""The FP8 shared expert and FP8 linear (E4M3FN weights, E8M0 block-32 scales).

Mirrors the reference's call surface:

* ``quantize_fp8_activation(x) -> QuantizedActivation``
  (``src/cachalot/model/fp8_linear_metal.py:30-53``): per 32-element block,
  ``amax = max(|x|, 1e-4)``, scale ``2^ceil(log2(amax / 448))``, E4M3 codes by
  round to nearest even.  ``values`` are the E4M3 bytes (uint8) and ``scales``
  the E8M0 exponent bytes (uint8, scale = 2^(byte - 127)); the reference keeps
  float32 scales, the same powers of two.
* ``fp8_linear_quantized`` / ``fp8_linear`` (``:56-107``): bf16 output.
* ``shared_expert_forward`` / ``shared_expert_forward_fused``
  (``shared_expert_metal.py:44-188``, one token) and
  ``shared_expert_forward_batched`` (``moe_prefill_batched.py:104-125``, rows):
  ``g = bf16(w1 q)``, ``u = bf16(w3 q)``, clamp, ``h = bf16(silu(g) u)``,
  ``y = bf16(w2 act_quant(h))``.  One device call computes the whole expert
  (w1 and w3 are read by one launch, so there is no concatenated ``w13`` to build).

Weights are device tensors: ``w`` uint8 ``[N, K]`` (E4M3 bytes, or a
``torch.float8_e4m3fn`` tensor, viewed as bytes) and ``scales`` uint8
``[ceil(N/32), K/32]``.
"""
from __future__ import annotations

import os

from dataclasses import dataclass

import torch

from . import _lib

BLOCK = 32

_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Scratch per (device, stream): calls on one stream are ordered, calls on two streams may overlap."""
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def _bytes(w: torch.Tensor, name: str) -> torch.Tensor:
    if w.dtype == torch.float8_e4m3fn:
        w = w.view(torch.uint8)
    if w.dtype != torch.uint8 or w.ndim != 2:
        raise ValueError(f"{name} must be a 2D uint8 (E4M3 bytes) tensor, got {w.dtype} {tuple(w.shape)}")
    return w.contiguous()


def _check_weight(w: torch.Tensor, s: torch.Tensor, name: str) -> tuple[torch.Tensor, torch.Tensor]:
    w = _bytes(w, name)
    n, k = w.shape
    if k % BLOCK:
        raise ValueError(f"{name}: K={k} is not divisible by {BLOCK}")
    want = (-(-n // BLOCK), k // BLOCK)
    if s.dtype != torch.uint8 or tuple(s.shape) != want:
        raise ValueError(f"{name} scales {s.dtype} {tuple(s.shape)} != uint8 {want}")
    _lib.require_cuda(w, s)
    return w, s.contiguous()


@dataclass
class QuantizedActivation:
    values: torch.Tensor      # uint8 E4M3 codes, x's shape
    scales: torch.Tensor      # uint8 E8M0 bytes, [..., K / 32]
    in_features: int


def quantize_fp8_activation(x: torch.Tensor) -> QuantizedActivation:
    """x [K] or [M, K] bf16 -> E4M3 codes and E8M0 block exponents (act_quant)."""
    if x.ndim not in (1, 2):
        raise ValueError(f"FP8 activation must be 1D or 2D, got {tuple(x.shape)}")
    if x.dtype != torch.bfloat16:
        raise TypeError("FP8 activation quantization expects bf16 input")
    _lib.require_cuda(x)
    k = x.shape[-1]
    if k % BLOCK:
        raise ValueError(f"K={k} must be divisible by block_size={BLOCK}")
    x2 = x.reshape(-1, k).contiguous()
    m = x2.shape[0]
    q = torch.empty((m, k), dtype=torch.uint8, device=x.device)
    s = torch.empty((m, k // BLOCK), dtype=torch.uint8, device=x.device)
    rc = _lib.lib().cachalot_fp8_act_quant(x2.data_ptr(), m, k, q.data_ptr(), s.data_ptr(),
                                           _lib.stream_handle(x.device))
    _lib.check(rc, "fp8_act_quant")
    return QuantizedActivation(q.reshape(x.shape), s.reshape(*x.shape[:-1], k // BLOCK), k)


def fp8_linear_quantized(x: QuantizedActivation, weight: torch.Tensor, weight_scales: torch.Tensor) -> torch.Tensor:
    """bf16 [..., N] = the block-scaled FP8 product of a quantized activation and E4M3 weights."""
    weight, weight_scales = _check_weight(weight, weight_scales, "weight")
    n, k = weight.shape
    if k != x.in_features:
        raise ValueError(f"weight expects {k} inputs, quantized activation has {x.in_features}")
    q = x.values.reshape(-1, k).contiguous()
    s = x.scales.reshape(-1, k // BLOCK).contiguous()
    m = q.shape[0]
    y = torch.empty((m, n), dtype=torch.bfloat16, device=q.device)
    rc = _lib.lib().cachalot_fp8_linear_quantized(q.data_ptr(), s.data_ptr(), weight.data_ptr(),
                                                  weight_scales.data_ptr(), m, k, n, y.data_ptr(),
                                                  _lib.stream_handle(q.device))
    _lib.check(rc, "fp8_linear_quantized")
    return y.reshape(*x.values.shape[:-1], n)


def fp8_linear(x: torch.Tensor, weight: torch.Tensor, weight_scales: torch.Tensor) -> torch.Tensor:
    return fp8_linear_quantized(quantize_fp8_activation(x), weight, weight_scales)


# moe_prefill_batched.py:28: CACHALOT_PREFILL_BF16_GEMM picks the operand dtype of the
# reference's dense FP8 row GEMMs; the kernels here take the E4M3 bytes directly.
PREFILL_BF16_GEMM = os.environ.get("CACHALOT_PREFILL_BF16_GEMM", "1") != "0"


def gemm_dtype() -> torch.dtype:
    """The dtype the reference dequantizes FP8 operands to for its row GEMMs (``moe_prefill_batched.py:88-89``)."""
    return torch.bfloat16 if PREFILL_BF16_GEMM else torch.float32


def _e8m0_values(s: torch.Tensor) -> torch.Tensor:
    """E8M0 bytes -> float32 2^(s - 127), built from the bits (exact; 0 -> 2^-127, 255 -> NaN)."""
    b = s.to(torch.int32)
    bits = torch.where(b == 0, torch.full_like(b, 0x00400000), b << 23)
    bits = torch.where(b == 255, torch.full_like(b, 0x7FC00000), bits)
    return bits.view(torch.float32)


def quantize_activation_fp8_rows(x: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """x [M, K] bf16 -> act_quant per 32-element block, returned dequantized in ``dtype``
    (E4M3 value x its power-of-two scale, exact in bf16 and fp32;
    ``moe_prefill_batched.py:62-73``).  The codes come from the act_quant kernel."""
    if x.ndim != 2:
        raise ValueError(f"x must be [rows, K], got {tuple(x.shape)}")
    qa = quantize_fp8_activation(x)
    m, k = x.shape
    vals = qa.values.view(torch.float8_e4m3fn).to(torch.float32).reshape(m, k // BLOCK, BLOCK)
    return (vals * _e8m0_values(qa.scales)[..., None]).reshape(m, k).to(dtype)


def dequantize_fp8_weight(weight: torch.Tensor, weight_scales: torch.Tensor,
                          dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """E4M3 weight [N, K] (uint8 or float8_e4m3fn) and E8M0 scales [ceil(N/32), K/32] -> [N, K]
    in ``dtype`` (exact; ``moe_prefill_batched.py:76-84``): row block n // 32, column block k // 32."""
    w = _bytes(weight, "weight")
    n, k = w.shape
    if k % BLOCK or tuple(weight_scales.shape) != ((n + BLOCK - 1) // BLOCK, k // BLOCK):
        raise ValueError(f"scales {tuple(weight_scales.shape)} do not match weight {(n, k)}")
    vals = w.contiguous().view(torch.float8_e4m3fn).to(torch.float32)
    sc = _e8m0_values(weight_scales.to(w.device))
    sc = sc.repeat_interleave(BLOCK, dim=0)[:n].repeat_interleave(BLOCK, dim=1)
    return (vals * sc).to(dtype)


def fp8_linear_rows(x: torch.Tensor, weight: torch.Tensor, weight_scales: torch.Tensor) -> torch.Tensor:
    """x [T, K] bf16 -> bf16 [T, N], the FP8 GEMM of the reference's prefill rows
    (``moe_prefill_batched.py:92-96``): act_quant rows times E4M3 weights, exact products
    accumulated in fp32, one bf16 cast."""
    if x.ndim != 2:
        raise ValueError(f"x must be [rows, K], got {tuple(x.shape)}")
    return fp8_linear(x, weight, weight_scales)


def _shared(x: torch.Tensor, w1, s1, w2, s2, w3, s3, swiglu_limit: float) -> torch.Tensor:
    if x.dtype != torch.bfloat16:
        raise TypeError("the shared expert expects bf16 activations")
    w1, s1 = _check_weight(w1, s1, "w1")
    w3, s3 = _check_weight(w3, s3, "w3")
    w2, s2 = _check_weight(w2, s2, "w2")
    f, d = w1.shape
    if tuple(w3.shape) != (f, d) or tuple(w2.shape) != (d, f):
        raise ValueError(f"w1 {tuple(w1.shape)}, w3 {tuple(w3.shape)}, w2 {tuple(w2.shape)} do not form an expert")
    if x.shape[-1] != d:
        raise ValueError(f"x has {x.shape[-1]} features, the expert expects {d}")
    _lib.require_cuda(x)
    x2 = x.reshape(-1, d).contiguous()
    m = x2.shape[0]
    y = torch.empty((m, d), dtype=torch.bfloat16, device=x.device)
    L = _lib.lib()
    nbytes = L.cachalot_shared_expert_fp8_workspace_bytes(m, d, f)
    ws = _workspace(x.device, nbytes)
    rc = L.cachalot_shared_expert_fp8(x2.data_ptr(), w1.data_ptr(), s1.data_ptr(), w3.data_ptr(), s3.data_ptr(),
                                      w2.data_ptr(), s2.data_ptr(), m, d, f, float(swiglu_limit), y.data_ptr(),
                                      ws.data_ptr(), nbytes, _lib.stream_handle(x.device))
    _lib.check(rc, "shared_expert_fp8")
    return y.reshape(x.shape)


def shared_expert_forward(x: torch.Tensor, *, w1, w1_scales, w2, w2_scales, w3, w3_scales,
                          swiglu_limit: float = 10.0) -> torch.Tensor:
    """One token: x [D] bf16 -> bf16 [D]."""
    if x.ndim != 1:
        raise ValueError(f"x must be 1D for decode, got {tuple(x.shape)}")
    return _shared(x, w1, w1_scales, w2, w2_scales, w3, w3_scales, swiglu_limit)


def shared_expert_forward_fused(x: torch.Tensor, *, w13, w13_scales, w2, w2_scales,
                                swiglu_limit: float = 10.0) -> torch.Tensor:
    """One token with w1 and w3 stacked along rows (w13 [2F, D], scales [2F/32, D/32])."""
    w13 = _bytes(w13, "w13")
    f = w13.shape[0] // 2
    if w13.shape[0] != 2 * f or f % BLOCK:
        raise ValueError(f"w13 rows {w13.shape[0]} must be 2 * F with F a multiple of {BLOCK}")
    return shared_expert_forward(x, w1=w13[:f], w1_scales=w13_scales[: f // BLOCK], w2=w2, w2_scales=w2_scales,
                                 w3=w13[f:], w3_scales=w13_scales[f // BLOCK:], swiglu_limit=swiglu_limit)


def shared_expert_forward_batched(x: torch.Tensor, *, w1, w1_scales, w2, w2_scales, w3, w3_scales,
                                  swiglu_limit: float = 10.0) -> torch.Tensor:
    """Rows: x [M, D] bf16 -> bf16 [M, D] (the decode path's casts, per row)."""
    if x.ndim != 2:
        raise ValueError(f"x must be 2D [tokens, hidden], got {tuple(x.shape)}")
    return _shared(x, w1, w1_scales, w2, w2_scales, w3, w3_scales, swiglu_limit)


def shared_weights(shared: dict, d_model: int) -> tuple:
    """The bundle's tensors checked for a layer of width d_model: (w1, s1, w3, s3, w2, s2, F)."""
    w1, s1 = _check_weight(shared["w1"], shared["w1_scales"], "w1")
    w3, s3 = _check_weight(shared["w3"], shared["w3_scales"], "w3")
    w2, s2 = _check_weight(shared["w2"], shared["w2_scales"], "w2")
    f, d = w1.shape
    if d != d_model or tuple(w3.shape) != (f, d) or tuple(w2.shape) != (d, f):
        raise ValueError(f"w1 {tuple(w1.shape)}, w3 {tuple(w3.shape)}, w2 {tuple(w2.shape)} do not form an expert "
                         f"of width {d_model}")
    return w1, s1, w3, s3, w2, s2, f


def shared_args(shared_w1, shared_w1_scales, shared_w2, shared_w2_scales, shared_w3, shared_w3_scales):
    """The six shared_* call-site arguments as one bundle (None when all are None)."""
    parts = (shared_w1, shared_w1_scales, shared_w2, shared_w2_scales, shared_w3, shared_w3_scales)
    if all(p is None for p in parts):
        return None
    if any(p is None for p in parts):
        raise ValueError("shared_w1/w2/w3 and their scales must be given together")
    return dict(w1=shared_w1, w1_scales=shared_w1_scales, w2=shared_w2, w2_scales=shared_w2_scales,
                w3=shared_w3, w3_scales=shared_w3_scales)
