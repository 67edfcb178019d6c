"""ctypes binding of libcachalot_amd.so (the C ABI in include/cachalot_amd.h).

The library must be built in-tree (``python -m cachalot_amd.build``).  There
is no fallback: if the .so is missing or a GPU call fails, the error surfaces
here.  ``torch`` is imported first so that the HIP runtime torch ships with
is the one the library binds to (both carry the soname libamdhip64.so.7).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads the process's HIP runtime before the library)

LIB_PATH = Path(os.environ.get("CACHALOT_AMD_LIB", Path(__file__).resolve().parent / "libcachalot_amd.so"))

OK = 0
EINVAL = -1
ENOTFOUND = -2
EHIP = -3
ESPACE = -4

SCORE_SQRT_SOFTPLUS = 0
SCORE_SIGMOID = 1
ORDER_ASCENDING = 0
ORDER_RANK = 1

SCORE_FNS = {"sqrt_softplus": SCORE_SQRT_SOFTPLUS, "sigmoid": SCORE_SIGMOID}
ORDERS = {"ascending": ORDER_ASCENDING, "rank": ORDER_RANK}

c_void_p = ctypes.c_void_p
c_int = ctypes.c_int
c_int64 = ctypes.c_int64
c_size_t = ctypes.c_size_t
c_float = ctypes.c_float
c_double = ctypes.c_double
c_uint64 = ctypes.c_uint64


class ExpertLayout(ctypes.Structure):
    """cachalot_expert_layout: record stride, nine tensor offsets and the 2-bit bank's
    scale / bias storage type (SCALE_BF16 or SCALE_F16)."""

    _fields_ = [("record_bytes", c_int64), ("offset", c_int64 * 9), ("scale_dtype", ctypes.c_int32)]


SCALE_BF16 = 0
SCALE_F16 = 1
SCALE_DTYPES = {"bfloat16": SCALE_BF16, "float16": SCALE_F16}


def scale_dtype_code(name: str) -> int:
    """The C ABI's code for a 2-bit bank's scale dtype name; other types are refused."""
    try:
        return SCALE_DTYPES[name]
    except KeyError:
        raise ValueError(f"2-bit bank scales/biases must be bfloat16 or float16, got {name!r}") from None


class CachalotError(RuntimeError):
    pass


# name -> (restype, argtypes)
_SIGNATURES = {
    "cachalot_version": (c_int, []),
    "cachalot_last_error": (ctypes.c_char_p, []),
    "cachalot_fill_synthetic": (c_int, [c_void_p, c_int64, c_int64, c_uint64, c_int, c_double, c_double,
                                        c_int64, c_int64, c_void_p]),
    "cachalot_router_topk": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                     c_int, c_int, c_float, c_float, c_int, c_int, c_void_p, c_void_p, c_void_p,
                                     c_void_p]),
    "cachalot_moe_decode_q2_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "cachalot_moe_decode_q2": (c_int, [c_void_p, c_void_p, ctypes.POINTER(ExpertLayout), c_void_p, c_void_p,
                                       c_void_p, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_size_t, c_void_p]),
    "cachalot_moe_decode_fp4_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "cachalot_moe_decode_fp4": (c_int, [c_void_p, c_void_p, ctypes.POINTER(ExpertLayout), c_void_p, c_void_p,
                                        c_void_p, c_int, c_int, c_int, c_int, c_float, c_void_p, c_void_p,
                                        c_void_p, c_void_p, c_size_t, c_void_p]),
    "cachalot_moe_layer_decode_q2": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_float, c_float,
                                             c_int, c_int, c_void_p, ctypes.POINTER(ExpertLayout), c_void_p, c_int,
                                             c_int, c_int, c_float, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                             c_void_p, c_void_p, c_size_t, c_void_p]),
    "cachalot_moe_layer_decode_q2_shared_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "cachalot_moe_layer_decode_q2_shared": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_float,
                                                    c_float, c_int, c_int, c_void_p, ctypes.POINTER(ExpertLayout),
                                                    c_void_p, c_int, c_int, c_int, c_float, c_void_p, c_void_p,
                                                    c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                                                    c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                                    c_void_p]),
    "cachalot_moe_layer_decode_fp4_shared_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "cachalot_moe_layer_decode_fp4_shared": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_float,
                                                     c_float, c_int, c_int, c_void_p, ctypes.POINTER(ExpertLayout),
                                                     c_void_p, c_int, c_int, c_float, c_void_p, c_void_p, c_void_p,
                                                     c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                                                     c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "cachalot_moe_layer_decode_q2_static_max_bytes": (c_size_t, []),
    "cachalot_moe_layer_decode_q2_static": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_float,
                                                    c_float, c_int, c_int, c_void_p, ctypes.POINTER(ExpertLayout),
                                                    c_void_p, c_int, c_int, c_int, c_float, c_void_p, c_void_p,
                                                    c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "cachalot_moe_layer_decode_fp4": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_float, c_float,
                                              c_int, c_int, c_void_p, ctypes.POINTER(ExpertLayout), c_void_p, c_int,
                                              c_int, c_float, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                              c_void_p, c_void_p, c_size_t, c_void_p]),
    "cachalot_permute": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                 c_void_p]),
    "cachalot_grouped_experts_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "cachalot_grouped_experts_q2": (c_int, [c_void_p, c_void_p, ctypes.POINTER(ExpertLayout), c_void_p, c_void_p,
                                            c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
                                            c_float, c_void_p, c_void_p, c_size_t, c_void_p]),
    "cachalot_grouped_experts_q2_routes": (c_int, [c_void_p, c_void_p, ctypes.POINTER(ExpertLayout), c_void_p,
                                                   c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                                   c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p,
                                                   c_void_p, c_size_t, c_void_p]),
    "cachalot_grouped_experts_fp4": (c_int, [c_void_p, c_void_p, ctypes.POINTER(ExpertLayout), c_void_p, c_void_p,
                                             c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                             c_float, c_void_p, c_void_p, c_size_t, c_void_p]),
    "cachalot_unpermute_combine": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "cachalot_fp8_act_quant": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "cachalot_fp8_linear_quantized": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                              c_void_p, c_void_p]),
    "cachalot_shared_expert_fp8_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "cachalot_shared_expert_fp8": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                           c_int, c_int, c_int, c_float, c_void_p, c_void_p, c_size_t, c_void_p]),
    "cachalot_copy_records": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p]),
    "cachalot_stream_read": (c_int, [c_void_p, c_size_t, c_void_p, c_int, c_void_p]),
    "cachalot_requant_fp4_to_q2": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int,
                                           c_void_p]),
    "cachalot_requant_fp4_to_affine": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p,
                                               c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "cachalot_moe_decode_affine_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "cachalot_moe_decode_affine": (c_int, [c_void_p, c_void_p, ctypes.POINTER(ExpertLayout), c_void_p, c_void_p,
                                           c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p,
                                           c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "cachalot_moe_layer_decode_affine": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_float,
                                                 c_float, c_int, c_int, c_void_p, ctypes.POINTER(ExpertLayout),
                                                 c_void_p, c_int, c_int, c_int, c_int, c_float, c_void_p, c_void_p,
                                                 c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                                 c_void_p]),
    "cachalot_grouped_experts_affine_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "cachalot_grouped_experts_affine": (c_int, [c_void_p, c_void_p, ctypes.POINTER(ExpertLayout), c_void_p,
                                                c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                                c_int, c_int, c_int, c_float, c_void_p, c_void_p, c_size_t,
                                                c_void_p]),
    "cachalot_dequant_affine": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
                                        c_int, c_void_p, c_void_p]),
    "cachalot_dequant_fp4": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
    "cachalot_dequant_q2": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
                                    c_void_p, c_void_p]),
}

_lib = None


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it was never built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m cachalot_amd.build` "
                "(the HIP path has no CPU fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().cachalot_last_error().decode(errors="replace")


def check(rc: int, what: str = "") -> None:
    if rc == OK:
        return
    msg = last_error()
    if what:
        msg = f"{what}: {msg}"
    if rc == EINVAL:
        raise ValueError(msg)
    if rc == ENOTFOUND:
        raise KeyError(msg)
    if rc == ESPACE:
        raise MemoryError(msg)
    raise CachalotError(msg)


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_handle(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_cuda(*tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("cachalot_amd kernels need device tensors (got a CPU tensor)")
