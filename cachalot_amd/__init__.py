"""cachalot_amd: the routed-expert MoE path of Cachalot, native to MI355X (gfx950).

Host side in PyTorch-ROCm, compute in hand-written HIP kernels behind the C ABI
of ``libcachalot_amd.so`` (``include/cachalot_amd.h``).  Public entry points
mirror the reference's call sites:

* routing: ``route_topk``, ``route_topk_fused``, ``route_topk_batch``, ``route_topk_rows``
* decode:  ``moe_layer_forward``, ``fused_routed_experts``, ``affine_routed_experts``
* prefill / batched decode: ``moe_prefill_grouped``, ``grouped_experts``; one expert over
  many rows: ``routed_expert_forward_batched``, ``routed_expert_forward_sgmm``,
  ``affine_expert_forward_batched``
* shared FP8 expert: ``shared_expert_forward``, ``shared_expert_forward_fused``,
  ``shared_expert_forward_batched``, ``fp8_linear``, ``quantize_fp8_activation``
* store:   ``ResidentExpertStore`` over an ``HBMSlotPool``; formats in ``storage.index``
"""
from __future__ import annotations

__version__ = "0.1.0"

__all__ = [
    "RouterResult", "route_topk", "route_topk_fused", "route_topk_batch", "route_topk_rows",
    "moe_layer_forward", "moe_prefill_grouped", "grouped_experts", "fused_routed_experts", "affine_routed_experts", "affine_expert_forward",
    "routed_expert_forward_batched", "routed_expert_forward_sgmm", "affine_expert_forward_batched",
    "shared_expert_forward", "shared_expert_forward_fused", "shared_expert_forward_batched", "fp8_linear",
    "fp8_linear_quantized", "quantize_fp8_activation",
    "ResidentExpertStore", "HBMSlotPool", "ExpertFormat", "FP4_FORMAT", "affine_format", "fp4_format",
]


def __getattr__(name):  # lazy: importing the package does not load torch or the library
    if name in ("RouterResult", "route_topk", "route_topk_fused", "route_topk_batch", "route_topk_rows"):
        from . import router
        return getattr(router, name)
    if name in ("fused_routed_experts", "affine_routed_experts", "affine_expert_forward"):
        from . import moe_decode
        return getattr(moe_decode, name)
    if name in ("routed_expert_forward_batched", "routed_expert_forward_sgmm", "affine_expert_forward_batched"):
        from . import expert_rows
        return getattr(expert_rows, name)
    if name in ("moe_prefill_grouped", "grouped_experts"):
        from . import moe_prefill
        return getattr(moe_prefill, name)
    if name in ("shared_expert_forward", "shared_expert_forward_fused", "shared_expert_forward_batched",
                "fp8_linear", "fp8_linear_quantized", "quantize_fp8_activation"):
        from . import shared_expert
        return getattr(shared_expert, name)
    if name == "moe_layer_forward":
        from .moe_layer import moe_layer_forward
        return moe_layer_forward
    if name == "ResidentExpertStore":
        from .cache.resident_store import ResidentExpertStore
        return ResidentExpertStore
    if name == "HBMSlotPool":
        from .cache.slots import HBMSlotPool
        return HBMSlotPool
    if name in ("ExpertFormat", "FP4_FORMAT", "affine_format", "fp4_format"):
        from .storage import index
        return getattr(index, name)
    raise AttributeError(name)
