"""MoE: routing, grouped expert compute and the host-offload expert cache.

Import surface of the reference's ``reframework.moe`` (reframework/moe/
__init__.py:8-18).
"""

from reframework_amd.moe.fused import fused_experts, torch_fused_topk
from reframework_amd.moe.moe_layer import CpuShuttle, FusedMoE
from reframework_amd.moe.offload_cache import (ExpertOffloadCache, ExpertPool, OffloadStats,
                                               Prediction)

__all__ = [
    "torch_fused_topk",
    "fused_experts",
    "FusedMoE",
    "CpuShuttle",
    "ExpertOffloadCache",
    "ExpertPool",
    "OffloadStats",
    "Prediction",
]
