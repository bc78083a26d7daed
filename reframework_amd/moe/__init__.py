"""MoE: routing, grouped expert compute and the host-offload expert cache.

Import surface of the reference's ``reframework.moe`` (reframework/moe/
__init__.py:8-18).
"""

import torch

from reframework_amd import _capi
from reframework_amd.moe.fused import fused_experts, torch_fused_topk
from reframework_amd.moe.moe_layer import CpuShuttle, FusedMoE
from reframework_amd.moe.offload_cache import (ExpertOffloadCache, ExpertPool, OffloadStats,
                                               Prediction)



def available() -> bool:
    """Whether this process can run the MI355X path: a ROCm GPU is visible and
    libmoe355.so loads. The drop-in import in the reference's
    ``reframework/moe/__init__.py`` checks this and keeps the reference's own
    modules (which also run on the CPU) when it is False."""
    if not torch.cuda.is_available():
        return False
    try:
        _capi.lib()
    except (_capi.MoeLibError, OSError):
        return False
    return True


__all__ = [
    "available",
    "torch_fused_topk",
    "fused_experts",
    "FusedMoE",
    "CpuShuttle",
    "ExpertOffloadCache",
    "ExpertPool",
    "OffloadStats",
    "Prediction",
]
