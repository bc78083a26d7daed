"""MoE: routing, grouped expert compute and the host-offload expert cache.

Import surface of the reference's ``reframework.moe`` (reframework/moe/
__init__.py:8-18).
"""

import importlib
import sys

import torch

from reframework_amd import _capi
from reframework_amd.moe import fused as _fused
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


# Names the reference's package and its submodules export, rebound by install().
_PACKAGE_NAMES = ("torch_fused_topk", "fused_experts", "FusedMoE", "ExpertOffloadCache",
                  "OffloadStats")
_SUBMODULE_NAMES = {
    "fused": ("torch_fused_topk", "fused_experts", "fused_experts_masked",
              "fused_experts_cpu_int8"),
    "moe_layer": ("FusedMoE", "CpuShuttle"),
    "offload_cache": ("ExpertOffloadCache", "OffloadStats", "Prediction"),
}


def install(package: str = "reframework.moe") -> bool:
    """Route the reference package's MoE names to this library, from its
    ``__init__`` (the drop-in patch): the package's own exports
    (reframework/moe/__init__.py:8-18) and the same names in its submodules,
    which other code imports directly (``from reframework.moe.fused import
    fused_experts`` in parallel/ep.py:32 and integrations/litemoe_adapter.py:39;
    ``from reframework.moe.moe_layer import CpuShuttle`` in
    engine/engine.py:460). Modules imported after the call see these names;
    the reference's own functions stay reachable as ``_reference_<name>`` on
    each module. Returns False and changes nothing when :func:`available` is
    false (no ROCm GPU, or libmoe355.so not built)."""
    if not available():
        return False
    ours = {"torch_fused_topk": torch_fused_topk, "fused_experts": fused_experts,
            "fused_experts_masked": _fused.fused_experts_masked,
            "fused_experts_cpu_int8": _fused.fused_experts_cpu_int8,
            "FusedMoE": FusedMoE, "CpuShuttle": CpuShuttle,
            "ExpertOffloadCache": ExpertOffloadCache, "OffloadStats": OffloadStats,
            "Prediction": Prediction}

    def rebind(module, names):
        for name in names:
            if hasattr(module, name) and not hasattr(module, "_reference_" + name):
                setattr(module, "_reference_" + name, getattr(module, name))
            setattr(module, name, ours[name])

    pkg = sys.modules.get(package) or importlib.import_module(package)
    for sub, names in _SUBMODULE_NAMES.items():
        rebind(importlib.import_module(f"{package}.{sub}"), names)
    rebind(pkg, _PACKAGE_NAMES)
    return True


__all__ = [
    "available",
    "install",
    "torch_fused_topk",
    "fused_experts",
    "FusedMoE",
    "CpuShuttle",
    "ExpertOffloadCache",
    "ExpertPool",
    "OffloadStats",
    "Prediction",
]
