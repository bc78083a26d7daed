"""reframework_amd — the MoE layer forward of Reframework, native to MI355X.

Python host code mirrors the reference's ``reframework.moe`` interface
(FusedMoE, torch_fused_topk, fused_experts, ExpertOffloadCache, Prediction,
OffloadStats) and drives libmoe355.so, a C-ABI library of hand-written gfx950
HIP kernels (include/moe355.h).
"""

__version__ = "0.1.0"
__all__ = ["__version__"]
