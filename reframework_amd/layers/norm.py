"""RMSNorm on libmoe355 (one HIP kernel per call, GPU tensors only).

Same class surface as the reference's RMSNorm (reframework/layers/norm.py:17-53):
``RMSNorm(size, eps, bias=False)`` with ``weight`` (and ``bias``) parameters,
``forward``, ``forward_inplace`` and ``forward_add_residual``. The norm is
computed in fp32 (``x / sqrt(mean(x^2) + eps) * weight (+ bias)``) and rounded
once to the input dtype; ``forward_add_residual`` first forms
``residual = x + residual`` in the input dtype and returns
``(rmsnorm(residual), residual)``. Parameters may be stored in fp32 or the
activation dtype.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from reframework_amd import _capi
from reframework_amd.layers.base import BaseOP


class RMSNorm(BaseOP):
    def __init__(self, size: int, eps: float, bias: bool = False) -> None:
        super().__init__()
        self.eps = eps
        self.size = size
        self.weight = nn.Parameter(torch.ones(size))
        self.bias = nn.Parameter(torch.zeros(size)) if bias else None

    def _params(self, x: torch.Tensor) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        if x.device.type != "cuda":
            raise RuntimeError(f"reframework_amd RMSNorm runs on a ROCm GPU; input is on {x.device}")
        w = self.weight.detach()
        b = None if self.bias is None else self.bias.detach()
        if w.device != x.device:
            raise RuntimeError("RMSNorm parameters must be on the input's device")
        return w.contiguous(), (None if b is None else b.to(w.dtype).contiguous())

    def _run(self, x: torch.Tensor, residual: Optional[torch.Tensor], out: torch.Tensor,
             residual_out: Optional[torch.Tensor]) -> None:
        w, b = self._params(x)
        _capi.add_rmsnorm(x.reshape(-1, self.size), None if residual is None else
                          residual.reshape(-1, self.size),
                          None if residual_out is None else residual_out.reshape(-1, self.size),
                          w, b, self.eps, out.reshape(-1, self.size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x.contiguous()
        out = torch.empty_like(x)
        self._run(x, None, out, None)
        return out

    def forward_inplace(self, x: torch.Tensor) -> None:
        if not x.is_contiguous():
            x.copy_(self.forward(x))
            return
        self._run(x, None, x, None)

    def forward_add_residual(self, x: torch.Tensor,
                             residual: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Fused ``residual = x + residual; x = rmsnorm(residual)``; returns
        (normed, new_residual). The inputs are not modified."""
        x = x.contiguous()
        residual = residual.to(x.dtype).contiguous()
        new_res = torch.empty_like(x)
        out = torch.empty_like(x)
        self._run(x, residual, out, new_res)
        return out, new_res


__all__ = ["RMSNorm"]
