"""Parameter-owning operator base class.

Same (de)serialisation contract as the reference's ``BaseOP``
(reframework/layers/base.py:17-44): ``state_dict(prefix=...)`` returns the
parameters under ``prefix.name`` keys and ``load_state_dict(sd, prefix=...)``
copies matching keys into them, casting to each parameter's dtype and device.
"""

from __future__ import annotations

from typing import Dict

import torch
import torch.nn as nn


class BaseOP(nn.Module):
    """An operator that owns parameters (weights)."""

    def _load_state_dict_raw(self, state_dict: Dict[str, torch.Tensor], prefix: str) -> None:
        own = self.state_dict(prefix=prefix)
        with torch.no_grad():
            for key, value in own.items():
                if key in state_dict:
                    src = state_dict[key].detach()
                    value.copy_(src.to(device=value.device, dtype=value.dtype))

    def load_state_dict(self, state_dict, *, prefix: str = "", strict: bool = True,
                        assign: bool = False):
        self._load_state_dict_raw(state_dict, prefix)

    def state_dict(self, *, prefix: str = "", result=None, destination=None,
                   keep_vars: bool = False) -> Dict[str, torch.Tensor]:
        out = destination if destination is not None else ({} if result is None else result)
        for name, param in self.named_parameters():
            out[f"{prefix}.{name}" if prefix else name] = param if keep_vars else param.detach()
        return out


__all__ = ["BaseOP"]
