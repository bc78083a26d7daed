"""Layer primitives the MoE path needs: the parameter-owning base class, the
gated-activation registry and the RMSNorm that precedes the MoE block."""

from .activation import GATED_ACTIVATIONS, activation_code
from .base import BaseOP
from .norm import RMSNorm

__all__ = ["BaseOP", "GATED_ACTIVATIONS", "activation_code", "RMSNorm"]
