"""Layer primitives the MoE path needs: the parameter-owning base class and the
gated-activation registry."""

from .activation import GATED_ACTIVATIONS, activation_code
from .base import BaseOP

__all__ = ["BaseOP", "GATED_ACTIVATIONS", "activation_code"]
