"""Gated activation names.

The reference computes ``act(x[..., :d/2]) * x[..., d/2:]`` with torch ops
(reframework/layers/activation.py:15-59): gate half first, up half second,
activations ``silu``, ``gelu`` (erf form) and ``gelu_tanh``, and a
``ValueError`` for any other name. Here the activation is applied inside the
gate_up kernel epilogue; this module only validates names and maps them to the
kernel's codes.
"""

from __future__ import annotations

GATED_ACTIVATIONS = ("silu", "gelu", "gelu_tanh")


def activation_code(activation: str) -> int:
    """Kernel code of a gated activation; ValueError for unknown names."""
    if activation in GATED_ACTIVATIONS:
        return GATED_ACTIVATIONS.index(activation)
    raise ValueError(f"unknown gated activation {activation!r}; known: {GATED_ACTIVATIONS}")


__all__ = ["GATED_ACTIVATIONS", "activation_code"]
