"""The reference's resident MoE forward, restated with torch CPU ops.

Test infrastructure and CPU baseline only (see oracle.py). This keeps the
reference's op sequence and its dtype roundings, which the fp64 oracle in
moe_oracle.c deliberately does not:

  * router: ``F.linear`` in the model dtype (logits rounded to it), fp32
    softmax, ``torch.topk``, optional renormalisation
    (reframework/moe/moe_layer.py:323-324, reframework/moe/fused.py:32-46);
  * banks: all experts stacked into fresh ``[E,2I,H]`` / ``[E,H,I]`` tensors on
    every call (moe_layer.py:443-447);
  * experts: ascending expert id; gather the routed rows, ``x @ w1[e]^T``,
    ``act(gate) * up`` on the gate-first halves, ``@ w2[e]^T``, scale by the
    routing weight cast to the activation dtype, ``index_add_`` into a
    zero-initialised output of the input dtype (fused.py:62-87).

Grouping uses one stable argsort instead of the reference's per-expert
boolean masks; the visit order (experts ascending, tokens ascending within an
expert) and every arithmetic op are the same.
"""

from __future__ import annotations

from typing import Optional, Sequence, Tuple

import torch
import torch.nn.functional as F


def _gated(activation: str, gu: torch.Tensor) -> torch.Tensor:
    half = gu.shape[-1] // 2
    g, u = gu[..., :half], gu[..., half:]
    if activation == "silu":
        return F.silu(g) * u
    if activation == "gelu":
        return F.gelu(g) * u
    if activation == "gelu_tanh":
        return F.gelu(g, approximate="tanh") * u
    raise ValueError(f"unknown gated activation {activation!r}")


def route(x: torch.Tensor, gate: torch.Tensor, top_k: int, renormalize: bool,
          dtype: torch.dtype, bias: Optional[torch.Tensor] = None
          ) -> Tuple[torch.Tensor, torch.Tensor]:
    logits = F.linear(x.to(dtype), gate)
    scores = logits.float() if bias is None else logits.float() + bias.float()
    probs = torch.softmax(scores, dim=-1)
    w, ids = torch.topk(probs, top_k, dim=-1)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return w.contiguous(), ids.contiguous()


def experts(h: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, topk_w: torch.Tensor,
            topk_ids: torch.Tensor, activation: str = "silu") -> torch.Tensor:
    M, H = h.shape
    K = topk_ids.shape[1]
    E = w1.shape[0]
    out = torch.zeros((M, H), dtype=h.dtype)
    flat_e = topk_ids.reshape(-1)
    flat_w = topk_w.reshape(-1)
    flat_t = torch.arange(M).repeat_interleave(K)
    order = torch.argsort(flat_e, stable=True)
    counts = torch.bincount(flat_e, minlength=E).tolist()
    start = 0
    for e, n in enumerate(counts):
        if n == 0:
            continue
        sel = order[start:start + n]
        start += n
        tok = flat_t[sel]
        y = _gated(activation, h[tok].to(w1.dtype) @ w1[e].t()) @ w2[e].t()
        y = y * flat_w[sel].to(h.dtype).unsqueeze(-1)
        out.index_add_(0, tok, y)
    return out


def forward(x: torch.Tensor, gate: torch.Tensor, w1_list: Sequence[torch.Tensor],
            w2_list: Sequence[torch.Tensor], top_k: int, renormalize: bool = True,
            activation: str = "silu", bias: Optional[torch.Tensor] = None,
            stacked: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> torch.Tensor:
    """Resident forward. ``stacked`` supplies pre-built banks (the pre-stacked
    baseline variant); otherwise the banks are stacked inside the call."""
    dtype = gate.dtype
    w, ids = route(x, gate, top_k, renormalize, dtype, bias)
    if stacked is None:
        w1 = torch.stack(list(w1_list), dim=0)
        w2 = torch.stack(list(w2_list), dim=0)
    else:
        w1, w2 = stacked
    return experts(x, w1, w2, w, ids, activation)
