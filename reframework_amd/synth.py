"""Deterministic synthetic MoE workloads.

A counter-based generator, identical on every machine and independent of
torch's RNG: element i of stream s under seed is

    u_j = (splitmix64(seed ^ (s << 40) ^ (2i + j)) >> 11 + 0.5) * 2^-53, j = 0, 1
    z   = sqrt(-2 ln u_0) * cos(2 pi u_1)        (Box-Muller, fp64)

scaled by sigma and rounded to the target dtype. Streams: x = 1, gate = 2,
router bias = 3, Zipf permutation = 4, routing trace = 5, w1[e] = 100 + e
(rows 0..I-1 gate_proj, I..2I-1 up_proj), w2[e] = 200 + e, shared experts
300 + j. Seed 0, sigma_x = 1, sigma_w = 0.02.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)

STREAM_X, STREAM_GATE, STREAM_BIAS, STREAM_PERM, STREAM_TRACE = 1, 2, 3, 4, 5
STREAM_W1, STREAM_W2, STREAM_SHARED = 100, 200, 300


def splitmix64(x: np.ndarray) -> np.ndarray:
    """Vectorised SplitMix64 finaliser on uint64 counters."""
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform(n: int, stream: int, seed: int = 0, offset: int = 0) -> np.ndarray:
    """n fp64 uniforms in (0, 1) from counters offset..offset+n-1."""
    key = np.uint64(seed) ^ (np.uint64(stream) << np.uint64(40))
    ctr = np.arange(offset, offset + n, dtype=np.uint64) ^ key
    return ((splitmix64(ctr) >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)


def normal(n: int, stream: int, seed: int = 0, sigma: float = 1.0) -> np.ndarray:
    """n fp64 N(0, sigma^2) samples of one stream."""
    key = np.uint64(seed) ^ (np.uint64(stream) << np.uint64(40))
    ctr = np.arange(2 * n, dtype=np.uint64) ^ key
    u = ((splitmix64(ctr) >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)
    u0, u1 = u[0::2], u[1::2]
    return sigma * np.sqrt(-2.0 * np.log(u0)) * np.cos(2.0 * np.pi * u1)


def to_dtype(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    """fp64 -> torch tensor of ``dtype`` with one round-to-nearest-even."""
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float64))
    return t.to(dtype)


@dataclass
class MoEShape:
    name: str
    hidden: int
    experts: int
    top_k: int
    inter: int
    shared: int = 0  # number of always-on shared experts of size `inter`


SHAPES: Dict[str, MoEShape] = {
    "tiny": MoEShape("tiny", 1024, 8, 2, 2816),
    "mixtral": MoEShape("mixtral", 4096, 8, 2, 14336),
    "phi35moe": MoEShape("phi35moe", 4096, 16, 2, 6400),
    "finegrained": MoEShape("finegrained", 2048, 64, 6, 1408, shared=2),
}


def make_layer(shape: MoEShape, dtype: torch.dtype, seed: int = 0, sigma_w: float = 0.02,
               hidden: Optional[int] = None, inter: Optional[int] = None,
               experts: Optional[int] = None) -> Dict[str, object]:
    """Weights of one MoE layer on the CPU: gate [E,H], w1[e] [2I,H], w2[e] [H,I]."""
    H = hidden or shape.hidden
    I = inter or shape.inter
    E = experts or shape.experts
    gate = to_dtype(normal(E * H, STREAM_GATE, seed, sigma_w).reshape(E, H), dtype)
    w1 = [to_dtype(normal(2 * I * H, STREAM_W1 + e, seed, sigma_w).reshape(2 * I, H), dtype)
          for e in range(E)]
    w2 = [to_dtype(normal(H * I, STREAM_W2 + e, seed, sigma_w).reshape(H, I), dtype)
          for e in range(E)]
    return {"gate": gate, "w1": w1, "w2": w2, "H": H, "I": I, "E": E}


def make_shared(n: int, H: int, I: int, dtype: torch.dtype, seed: int = 0,
                sigma_w: float = 0.02) -> Dict[str, object]:
    """``n`` shared experts of width ``I`` (stream 300+j), as pieces w1[j]
    [2I,H] (gate rows first) / w2[j] [H,I], and as the merged HF tensors
    ``gate_proj``/``up_proj`` [n*I,H] and ``down_proj`` [H,n*I]."""
    w1 = [to_dtype(normal(2 * I * H, STREAM_SHARED + j, seed, sigma_w).reshape(2 * I, H), dtype)
          for j in range(n)]
    w2 = [to_dtype(normal(H * I, STREAM_SHARED + 64 + j, seed, sigma_w).reshape(H, I), dtype)
          for j in range(n)]
    return {"w1": w1, "w2": w2,
            "gate_proj": torch.cat([w[:I] for w in w1]) if n else None,
            "up_proj": torch.cat([w[I:] for w in w1]) if n else None,
            "down_proj": torch.cat(w2, dim=1) if n else None}


def offload_trace(n_layers: int, steps: int, T: int, E: int, seed: int = 0,
                  p_repeat: float = 0.7, zipf_s: float = 1.2):
    """Synthetic decode routing for offload runs (bypasses the router).

    Per layer and token: with probability ``p_repeat`` the previous step's
    expert pair again, else two distinct experts drawn from Zipf(``zipf_s``)
    popularity over a seeded per-layer rank permutation. Weights are the
    softmax of two N(0,1) logits, largest first. Returns (ids int32, w fp32),
    both [steps, n_layers, T, 2].
    """
    rng = np.random.Generator(np.random.PCG64([seed, STREAM_TRACE]))
    pops = []
    for _ in range(n_layers):
        ranks = np.empty(E, dtype=np.int64)
        ranks[rng.permutation(E)] = np.arange(1, E + 1)
        pop = ranks.astype(np.float64) ** (-zipf_s)
        pops.append(pop / pop.sum())
    ids = np.zeros((steps, n_layers, T, 2), dtype=np.int32)
    w = np.zeros((steps, n_layers, T, 2), dtype=np.float32)
    for st in range(steps):
        for li in range(n_layers):
            for t in range(T):
                if st > 0 and rng.random() < p_repeat:
                    ids[st, li, t] = ids[st - 1, li, t]
                else:
                    ids[st, li, t] = rng.choice(E, size=2, replace=False, p=pops[li])
                lg = rng.standard_normal(2)
                pr = np.exp(lg - lg.max())
                pr = np.sort(pr / pr.sum())[::-1]
                w[st, li, t] = pr
    return ids, w


def make_tokens(T: int, H: int, dtype: torch.dtype, seed: int = 0) -> torch.Tensor:
    return to_dtype(normal(T * H, STREAM_X, seed, 1.0).reshape(T, H), dtype)


def mixtral_router_bias(E: int, seed: int = 0) -> torch.Tensor:
    """Fixed per-expert router bias N(0, 0.5^2), fp32: mildly skewed load."""
    return to_dtype(normal(E, STREAM_BIAS, seed, 0.5), torch.float32)


def zipf_router_bias(E: int, s: float, seed: int = 0) -> torch.Tensor:
    """log of a Zipf(s) popularity over a seeded rank permutation of experts."""
    perm = np.argsort(uniform(E, STREAM_PERM, seed), kind="stable")
    ranks = np.empty(E, dtype=np.int64)
    ranks[perm] = np.arange(1, E + 1)
    pop = ranks.astype(np.float64) ** (-s)
    return to_dtype(np.log(pop / pop.sum()), torch.float32)


__all__ = [
    "splitmix64", "uniform", "normal", "to_dtype", "MoEShape", "SHAPES", "make_layer",
    "make_shared", "offload_trace",
    "make_tokens", "mixtral_router_bias", "zipf_router_bias",
]
