"""Brute-force replay of the offload cache's residency decisions (test
infrastructure, not collected: no test_ prefix).

Restates, without importing reframework_amd.moe.offload_cache, what the
reference decides per request with the default ``lru`` policy and no
lookahead or similarity table:

  * which experts a layer requests: the offload forward keeps the
    ``RE_MAX_PACK`` experts of largest summed routing weight, ties by first
    appearance (reframework/moe/moe_layer.py:426-442); the streaming forward
    requests every routed expert, ascending, in chunks of ``RE_CHUNK_SIZE``
    (moe_layer.py:367-376);
  * what one request does: for each requested id in ascending order a hit
    (resident) moves it to the most recent end, a miss appends it; then the
    oldest entries outside the request are evicted while the window is over
    capacity (offload_cache.py:478-507, 654-711). A request larger than the
    capacity overflows it.

``LruReplay`` is one layer's window; ``PoolReplay`` is one window over
(layer, expert) shared by every layer, as ``ExpertPool`` keeps it.
"""

from __future__ import annotations

from typing import Dict, List, Sequence, Tuple

import numpy as np


def truncated_request(ids: np.ndarray, w: np.ndarray, max_pack: int) -> List[int]:
    """Experts of largest summed weight (ties: first appearance), ascending."""
    sums: Dict[int, float] = {}
    for e, v in zip(np.asarray(ids).reshape(-1).tolist(), np.asarray(w).reshape(-1).tolist()):
        if e >= 0:
            sums[e] = sums.get(e, 0.0) + v
    order = sorted(sums, key=lambda e: -sums[e])  # stable: ties keep first appearance
    return sorted(order[:max_pack])


def chunked_requests(ids: np.ndarray, chunk: int) -> List[List[int]]:
    uniq = sorted({int(e) for e in np.asarray(ids).reshape(-1).tolist() if e >= 0})
    return [uniq[i:i + chunk] for i in range(0, len(uniq), chunk)]


class LruReplay:
    """One layer's LRU window of ``capacity`` experts."""

    def __init__(self, capacity: int) -> None:
        self.capacity = capacity
        self.order: List[int] = []  # oldest first
        self.hits = self.misses = self.evictions = 0
        self.peak = 0

    def admit(self, request: Sequence[int]) -> None:
        req = sorted(set(int(i) for i in request))
        for e in req:
            if e in self.order:
                self.hits += 1
                self.order.remove(e)
            else:
                self.misses += 1
            self.order.append(e)
        self.peak = max(self.peak, len(self.order))
        while len(self.order) > self.capacity:
            victim = next((e for e in self.order if e not in req), None)
            if victim is None:
                break
            self.order.remove(victim)
            self.evictions += 1


class PoolReplay:
    """One LRU window of ``capacity`` (layer, expert) entries for all layers."""

    def __init__(self, capacity: int, n_layers: int) -> None:
        self.capacity = capacity
        self.order: List[Tuple[int, int]] = []
        self.hits = [0] * n_layers
        self.misses = [0] * n_layers
        self.evictions = [0] * n_layers  # counted on the layer that owned the victim
        self.peak = 0

    def admit(self, layer: int, request: Sequence[int]) -> None:
        req = [(layer, e) for e in sorted(set(int(i) for i in request))]
        for key in req:
            if key in self.order:
                self.hits[layer] += 1
                self.order.remove(key)
            else:
                self.misses[layer] += 1
            self.order.append(key)
        self.peak = max(self.peak, len(self.order))
        while len(self.order) > self.capacity:
            victim = next((k for k in self.order if k not in req), None)
            if victim is None:
                break
            self.order.remove(victim)
            self.evictions[victim[0]] += 1
