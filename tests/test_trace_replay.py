"""Replay of the reference's recorded routing traces through the expert caches.

The traces are the reference's own activation logs (litemoe/data/activation_logs/
tiny.jsonl and huihui.jsonl, kept here as fixtures): one record per (decode step,
layer) with the experts that layer routed to. Each is replayed, on the CPU,
through:

  * one ExpertOffloadCache per layer (the reference's per-layer LRU window:
    ``prefetch`` of the step's experts, then eviction of the oldest entries
    outside the request, reframework/moe/offload_cache.py:478-507, 654-711);
  * one ExpertPool shared by every layer's cache (a global LRU over
    (layer, expert), as litemoe's cache, litemoe/src/litemoe/cache/lru.py:66-102,
    except that it never evicts an expert of the request being served).

Hit, miss and eviction counts are checked against brute-force simulations
written here with plain lists, for several capacities; on the single-expert
trace the pool must also give exactly the counts of litemoe's own eviction rule
(evict the oldest before each insert), since with one expert per request the
two rules coincide; and a few totals are worked out by hand.
"""

from __future__ import annotations

import json
import os
from typing import Dict, List, Tuple

import pytest
import torch

from reframework_amd.moe import ExpertOffloadCache, ExpertPool

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _trace(name: str) -> List[Tuple[int, int, List[int]]]:
    with open(os.path.join(GOLDEN, f"trace_{name}.jsonl")) as f:
        recs = [json.loads(line) for line in f if line.strip()]
    return [(int(r["step"]), int(r["layer"]), [int(e) for e in r["experts"]]) for r in recs]


def _shape(trace):
    n_layers = 1 + max(r[1] for r in trace)
    n_experts = 1 + max(e for r in trace for e in r[2])
    return n_layers, n_experts


# ------------------------------------------------------------- brute force
def brute_per_layer(trace, capacity):
    """Per-layer LRU window, reference rules: the request's distinct experts
    in ascending order, a hit moves to the back, a miss is appended; then the
    oldest entries outside the request go until the window fits."""
    lru: Dict[int, List[int]] = {}
    hits = misses = evictions = 0
    for _, layer, experts in trace:
        q = lru.setdefault(layer, [])
        req = sorted(set(experts))
        for e in req:
            if e in q:
                hits += 1
                q.remove(e)
            else:
                misses += 1
            q.append(e)
        while len(q) > capacity:
            victim = next((e for e in q if e not in req), None)
            if victim is None:
                break
            q.remove(victim)
            evictions += 1
    return hits, misses, evictions


def brute_pool(trace, capacity):
    """One LRU over (layer, expert): the same rules over the shared order."""
    q: List[Tuple[int, int]] = []
    hits = misses = evictions = 0
    for _, layer, experts in trace:
        req = [(layer, e) for e in sorted(set(experts))]
        for k in req:
            if k in q:
                hits += 1
                q.remove(k)
            else:
                misses += 1
            q.append(k)
        while len(q) > capacity:
            victim = next((k for k in q if k not in req), None)
            if victim is None:
                break
            q.remove(victim)
            evictions += 1
    return hits, misses, evictions


def brute_litemoe(trace, capacity):
    """litemoe's LRUExpertCache.get per expert in request order: a miss first
    evicts the oldest entries until one slot is free, then inserts."""
    q: List[Tuple[int, int]] = []
    hits = misses = evictions = 0
    for _, layer, experts in trace:
        for e in dict.fromkeys(experts):
            k = (layer, e)
            if k in q:
                hits += 1
                q.remove(k)
                q.append(k)
                continue
            misses += 1
            while len(q) + 1 > capacity:
                q.pop(0)
                evictions += 1
            q.append(k)
    return hits, misses, evictions


# ------------------------------------------------------------- the product
def _caches(n_layers, n_experts, capacity, pool):
    caches = []
    for _ in range(n_layers):
        c = ExpertOffloadCache(device="cpu", lru_capacity=capacity, dtype=torch.float32, pool=pool)
        c.load([{"w1": torch.full((4, 2), float(e)), "w2": torch.full((2, 2), float(e))}
                for e in range(n_experts)])
        caches.append(c)
    return caches


def replay(trace, capacity, shared):
    n_layers, n_experts = _shape(trace)
    pool = ExpertPool(capacity=capacity) if shared else None
    caches = _caches(n_layers, n_experts, capacity, pool)
    for _, layer, experts in trace:
        w1, w2, local = caches[layer].prefetch(experts)
        # the banks handed back are the requested experts' own weights
        for e, row in local.items():
            assert float(w1[row][0, 0]) == float(e) and float(w2[row][0, 0]) == float(e)
    s = [c.stats for c in caches]
    return (sum(x.hits for x in s), sum(x.misses for x in s), sum(x.evictions for x in s)), pool


@pytest.mark.parametrize("name", ["tiny", "huihui"])
@pytest.mark.parametrize("capacity", [1, 2, 3, 4, 8])
def test_per_layer_lru_replay_matches_brute_force(name, capacity):
    trace = _trace(name)
    got, _ = replay(trace, capacity, shared=False)
    assert got == brute_per_layer(trace, capacity)
    assert got[0] + got[1] == sum(len(set(r[2])) for r in trace)


@pytest.mark.parametrize("name", ["tiny", "huihui"])
@pytest.mark.parametrize("capacity", [1, 2, 4, 8, 16, 64])
def test_shared_pool_replay_matches_brute_force(name, capacity):
    trace = _trace(name)
    got, pool = replay(trace, capacity, shared=True)
    assert got == brute_pool(trace, capacity)
    # the pool holds at most its capacity, or one request when that is larger
    assert len(pool) <= max(capacity, max(len(set(r[2])) for r in trace))


@pytest.mark.parametrize("capacity", [1, 2, 3, 5, 8, 12])
def test_shared_pool_equals_litemoe_lru_on_single_expert_requests(capacity):
    """huihui routes one expert per layer and step: the pool's rule and
    litemoe's evict-before-insert rule then make the same decisions."""
    trace = _trace("huihui")
    assert all(len(r[2]) == 1 for r in trace)
    got, _ = replay(trace, capacity, shared=True)
    assert got == brute_litemoe(trace, capacity)


def test_known_counts_worked_by_hand():
    """tiny: layer 0 routes [6,1], then [5,1] on every later step; layer 1
    routes [5,7], then [3,0]. With a per-layer window of 2, each layer misses
    its first two requests (4 misses; 1 of layer 0's second request is a hit)
    and hits forever after; with a shared pool of 4 nothing is evicted after
    the first two steps."""
    trace = _trace("tiny")
    steps = 1 + max(r[0] for r in trace)
    assert steps == 33 and {tuple(r[2]) for r in trace if r[0] > 0 and r[1] == 0} == {(5, 1)}
    (h, m, ev), _ = replay(trace, 2, shared=False)
    # layer 0: 6,1 miss; 5 miss, 1 hit; layer 1: 5,7 miss; 3,0 miss
    assert m == 2 + 1 + 2 + 2 and ev == 1 + 2
    assert h == 2 * 2 * steps - m
    (h4, m4, ev4), _ = replay(trace, 4, shared=True)
    # step 0 fills 4; step 1 adds (0,5), (1,3), (1,0): 3 evictions, 1 hit
    assert m4 == 4 + 3 and ev4 == 3 and h4 == 2 * 2 * steps - m4
