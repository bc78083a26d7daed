"""Shared expert pool (one HBM LRU across layers), host-side policy on the CPU.

Not in the reference, whose offload caches are per layer
(reframework/moe/offload_cache.py); the semantics follow litemoe's global LRU
(litemoe/src/litemoe/cache/lru.py:66-102: hit -> move to back, miss ->
append, evict oldest over capacity) with one difference: the experts of the
request being served are never evicted by it. Expectations below are worked
out by hand.
"""

from __future__ import annotations

import torch

from reframework_amd.moe import ExpertOffloadCache, ExpertPool


def _cache(pool, E=6):
    c = ExpertOffloadCache("cpu", lru_capacity=1, dtype=torch.float32, pool=pool)
    c.load([{"w1": torch.full((4, 2), float(e)), "w2": torch.full((2, 2), float(e))}
            for e in range(E)])
    return c


def test_global_lru_known_answer():
    pool = ExpertPool(capacity=3)
    A, B = _cache(pool), _cache(pool)
    A.prefetch([0, 1])                 # A0 A1
    B.prefetch([0])                    # A0 A1 B0
    B.prefetch([1])                    # A0 evicted: A1 B0 B1
    assert set(A._lru) == {1} and set(B._lru) == {0, 1}
    A.prefetch([1])                    # hit: B0 B1 A1
    A.prefetch([0, 2])                 # B0, B1 evicted: A1 A0 A2
    assert set(B._lru) == set() and set(A._lru) == {0, 1, 2}
    A.prefetch([0, 1, 2, 3])           # all protected: overflow to 4
    assert len(pool) == 4 and set(A._lru) == {0, 1, 2, 3}
    B.prefetch([0])                    # A1, A0 evicted: A2 A3 B0
    assert set(A._lru) == {2, 3} and set(B._lru) == {0}
    assert (A.stats.hits, A.stats.misses, A.stats.evictions) == (4, 5, 3)
    assert (B.stats.hits, B.stats.misses, B.stats.evictions) == (0, 3, 2)


def test_pool_serves_right_tensors_and_forgets_on_reset():
    pool = ExpertPool(capacity=2)
    A, B = _cache(pool), _cache(pool)
    w1, w2, idx = A.prefetch([4, 1])
    assert idx == {1: 0, 4: 1} and torch.all(w1[1] == 4.0) and torch.all(w2[0] == 1.0)
    B.prefetch([5])                    # evicts A1 (oldest)
    assert set(A._lru) == {4}
    A.reset_lru()
    assert len(pool) == 1 and set(B._lru) == {5}
    B.prefetch([2, 3])                 # B5 evicted; the pool holds exactly the request
    assert set(B._lru) == {2, 3} and len(pool) == 2


def test_reserve_respects_the_shared_capacity():
    pool = ExpertPool(capacity=3)
    A, B = _cache(pool), _cache(pool)
    B.prefetch([0, 1])
    A.prefetch([0])
    n = A.reserve([2, 3], protect_current=[0])
    # loading 2 evicts B0 (oldest); loading 3 evicts B1; capacity is never exceeded
    assert n == 2 and set(A._lru) == {0, 2, 3} and set(B._lru) == set() and len(pool) == 3


def test_share_host_reuses_the_pool_with_separate_residency():
    A = _cache(None)
    B = ExpertOffloadCache("cpu", lru_capacity=1, dtype=torch.float32)
    B.share_host(A)
    assert B._host_buf is A._host_buf and B.num_experts == A.num_experts
    w1, w2, idx = B.prefetch([3])
    assert idx == {3: 0} and torch.all(w1[0] == 3.0) and torch.all(w2[0] == 3.0)
    assert set(B._lru) == {3} and set(A._lru) == set()
    assert (B.stats.misses, A.stats.misses) == (1, 0)
    A.prefetch([2])
    assert set(A._lru) == {2} and set(B._lru) == {3}


def test_share_host_rejects_empty_or_other_dtype():
    import pytest

    empty = ExpertOffloadCache("cpu", lru_capacity=1, dtype=torch.float32)
    with pytest.raises(ValueError):
        ExpertOffloadCache("cpu", lru_capacity=1, dtype=torch.float32).share_host(empty)
    with pytest.raises(ValueError):
        ExpertOffloadCache("cpu", lru_capacity=1, dtype=torch.float16).share_host(_cache(None))
