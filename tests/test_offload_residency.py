"""Residency decisions of the offload caches over the offload-decode routing
trace, against an independent brute-force replay (tests/_offload_replay.py),
and the release order of a shared host pool. Host-side policy on the CPU.

Reference: ExpertOffloadCache.prefetch / _evict (reframework/moe/
offload_cache.py:478-507, 654-711) driven by FusedMoE._banks (truncation to
RE_MAX_PACK, moe_layer.py:426-442) and _forward_streaming (chunks of
RE_CHUNK_SIZE, moe_layer.py:367-376). The caches here evict before they
admit a request's misses (so a slot is reused instead of allocated); the
replay evicts afterwards, as the reference does. Hits, misses and evictions
must agree layer by layer, and the resident set may never exceed
max(capacity, request) at any moment.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _offload_replay import LruReplay, PoolReplay, chunked_requests, truncated_request
from reframework_amd import synth
from reframework_amd.moe import ExpertOffloadCache, ExpertPool
from reframework_amd.moe.offload_cache import _HostPool

N_LAYERS, STEPS, T, E = 32, 96, 8, 8


class _PeakCache(ExpertOffloadCache):
    """Records the largest resident set and pool size seen right after a fill."""

    peak = 0
    pool_peak = 0

    def _fill(self, idx: int) -> None:
        super()._fill(idx)
        self.peak = max(self.peak, len(self._lru))
        if self._pool is not None:
            self.pool_peak = max(self.pool_peak, len(self._pool) + 1)


def _caches(pool, cap):
    out = []
    for _ in range(N_LAYERS):
        c = _PeakCache("cpu", lru_capacity=cap, dtype=torch.float32, pool=pool)
        c.load([{"w1": torch.full((4, 2), float(e)), "w2": torch.full((2, 2), float(e))}
                for e in range(E)])
        out.append(c)
    return out


def _requests(ids, w, st, li, mode):
    if mode == "truncate":
        return [truncated_request(ids[st, li], w[st, li], 2)]
    return chunked_requests(ids[st, li], int(mode.split("_")[1]))


@pytest.mark.parametrize("mode", ["truncate", "chunk_1", "chunk_2", "chunk_8"])
@pytest.mark.parametrize("cap", [2, 3])
def test_per_layer_windows_match_replay(mode, cap):
    ids, w = synth.offload_trace(N_LAYERS, STEPS, T, E)
    caches = _caches(None, cap)
    replay = [LruReplay(cap) for _ in range(N_LAYERS)]
    biggest = 0
    for st in range(STEPS):
        for li in range(N_LAYERS):
            for req in _requests(ids, w, st, li, mode):
                caches[li].prefetch_slots(req)
                replay[li].admit(req)
                biggest = max(biggest, len(req))
    for c, r in zip(caches, replay):
        assert (c.stats.hits, c.stats.misses, c.stats.evictions) == (r.hits, r.misses, r.evictions)
        assert list(c._lru) == r.order
        # evicting first: never more than max(capacity, request) resident
        assert c.peak <= max(cap, biggest)
    total = sum(r.hits + r.misses for r in replay)
    print(f"  {mode} cap {cap}: hit rate {sum(r.hits for r in replay) / total:.3f}")


@pytest.mark.parametrize("mode", ["truncate", "chunk_1", "chunk_8"])
def test_shared_pool_matches_replay(mode):
    ids, w = synth.offload_trace(N_LAYERS, STEPS, T, E)
    pool = ExpertPool(capacity=2 * N_LAYERS)
    caches = _caches(pool, 2)
    replay = PoolReplay(2 * N_LAYERS, N_LAYERS)
    biggest = 0
    for st in range(STEPS):
        for li in range(N_LAYERS):
            for req in _requests(ids, w, st, li, mode):
                caches[li].prefetch_slots(req)
                replay.admit(li, req)
                biggest = max(biggest, len(req))
    for li, c in enumerate(caches):
        assert (c.stats.hits, c.stats.misses, c.stats.evictions) == \
            (replay.hits[li], replay.misses[li], replay.evictions[li])
    assert [(caches.index(c), e) for (_, e), c in pool._order.items()] == replay.order
    assert max(c.pool_peak for c in caches) <= max(pool.capacity, biggest)


def test_lookahead_reserve_frees_stale_slots_before_copying():
    """reserve() evicts a stale entry before each lookahead copy, so the
    window stays within capacity while stale entries are left; with none left
    it loads one more and stops (offload_cache.py:569-643), as before."""
    c = _caches(None, 3)[0]
    c.prefetch_slots([0, 1, 2])
    assert c.reserve([4, 5], protect_current=[0]) == 2  # 1 and 2 make room for 4 and 5
    assert list(c._lru) == [0, 4, 5] and c.peak == 3 and c.stats.evictions == 2
    d = _caches(None, 3)[0]
    d.prefetch_slots([0, 1])
    # 4 fits; 1 makes room for 5; nothing stale is left for 6: loaded, then stop
    assert d.reserve([4, 5, 6, 7], protect_current=[0]) == 3
    assert list(d._lru) == [0, 4, 5, 6] and d.peak == 4 and d.stats.evictions == 1


class _FakeEvent:
    def __init__(self, log, name):
        self.log, self.name = log, name

    def synchronize(self):
        self.log.append(self.name)


def test_host_pool_waits_for_every_sharers_copies_before_release():
    """The staged buffer is released only after the last copy of every copy
    stream that read it: the holder drains them when the last cache drops it."""
    log = []
    buf = torch.zeros(16)
    holder = _HostPool(buf)
    holder.note_copy(1, _FakeEvent(log, "s1-a"))
    holder.note_copy(2, _FakeEvent(log, "s2-a"))
    holder.note_copy(1, _FakeEvent(log, "s1-b"))  # stream order: covers s1-a
    del holder
    assert sorted(log) == ["s1-b", "s2-a"]


def test_share_host_keeps_one_holder_until_the_last_cache_lets_go():
    A = _caches(None, 2)[0]
    B = ExpertOffloadCache("cpu", lru_capacity=1, dtype=torch.float32)
    B.share_host(A)
    assert B._host_pool is A._host_pool
    log = []
    A._host_pool.note_copy(7, _FakeEvent(log, "B-copy"))
    A.load([{"w1": torch.zeros(4, 2), "w2": torch.zeros(2, 2)}])  # A restages: B still reads
    assert log == [] and B._host_pool is not A._host_pool
    del B
    assert log == ["B-copy"]
