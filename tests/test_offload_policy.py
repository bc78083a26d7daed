"""Expert-cache policy known-answer tests on the CPU.

Restates the reference's cache/predictor/eviction tests
(tests/test_moe_prefetch.py:52-194, tests/test_moe_eviction_policy.py:50-186)
against reframework_amd's ExpertOffloadCache with device="cpu", where the
"HBM" is host memory and only the policy is under test. The bandwidth cap is
exercised by setting ``_bw_gb_s`` directly, as the reference does.
"""

from __future__ import annotations

import os

import pytest
import torch

from reframework_amd import env
from reframework_amd.moe import CpuShuttle, ExpertOffloadCache, OffloadStats, Prediction

DEVICE = torch.device("cpu")


def _cache(E: int, cap: int, H: int = 4, I: int = 2) -> ExpertOffloadCache:
    cache = ExpertOffloadCache(device=DEVICE, lru_capacity=cap, dtype=torch.float16)
    cache.load([{"w1": torch.randn(2 * I, H, dtype=torch.float16),
                 "w2": torch.randn(H, I, dtype=torch.float16)} for _ in range(E)])
    return cache


def _expert_bytes(cache: ExpertOffloadCache) -> int:
    w1, w2 = cache._host[0]
    return (w1.numel() + w2.numel()) * cache.dtype.itemsize


@pytest.fixture
def policy(monkeypatch):
    def _set(value: str) -> None:
        monkeypatch.setenv("RE_CACHE_POLICY", value)
    return _set


# ------------------------------------------------------------------ Prediction
def test_predict_next_ranks_by_frequency_and_filters_resident():
    cache = _cache(E=6, cap=6)
    cache.prefetch([0, 1])
    pred = Prediction(cache, window=16)
    pred._history = [frozenset({2, 4, 0}), frozenset({2, 3, 1}), frozenset({2, 3})]
    pred._age = {2: 0, 3: 1, 4: 2}
    ranked = pred.predict_next()
    assert ranked == [2, 3, 4]
    assert pred.predict_next(limit=2) == [2, 3]


def test_predict_next_recency_tiebreak_then_id():
    cache = _cache(E=4, cap=8)
    pred = Prediction(cache, window=16)
    pred._history.append(frozenset({0}))
    pred._history.append(frozenset({1}))
    pred._age = {0: 1, 1: 0}
    assert pred.predict_next() == [1, 0]
    pred._age = {0: 1, 1: 1}
    assert pred.predict_next() == [0, 1]


def test_prefill_resets_history():
    cache = _cache(E=4, cap=8)
    pred = Prediction(cache, window=16)
    pred.record_step([0], is_prefill=False, forward_ms=0.0)
    pred.record_step([1], is_prefill=False, forward_ms=0.0)
    assert pred._history
    pred.record_step([0, 1, 2, 3], is_prefill=True, forward_ms=0.0)
    assert list(pred._history) == [] and pred._age == {}
    assert pred.predict_next() == []


def test_record_step_ages_and_windows():
    cache = _cache(E=8, cap=1)
    pred = Prediction(cache, window=2)
    for routed in ([0], [1], [2]):
        pred.record_step(routed, is_prefill=False, forward_ms=0.0)
    assert [set(s) for s in pred._history] == [{1}, {2}]
    assert pred._age == {0: 2, 1: 1, 2: 0}


# ------------------------------------------------------------------ reserve
def test_reserve_bandwidth_caps_k():
    cache = _cache(E=8, cap=16)
    b = _expert_bytes(cache)
    cache._bw_headroom = 1.0
    cache._bw_gb_s = 1e9
    n = cache.reserve([0, 1, 2, 3], forward_ms=2.5 * b / 1e15, protect_current=[])
    assert n == 2
    assert set(cache._lru) == {0, 1}
    assert cache._next_reserve == frozenset({0, 1})
    assert cache.stats.predicts == 2


def test_reserve_first_expert_always_loads_and_inflight_is_deducted():
    cache = _cache(E=8, cap=16)
    b = _expert_bytes(cache)
    cache._bw_headroom = 1.0
    cache._bw_gb_s = 1e9
    # budget 0.5 experts: the first still loads (n == 0), the second does not
    assert cache.reserve([5, 6], forward_ms=0.5 * b / 1e15) == 1
    cache2 = _cache(E=8, cap=16)
    cache2._bw_headroom = 1.0
    cache2._bw_gb_s = 1e9
    n = cache2.reserve([0, 1, 2], forward_ms=3.5 * b / 1e15, inflight_bytes=2 * b)
    assert n == 1 and cache2.stats.inflight_bytes == 2 * b


def test_reserve_lru_room_caps_k_and_evicts_stale():
    cache = _cache(E=8, cap=4)
    cache.prefetch([0, 1, 2, 3])
    n = cache.reserve([4, 5], forward_ms=0.0, protect_current=[2, 3])
    assert n == 2
    assert set(cache._lru) == {2, 3, 4, 5}
    assert cache._next_reserve == frozenset({4, 5})


def test_reserve_stops_when_nothing_stale_is_left():
    cache = _cache(E=8, cap=2)
    cache.prefetch([0, 1])
    n = cache.reserve([2, 3, 4], forward_ms=0.0, protect_current=[0, 1])
    assert n == 1 and set(cache._lru) == {0, 1, 2}


def test_reserve_skips_resident_and_noop():
    cache = _cache(E=4, cap=4)
    cache.prefetch([0])
    assert cache.reserve([0, 1, 2], forward_ms=0.0, protect_current=[0]) == 2
    assert set(cache._lru) == {0, 1, 2}
    assert cache.reserve([], forward_ms=0.0) == 0
    zero = _cache(E=4, cap=0)
    assert zero.reserve([1], forward_ms=0.0) == 0


# ------------------------------------------------------------- prefetch tiers
def test_prefetch_counts_and_returns_ascending_banks():
    cache = _cache(E=6, cap=6)
    w1, w2, idx = cache.prefetch([4, 1, 4, -1])
    assert idx == {1: 0, 4: 1}
    assert torch.equal(w1[1], cache._host[4][0]) and torch.equal(w2[0], cache._host[1][1])
    assert (cache.stats.hits, cache.stats.misses) == (0, 2)
    cache.prefetch([1, 2])
    assert (cache.stats.hits, cache.stats.misses) == (1, 3)
    assert cache.stats.transfers_bytes == 3 * _expert_bytes(cache)


def test_prefetch_evicts_stale_not_soft():
    cache = _cache(E=8, cap=4)
    cache.prefetch([0, 1, 7])
    cache._next_reserve = frozenset({0, 1})
    cache.prefetch([2, 3])
    assert set(cache._lru) == {0, 1, 2, 3}


def test_prefetch_evicts_stale_first_then_soft():
    cache = _cache(E=6, cap=4)
    cache.prefetch([0, 1])
    cache._next_reserve = frozenset({0, 1})
    cache.prefetch([2, 3, 4])
    assert {2, 3, 4} <= set(cache._lru) and 0 not in cache._lru and 1 in cache._lru


def test_prefetch_hard_never_evicted_when_only_hard_exceeds():
    cache = _cache(E=6, cap=2)
    cache.prefetch([0, 1, 2])
    assert set(cache._lru) == {0, 1, 2}


def test_reset_lru_clears_reserve_and_history():
    cache = _cache(E=6, cap=4)
    cache.attach_predictor(window=4)
    cache._predictor.record_step([0], is_prefill=False, forward_ms=0.0)
    cache.reserve([3], forward_ms=0.0, protect_current=[0])
    assert cache._next_reserve
    cache.reset_lru()
    assert len(cache._lru) == 0 and cache._next_reserve == frozenset()
    assert list(cache._predictor._history) == []


def test_split_prefetch_and_reactive_load():
    cache = _cache(E=6, cap=3)
    cache.prefetch([0, 1])
    (w1, w2, idx), misses = cache.split_prefetch([1, 3, 0, 5])
    assert idx == {0: 0, 1: 1} and misses == [3, 5] and w1.shape[0] == 2
    cache.reactive_load(misses)
    assert {3, 5} <= set(cache._lru) and len(cache._lru) == 3


# ------------------------------------------------------------------ eviction policy
def test_lru_is_default_when_unset(monkeypatch):
    monkeypatch.delenv("RE_CACHE_POLICY", raising=False)
    cache = _cache(E=6, cap=3)
    cache.prefetch([0, 1, 2])
    cache.prefetch([3])
    assert set(cache._lru) == {1, 2, 3}


def test_lru_invalid_value_falls_back(policy):
    policy("bogus_policy")
    cache = _cache(E=6, cap=3)
    cache.prefetch([0, 1, 2])
    cache.prefetch([3])
    assert set(cache._lru) == {1, 2, 3}


def _aged(cache, ages):
    pred = Prediction(cache, window=16)
    cache._predictor = pred
    pred._age = dict(ages)
    return pred


def test_least_stale_evicts_most_stale_not_lru_oldest(policy):
    policy("least_stale")
    cache = _cache(E=8, cap=3)
    cache.prefetch([0, 1, 2])
    _aged(cache, {0: 1, 1: 4, 2: 8})
    cache.prefetch([3])
    assert set(cache._lru) == {0, 1, 3}


def test_least_stale_without_predictor_degrades_to_lru(policy):
    policy("least_stale")
    cache = _cache(E=6, cap=3)
    cache.prefetch([0, 1, 2])
    cache.prefetch([3])
    assert set(cache._lru) == {1, 2, 3}


def test_least_stale_never_seen_counts_as_maximally_stale(policy):
    policy("least_stale")
    cache = _cache(E=8, cap=3)
    cache.prefetch([0, 1, 2])
    _aged(cache, {0: 1, 2: 3})
    cache.prefetch([3])
    assert set(cache._lru) == {0, 2, 3}


def test_least_stale_tie_breaks_by_lru_order(policy):
    policy("least_stale")
    cache = _cache(E=8, cap=3)
    cache.prefetch([0, 1, 2])
    _aged(cache, {0: 5, 1: 5, 2: 2})
    cache.prefetch([3])
    assert set(cache._lru) == {1, 2, 3}


def test_least_stale_hard_never_evicted(policy):
    policy("least_stale")
    cache = _cache(E=6, cap=2)
    cache.prefetch([0, 1])
    _aged(cache, {0: 10, 1: 10, 2: 0})
    cache.prefetch([2])
    assert 2 in cache._lru and len(cache._lru) == 2


def test_least_stale_soft_evicted_only_after_stale(policy):
    policy("least_stale")
    cache = _cache(E=8, cap=4)
    cache.prefetch([0, 1, 7])
    cache._next_reserve = frozenset({0, 1})
    _aged(cache, {0: 9, 1: 9, 7: 1})
    cache.prefetch([2, 3])
    assert 7 not in cache._lru and {0, 1, 2, 3} <= set(cache._lru)


def test_least_stale_picks_stalest_soft_when_no_stale_left(policy):
    policy("least_stale")
    cache = _cache(E=6, cap=3)
    cache.prefetch([0, 1])
    cache._next_reserve = frozenset({0, 1})
    _aged(cache, {0: 2, 1: 7})
    cache.prefetch([2, 3])
    assert set(cache._lru) == {0, 2, 3}


def test_lru_oldest_wins_same_scenario(policy):
    policy("lru")
    cache = _cache(E=8, cap=3)
    cache.prefetch([0, 1, 2])
    _aged(cache, {0: 1, 1: 4, 2: 8})
    cache.prefetch([3])
    assert set(cache._lru) == {1, 2, 3}


def test_env_getter_normalizes(monkeypatch):
    for raw, expected in {"least_stale": "least_stale", "LEAST_STALE": "least_stale",
                          "lru": "lru", "garbage": "lru"}.items():
        monkeypatch.setenv("RE_CACHE_POLICY", raw)
        assert env.get_moe_cache_policy() == expected


# ------------------------------------------------------------------ substitution & stats
def test_substitution_serves_most_similar_resident():
    cache = _cache(E=4, cap=4)
    sim = torch.tensor([[1.0, 0.1, 0.9, 0.3],
                        [0.1, 1.0, 0.2, 0.8],
                        [0.9, 0.2, 1.0, 0.1],
                        [0.3, 0.8, 0.1, 1.0]])
    cache.prefetch([0, 3])  # no table yet: two normal loads
    assert cache.stats.misses == 2
    cache.set_sim_table(sim)
    cache.prefetch([2])  # residents {0, 3}: sim[2,0] = 0.9 > sim[2,3] = 0.1
    assert cache.stats.subs == 1 and cache.stats.misses == 2
    assert cache._lru[2][0] is cache._lru[0][0]
    cache.prefetch([1])  # residents {0, 2, 3}: sim[1,3] = 0.8 is the largest
    assert cache.stats.subs == 2 and cache._lru[1][0] is cache._lru[3][0]
    with pytest.raises(ValueError, match="sim_table shape"):
        cache.set_sim_table(torch.zeros(3, 3))


def test_stats_and_report_keys():
    s = OffloadStats(hits=3, misses=1, transfers_bytes=3 * 1024 * 1024)
    d = s.as_dict()
    assert set(d) == {"hits", "misses", "evictions", "subs", "predicts", "inflight_bytes",
                      "transfer_mb"}
    assert d["transfer_mb"] == 3.0
    s.reset()
    assert s.as_dict()["hits"] == 0
    cache = _cache(E=2, cap=2)
    cache.prefetch([0])
    assert cache.report().startswith("offload: hit=0 miss=1 sub=0 pred=0 evict=0 transfer=")


def test_int8_host_bank():
    cache = _cache(E=3, cap=3, H=8, I=4)
    cache.quantize_int8_host()
    assert cache.cpu_split
    q1, q2, s1, s2, idx = cache.cpu_banks([2, 0])
    assert idx == {0: 0, 2: 1} and q1.dtype == torch.int8 and q1.shape == (2, 8, 8)
    w = cache._host[2][0].float()
    assert torch.allclose(q1[1].float() * s1[1], w, atol=float(s1[1]) / 2 + 1e-6)
    assert int(q1.abs().max()) <= 127


def test_int8_bank_follows_a_reloaded_pool():
    """Restaging the pool (load) while the int8 split is armed rebuilds the
    bank from the new weights; quantize_int8_host alone selects the int8 host
    half, as in the reference; the 16-bit split drops the bank."""
    cache = _cache(E=2, cap=2, H=8, I=4)
    cache.enable_host_experts(int8=True)
    assert cache.cpu_split and cache.host_int8
    new = [{"w1": torch.randn(8, 8, dtype=torch.float16) * 5,
            "w2": torch.randn(8, 4, dtype=torch.float16) * 5} for _ in range(2)]
    cache.load(new)
    assert cache.cpu_split and cache.host_int8 and len(cache._int8_host) == 2
    for e in range(2):
        q1, q2, s1, s2 = cache._int8_host[e]
        assert torch.allclose(q1.float() * s1, new[e]["w1"].float(), atol=s1 / 2 + 1e-6)
        assert torch.allclose(q2.float() * s2, new[e]["w2"].float(), atol=s2 / 2 + 1e-6)
        r1, r2 = cache._int8_rowsums[e]
        assert torch.equal(r1, q1.int().sum(dim=1)) and torch.equal(r2, q2.int().sum(dim=1))
    cache.enable_host_experts(int8=False)
    assert cache.cpu_split and not cache.host_int8
    cache.load(new)
    assert cache.cpu_split and not cache.host_int8 and not cache._int8_host
    fresh = _cache(E=2, cap=2, H=8, I=4)
    fresh.quantize_int8_host()
    assert fresh.cpu_split and fresh.host_int8


def test_cpu_shuttle_decay():
    sh = CpuShuttle(n_steps=2)
    sh.send(torch.zeros(4, dtype=torch.float32))  # 16 bytes
    assert sh.inflight_bytes() == 16.0
    sh.send(torch.zeros(0))
    assert sh.inflight_bytes() == 8.0
    sh.advance_step()
    assert sh.inflight_bytes() == 0.0
    sh.send(torch.zeros(2))
    sh.sync()
    assert sh.inflight_bytes() == 0.0


def test_from_config_and_env_defaults(monkeypatch):
    class Cfg:
        device = "cpu"
        dtype = torch.bfloat16

    monkeypatch.setenv("RE_MOE_CACHE_SIZE", "7")
    c = ExpertOffloadCache.from_config(Cfg())
    assert c.lru_capacity == 7 and c.dtype == torch.bfloat16 and c.device == DEVICE
    assert ExpertOffloadCache.from_config(Cfg(), lru_capacity=3).lru_capacity == 3
    monkeypatch.delenv("RE_MAX_PACK", raising=False)
    assert env.get_max_pack(2) == 2 and env.get_max_pack(4) == 4
    assert env.get_chunk_size(0) == int(os.environ.get("RE_CHUNK_SIZE", "0"))
