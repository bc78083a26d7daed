"""GPU parity of the expert-offload decode at Mixtral-8x7B shape.

A stack of offloaded Mixtral-shape layers (H=4096, I=14336, 8 experts, top-2,
bf16: 352 MB per expert, staged in pinned host memory) decodes 8 tokens per
step through the routing trace of the offload benchmark (per layer and token:
p=0.7 the previous step's pair, else two experts from Zipf(1.2)). Each step's
input is a fresh [8, 4096] batch chained through the layers, as a decode step
is. Reference: FusedMoE.forward over an ExpertOffloadCache
(reframework/moe/moe_layer.py:354-447, 451-519, 523-627; offload_cache.py:
478-507, 654-711).

Every mode is checked twice:
  * every token of every (step, layer) output against the fp64 oracle on that
    layer's actual input and that step's routing, with the slots the forward
    drops removed (RE_MAX_PACK truncation): <= 2e-2 max-relative, and every
    element within its own bf16 rounding plus the oracle's fp32 bound
    (intermediate rounded to bf16, y in fp32 at this size);
  * hits, misses and evictions of every layer against a brute-force replay of
    the same requests (tests/_offload_replay.py), and the HBM slots used
    against max(capacity, largest request).
Modes: per-layer LRU of 2 experts and one pool of 2 per layer shared by all
layers, each with the truncating forward (RE_MAX_PACK=2) and the exact
streaming forward (RE_CHUNK_SIZE=2 / 1); and the CPU/GPU split forward, where
the experts not resident run on the host cores (its residency depends on copy
timing, so only outputs, counts that must add up, and the slot bound are
checked), with the 16-bit host half and with the int8 one. The int8 host
half has the reference's int8 numerics (fused_experts_cpu_int8, fused.py:
140-197): its experts are checked against the oracle's int8 restatement on the
slots each host call was given, the rest against the fp64 oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import ROUND, assert_matches_rounded, banner, y_round_of
from _offload_replay import LruReplay, PoolReplay, chunked_requests, truncated_request
from oracle import oracle
from reframework_amd import _capi, synth
from reframework_amd.moe import ExpertPool, FusedMoE

pytestmark = pytest.mark.gpu

H, I, E, K = 4096, 14336, 8, 2
N_LAYERS, T, STEPS = 4, 8, 8


@pytest.fixture(scope="module")
def stack(dev):
    g = torch.Generator(device=dev).manual_seed(0)
    layers = []
    for _ in range(N_LAYERS):
        moe = FusedMoE(E, K, H, I, dtype=torch.bfloat16).to(dev)
        with torch.no_grad():
            for prm in moe.parameters():
                prm.copy_(torch.randn(prm.shape, generator=g, device=dev) * 0.02)
        moe.build_offload_cache(dev, lru_capacity=2)
        assert moe._cache._pinned
        layers.append(moe)
    ids, w = synth.offload_trace(N_LAYERS, STEPS, T, E, seed=5)
    xs = [synth.make_tokens(T, H, torch.bfloat16, seed=100 + st) for st in range(STEPS)]
    yield {"layers": layers, "ids": ids, "w": w, "xs": xs}
    for moe in layers:
        moe._cache.use_pool(None)
    layers.clear()
    torch.cuda.empty_cache()


class _Routed:
    """Feeds a layer's forward this step's routing from the trace instead of
    its router (the benchmark's routing bypasses the router too)."""

    def __init__(self, moe):
        self.moe = moe
        self.route = None

    def __call__(self, xd, with_shared_cols=False):
        return self.route


MODES = [
    # name, residency, forward, RE_CHUNK_SIZE
    ("per_layer_truncate", "per_layer", "truncate", None),
    ("per_layer_exact_chunk2", "per_layer", "exact", 2),
    ("pool_truncate", "pool", "truncate", None),
    ("pool_exact_chunk1", "pool", "exact", 1),
    ("per_layer_split_truncate", "per_layer", "split", None),
    ("per_layer_split_int8_truncate", "per_layer", "split_int8", None),
]


@pytest.mark.parametrize("mode", MODES, ids=lambda m: m[0])
def test_offload_decode_mixtral_shape(mode, stack, dev, monkeypatch):
    name, residency, fwd, chunk = mode
    layers, ids, w, xs = stack["layers"], stack["ids"], stack["w"], stack["xs"]
    monkeypatch.setenv("RE_MAX_PACK", "2")
    if chunk:
        monkeypatch.setenv("RE_CHUNK_SIZE", str(chunk))
    else:
        monkeypatch.delenv("RE_CHUNK_SIZE", raising=False)
    pool = ExpertPool(capacity=2 * N_LAYERS) if residency == "pool" else None
    banner(f"offload decode mixtral shape: {name}, {N_LAYERS} layers x {STEPS} steps, T={T}")
    routers = []
    for moe in layers:
        moe._cache.use_pool(pool)
        moe._cache.stats.reset()
        moe._cpu_split_enabled = False
        if fwd.startswith("split"):
            moe.enable_cpu_split(int8=fwd == "split_int8")
        r = _Routed(moe)
        monkeypatch.setattr(moe, "_route32", r)
        routers.append(r)
    # the int8 host half: which experts ran on the host, with which slots, per forward
    host_calls = {}
    if fwd == "split_int8":
        code_of = [{m._cache._int8_host[e][0].data_ptr(): e for e in range(E)} for m in layers]
        real = _capi.host_experts_int8
        current = {}

        def record(x, w1q, *args, **kw):
            host_calls.setdefault(current["n"], []).append(
                ([code_of[current["li"]][q.data_ptr()] for q in w1q], args[5].copy(),
                 args[6].copy(), args[7].copy()))
            return real(x, w1q, *args, **kw)

        monkeypatch.setattr(_capi, "host_experts_int8", record)
    ins, outs = [], []
    try:
        for st in range(STEPS):
            y = xs[st].to(dev)
            for li, moe in enumerate(layers):
                routers[li].route = (torch.from_numpy(w[st, li]).to(dev),
                                     torch.from_numpy(ids[st, li]).to(dev))
                ins.append(y)
                if fwd == "split_int8":
                    current.update(n=len(outs), li=li)
                y = moe(y)
                outs.append(y)
        torch.cuda.synchronize()
    finally:
        for moe in layers:
            moe._cpu_split_enabled = False
            moe._cache._cpu_split = False
            moe._cache._host_int8 = False
    print(f"  forwards done: {len(outs)}", flush=True)

    # residency decisions against the brute-force replay
    biggest = 2 if fwd != "exact" else chunk
    if fwd.startswith("split"):
        runs = sum(len(truncated_request(ids[st, li], w[st, li], 2))
                   for st in range(STEPS) for li in range(N_LAYERS))
        st_ = [m._cache.stats for m in layers]
        hits, host = sum(s.hits for s in st_), sum(s.host_experts for s in st_)
        print(f"  split: {hits} experts on the GPU, {host} on the host, "
              f"{sum(s.misses for s in st_)} copied", flush=True)
        assert hits + host == runs and host > 0
    else:
        replay = [LruReplay(2) for _ in range(N_LAYERS)] if pool is None else \
            PoolReplay(2 * N_LAYERS, N_LAYERS)
        for st in range(STEPS):
            for li in range(N_LAYERS):
                reqs = [truncated_request(ids[st, li], w[st, li], 2)] if fwd == "truncate" \
                    else chunked_requests(ids[st, li], chunk)
                for req in reqs:
                    if pool is None:
                        replay[li].admit(req)
                    else:
                        replay.admit(li, req)
        for li, moe in enumerate(layers):
            s = moe._cache.stats
            want = (replay[li].hits, replay[li].misses, replay[li].evictions) if pool is None \
                else (replay.hits[li], replay.misses[li], replay.evictions[li])
            assert (s.hits, s.misses, s.evictions) == want, (li, (s.hits, s.misses, s.evictions))
        print(f"  hits/misses/evictions match the replay", flush=True)
    slots = pool.n_slots if pool is not None else max(m._cache._n_slots for m in layers)
    assert slots <= (max(pool.capacity, biggest) if pool is not None else max(2, biggest))

    # every token of every (step, layer) against the oracle
    plan = _capi.make_plan(T, H, I, 2, K, _capi.BF16)
    assert y_round_of(plan, torch.bfloat16) == 0  # decode path: y stays fp32
    worst = 0.0
    for st in range(STEPS):
        for li, moe in enumerate(layers):
            n = st * N_LAYERS + li
            x_in = ins[n].cpu()
            ii = ids[st, li].astype(np.int64)
            if fwd != "exact":
                kept = truncated_request(ids[st, li], w[st, li], 2)
                ii = np.where(np.isin(ii, kept), ii, -1)
            host = moe._cache._host
            w1 = [host[e][0] for e in range(E)]
            w2 = [host[e][1] for e in range(E)]
            got = outs[n].float().cpu().numpy().astype(np.float64)
            int8_part = 0.0
            if fwd == "split_int8":
                # the host experts with the reference's int8 numerics (the oracle's
                # restatement, which the host library matches bit for bit); the
                # GPU part on the others
                on_host = [e for c in host_calls.get(n, []) for e in c[0]]
                want = sorted((t, e) for t in range(T) for e in ii[t] if e in on_host)
                seen = sorted((int(tk), e) for ids_c, offs, toks, _ in host_calls.get(n, [])
                              for k, e in enumerate(ids_c) for tk in toks[offs[k]:offs[k + 1]])
                assert seen == want, (st, li)
                for ids_c, offs, toks, wts in host_calls.get(n, []):
                    bank = [moe._cache._int8_host[e] for e in ids_c]
                    int8_part = int8_part + oracle.experts_int8(
                        x_in, [b[0].numpy() for b in bank], [b[1].numpy() for b in bank],
                        [b[2] for b in bank], [b[3] for b in bank], offs, toks, wts, 0)
                ii = np.where(np.isin(ii, on_host), -1, ii)
            exact = oracle.fused_experts(x_in, w1, w2, w[st, li], ii) + int8_part
            err = oracle.max_rel(got, exact)
            worst = max(worst, err)
            assert err <= 2e-2, (st, li, err)
            rounded, allow = oracle.fused_experts_bound(x_in, w1, w2, w[st, li], ii, 0,
                                                        ROUND[torch.bfloat16])
            assert_matches_rounded(got, rounded + int8_part, allow, torch.bfloat16)
    print(f"  {STEPS * N_LAYERS} layer outputs x {T} tokens: worst max_rel vs fp64 {worst:.2e}",
          flush=True)
