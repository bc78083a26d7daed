"""GPU parity of the CPU/GPU split forward beyond the Mixtral-shape decode of
test_gpu_offload_mixtral.py: other dtypes, shared experts, every routed
expert (RE_CHUNK_SIZE), and token counts past the zero-copy staging buffer
(the layer then moves routing, hidden states and the host half with ordinary
copies).

Reference: FusedMoE._forward_split (reframework/moe/moe_layer.py:523-627),
with the experts the offload forward would run (RE_MAX_PACK truncation or
every routed expert), each slot's output on its own token. Every step's
output is checked against the fp64 oracle with the dropped slots removed:
<= 2e-2 max-relative for bf16/f16, <= 1e-5 for fp32. The layer's 2-slot
window guarantees that some experts of every step run on the host and some,
resident from earlier steps, on the GPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import banner
from _offload_replay import truncated_request
from oracle import oracle
from reframework_amd import _capi, synth
from reframework_amd.moe import FusedMoE

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _layer(E, K, H, I, dtype, seed, n_shared=0):
    moe = FusedMoE(num_experts=E, top_k=K, hidden_size=H, intermediate_size=I, dtype=dtype,
                   n_shared_experts=n_shared)
    layer = synth.make_layer(synth.MoEShape("t", H, E, K, I), dtype, seed=seed, sigma_w=0.02)
    sd = {"gate.weight": (layer["gate"].double() * 10.0).to(dtype)}
    for e in range(E):
        sd[f"experts.{e}.gate_proj.weight"] = layer["w1"][e][:I]
        sd[f"experts.{e}.up_proj.weight"] = layer["w1"][e][I:]
        sd[f"experts.{e}.down_proj.weight"] = layer["w2"][e]
    sh = None
    if n_shared:
        sh = synth.make_shared(1, H, n_shared * I, dtype, seed=seed)
        sd["shared_experts.gate_proj.weight"] = sh["gate_proj"]
        sd["shared_experts.up_proj.weight"] = sh["up_proj"]
        sd["shared_experts.down_proj.weight"] = sh["down_proj"]
    moe.load_state_dict(sd)
    return moe, layer, sh


@pytest.mark.parametrize("dtype,T,H,I,exact,n_shared", [
    (torch.bfloat16, 8, 512, 512, False, 0),
    (torch.float16, 5, 512, 768, False, 0),
    (torch.float32, 6, 256, 512, False, 0),
    (torch.bfloat16, 8, 512, 512, True, 0),
    (torch.bfloat16, 4, 512, 256, False, 2),
    # past the 8 MB staging buffer at this width: ordinary copies
    (torch.bfloat16, 3000, 512, 256, False, 0),
])
def test_split_forward_matches_oracle(dtype, T, H, I, exact, n_shared, dev, monkeypatch):
    E, K = 8, 2
    monkeypatch.setenv("RE_MAX_PACK", "2")
    if exact:
        monkeypatch.setenv("RE_CHUNK_SIZE", "8")
    else:
        monkeypatch.delenv("RE_CHUNK_SIZE", raising=False)
    staged = T * (H * (4 + torch.tensor([], dtype=dtype).element_size()) + 2 * K * 4) + 4096 \
        <= _capi.HostStaging.CAPACITY
    banner(f"split forward {dtype} T={T} H={H} I={I} exact={exact} shared={n_shared} "
           f"staged={staged}")
    moe, layer, sh = _layer(E, K, H, I, dtype, seed=T + H, n_shared=n_shared)
    moe.gate.data = moe.gate.data.to(dev)
    for p in list(moe.shared_w1) + list(moe.shared_w2):
        p.data = p.data.to(dev)
    cache = moe.build_offload_cache(dev, lru_capacity=2)
    moe.enable_cpu_split()
    assert moe.cpu_split
    outs, xs, routes = [], [], []
    for step in range(5):
        x = synth.make_tokens(T, H, dtype, seed=100 + step).to(dev)
        xs.append(x)
        routes.append(moe.route(x))
        outs.append(moe(x))
    torch.cuda.synchronize()
    st = cache.stats
    print(f"  {st.hits} experts on the GPU, {st.host_experts} on the host, {st.misses} copied",
          flush=True)
    assert st.host_experts > 0 and st.hits > 0
    assert cache._n_slots <= 2 or exact
    for step in range(5):
        wn, idn = (t.cpu().numpy() for t in routes[step])
        if not exact:
            kept = truncated_request(idn, wn, 2)
            idn = np.where(np.isin(idn, kept), idn, -1)
        x = xs[step].cpu()
        ref = oracle.fused_experts(x, layer["w1"], layer["w2"], wn, idn)
        if n_shared:
            ref = ref + oracle.fused_experts(x, sh["w1"], sh["w2"], np.ones((T, 1), np.float32),
                                             np.zeros((T, 1), np.int64))
        err = oracle.max_rel(outs[step].float().cpu().numpy(), ref)
        print(f"  step {step}: max_rel {err:.2e}", flush=True)
        assert err <= TOL[dtype]


@pytest.mark.parametrize("exact", [False, True])
def test_split_forward_int8_host_half_matches_oracle(exact, dev, monkeypatch):
    """The split with the int8 host bank (the reference's numerics for the
    host half, fused_experts_cpu_int8, fused.py:140-197): every step equals
    the fp64 oracle on the experts that ran on the GPU plus the int8 oracle
    on the ones that ran on the host (recorded from the host calls), within
    the bf16 bar. The bf16 host path's bar alone would not hold: the int8
    half is ~4-5 % off the exact layer."""
    E, K, T, H, I = 8, 2, 8, 512, 512
    dtype = torch.bfloat16
    monkeypatch.setenv("RE_MAX_PACK", "2")
    if exact:
        monkeypatch.setenv("RE_CHUNK_SIZE", "8")
    else:
        monkeypatch.delenv("RE_CHUNK_SIZE", raising=False)
    banner(f"split forward, int8 host half, exact={exact}")
    moe, layer, _ = _layer(E, K, H, I, dtype, seed=3)
    moe.gate.data = moe.gate.data.to(dev)
    cache = moe.build_offload_cache(dev, lru_capacity=2)
    moe.enable_cpu_split(int8=True)
    assert moe.cpu_split and cache.host_int8
    code_of = {cache._int8_host[e][0].data_ptr(): e for e in range(E)}
    calls = []
    real = _capi.host_experts_int8

    def record(x, w1q, *args, **kw):
        calls.append(([code_of[q.data_ptr()] for q in w1q], args[5].copy(), args[6].copy(),
                      args[7].copy()))
        return real(x, w1q, *args, **kw)

    monkeypatch.setattr(_capi, "host_experts_int8", record)
    outs, xs, routes, host = [], [], [], []
    for step in range(5):
        x = synth.make_tokens(T, H, dtype, seed=200 + step).to(dev)
        xs.append(x)
        routes.append(moe.route(x))
        n = len(calls)
        outs.append(moe(x))
        host.append(calls[n:])
    torch.cuda.synchronize()
    assert cache.stats.host_experts > 0 and cache.stats.hits > 0
    for step in range(5):
        wn, idn = (t.cpu().numpy() for t in routes[step])
        if not exact:
            kept = truncated_request(idn, wn, 2)
            idn = np.where(np.isin(idn, kept), idn, -1)
        x = xs[step].cpu()
        on_host = [e for c in host[step] for e in c[0]]
        ref = oracle.fused_experts(x, layer["w1"], layer["w2"], wn,
                                   np.where(np.isin(idn, on_host), -1, idn))
        for ids_c, offs, toks, wts in host[step]:
            bank = [cache._int8_host[e] for e in ids_c]
            ref = ref + oracle.experts_int8(x, [b[0].numpy() for b in bank],
                                            [b[1].numpy() for b in bank], [b[2] for b in bank],
                                            [b[3] for b in bank], offs, toks, wts, 0)
        # the host calls cover exactly the kept slots of the host experts
        want = sorted((t, e) for t in range(T) for e in idn[t] if e in on_host)
        got = sorted((int(tk), e) for ids_c, offs, toks, _ in host[step]
                     for k, e in enumerate(ids_c) for tk in toks[offs[k]:offs[k + 1]])
        assert got == want
        err = oracle.max_rel(outs[step].float().cpu().numpy(), ref)
        print(f"  step {step}: {len(on_host)} experts on the host, max_rel {err:.2e}", flush=True)
        assert err <= TOL[dtype]


@pytest.mark.parametrize("dtype,T,K,E,H,I", [
    (torch.bfloat16, 37, 2, 8, 512, 768),
    (torch.float16, 300, 2, 8, 256, 512),
    (torch.float32, 16, 6, 12, 256, 128),
])
def test_masked_halves_match_oracle(dtype, T, K, E, H, I, dev):
    """The split's halves as the reference's module functions
    (fused_experts_masked on the GPU, fused_experts_cpu_int8 on the host,
    fused.py:90-197) over complementary masks: the GPU half within the bar of
    the fp64 oracle on its active slots (tokens without one exactly zero),
    and the sum of both halves within the bar of the oracle's fp64 GPU part
    plus its int8 host part."""
    from reframework_amd.moe.fused import fused_experts_cpu_int8, fused_experts_masked
    banner(f"masked halves {dtype} T={T} K={K} E={E} H={H} I={I}")
    g = torch.Generator().manual_seed(T + E)
    w1 = [(torch.randn(2 * I, H, generator=g) * 0.05).to(dtype) for _ in range(E)]
    w2 = [(torch.randn(H, I, generator=g) * 0.05).to(dtype) for _ in range(E)]
    x = (torch.randn(T, H, generator=g) * 0.7).to(dtype)
    rng = np.random.default_rng(T * K)
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.random((T, K)).astype(np.float32)
    on_gpu = rng.random((T, K)) < 0.5
    on_gpu[0] = False  # a token with no GPU slot
    out = fused_experts_masked(x.to(dev), torch.stack(w1).to(dev), torch.stack(w2).to(dev),
                               torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                               torch.from_numpy(on_gpu).to(dev))
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == (T, H)
    got = out.float().cpu().numpy()
    ref = oracle.fused_experts(x, w1, w2, w, np.where(on_gpu, ids, -1))
    err = oracle.max_rel(got, ref)
    print(f"  GPU half: max_rel {err:.2e}", flush=True)
    assert err <= TOL[dtype]
    assert not got[~on_gpu.any(axis=1)].any()
    # the host half over the other slots, from int8 banks
    q1 = [_capi.host_quantize_int8(a) for a in w1]
    q2 = [_capi.host_quantize_int8(b) for b in w2]
    w1q, w2q = torch.stack([q[0] for q in q1]), torch.stack([q[0] for q in q2])
    s1 = torch.tensor([q[1] for q in q1], dtype=torch.float32)
    s2 = torch.tensor([q[1] for q in q2], dtype=torch.float32)
    on_host = ~on_gpu
    host = fused_experts_cpu_int8(x.to(dev), w1q, w2q, s1, s2, torch.from_numpy(w).to(dev),
                                  torch.from_numpy(ids).to(dev), torch.from_numpy(on_host).to(dev))
    used, offs, toks, wts = [], [0], [], []
    for e in range(E):
        t, k = np.nonzero(on_host & (ids == e))
        if len(t):
            used.append(e)
            toks += t.tolist()
            wts += w[t, k].tolist()
            offs.append(len(toks))
    ref_host = oracle.experts_int8(x, [w1q[e].numpy() for e in used],
                                   [w2q[e].numpy() for e in used], [float(s1[e]) for e in used],
                                   [float(s2[e]) for e in used], np.asarray(offs, np.int32),
                                   np.asarray(toks, np.int32), np.asarray(wts, np.float32))
    assert np.array_equal(host.numpy(), ref_host)
    total = (out.float() + host.to(dev)).to(dtype).float().cpu().numpy()
    err = oracle.max_rel(total, ref + ref_host)
    print(f"  both halves: max_rel {err:.2e}", flush=True)
    assert err <= TOL[dtype]
