"""GPU parity of the FusedMoE drop-in (resident, offload and streaming forward).

Reference: FusedMoE (reframework/moe/moe_layer.py:132-660). Routing is
checked bit-exact on the layer's own fp32 logits; outputs against the fp64
oracle within 1e-5 (fp32) / 2e-2 (bf16, f16) max-relative. The offload tests
restate the reference's layer-level lookahead tests
(tests/test_moe_prefetch.py:198-258) on the GPU, and check that the
truncating offload forward equals the oracle with the dropped slots removed.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import ROUND, banner
from oracle import oracle
from reframework_amd import synth
from reframework_amd.moe import FusedMoE

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _build(E, K, H, I, dtype, seed=0, gate_sigma=0.02):
    moe = FusedMoE(num_experts=E, top_k=K, hidden_size=H, intermediate_size=I, dtype=dtype)
    layer = synth.make_layer(synth.MoEShape("t", H, E, K, I), dtype, seed=seed, sigma_w=0.02)
    sd = {"gate.weight": (layer["gate"].double() * (gate_sigma / 0.02)).to(dtype)}
    for e in range(E):
        sd[f"experts.{e}.gate_proj.weight"] = layer["w1"][e][:I]
        sd[f"experts.{e}.up_proj.weight"] = layer["w1"][e][I:]
        sd[f"experts.{e}.down_proj.weight"] = layer["w2"][e]
    moe.load_state_dict(sd)
    return moe


def _oracle_layer(moe_cpu_w1, moe_cpu_w2, x_cpu, logits, K, renorm=True, act=0, round_mode=None,
                  tokens=None):
    w, ids = oracle.topk(logits, K, renorm)
    return oracle.fused_experts(x_cpu, moe_cpu_w1, moe_cpu_w2, w, ids.astype(np.int64),
                                activation=act, inter_round=round_mode or 0, tokens=tokens), ids


@pytest.mark.parametrize("dtype,T", [(torch.float32, 512), (torch.bfloat16, 512),
                                     (torch.float16, 64), (torch.bfloat16, 3)])
def test_tiny_config_layer_matches_oracle(dtype, T, dev):
    """The tiny CPU-reference shape: hidden 1024, 8 experts, top-2, ffn 2816."""
    banner(f"FusedMoE tiny {dtype} T={T}")
    E, K, H, I = 8, 2, 1024, 2816
    moe = _build(E, K, H, I, dtype)
    w1 = [p.detach().clone() for p in moe.experts_w1]
    w2 = [p.detach().clone() for p in moe.experts_w2]
    gate = moe.gate.detach().clone()
    moe = moe.to(dev)
    x = synth.make_tokens(T, H, dtype)
    out = moe(x.to(dev))
    torch.cuda.synchronize()
    assert out.shape == (T, H) and out.dtype == dtype
    rw, rids = moe.route(x.to(dev))
    assert rids.dtype == torch.int64 and rw.dtype == torch.float32
    # routing: bit-exact on the layer's fp32 logits (rounded to the model dtype)
    lg = oracle.router_logits(x, gate, None, round_mode={torch.float32: 0, torch.bfloat16: 1,
                                                           torch.float16: 2}[dtype])
    ow, oids = oracle.topk(lg, K, True)
    agree = (rids.cpu().numpy() == oids).all(1)
    assert agree.mean() > 0.98  # fp32 sums may round a bf16/f16 logit one unit apart
    # outputs: oracle on the kernel's own routing
    ref = oracle.fused_experts(x, w1, w2, rw.cpu().numpy(), rids.cpu().numpy())
    err = oracle.max_rel(out.float().cpu().numpy(), ref)
    print(f"  max_rel {err:.2e}", flush=True)
    assert err <= TOL[dtype]


def test_x_dtype_follows_input_and_1d_input(dev):
    banner("FusedMoE dtype plumbing")
    moe = _build(4, 2, 256, 256, torch.bfloat16).to(dev)
    x = torch.randn(6, 256, generator=torch.Generator().manual_seed(41)).to(dev)
    out = moe(x)
    assert out.dtype == torch.float32 and out.shape == (6, 256)
    out1 = moe(x[0])
    assert out1.shape == (1, 256)
    assert torch.allclose(out1[0], out[0], rtol=0, atol=0)


def test_cpu_input_is_an_error():
    moe = _build(4, 2, 256, 256, torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        moe(torch.randn(2, 256, generator=torch.Generator().manual_seed(43)).to(torch.bfloat16))


def test_offload_forward_truncates_like_reference(dev, monkeypatch):
    """RE_MAX_PACK=2: only the two experts with the largest summed weight run."""
    monkeypatch.delenv("RE_CHUNK_SIZE", raising=False)
    monkeypatch.setenv("RE_MAX_PACK", "2")
    banner("offload forward truncation")
    E, K, H, I, T = 8, 2, 512, 512, 6
    moe = _build(E, K, H, I, torch.bfloat16, gate_sigma=0.2)
    w1 = [p.detach().clone() for p in moe.experts_w1]
    w2 = [p.detach().clone() for p in moe.experts_w2]
    moe.gate.data = moe.gate.data.to(dev)
    moe.build_offload_cache(dev, lru_capacity=4)
    x = synth.make_tokens(T, H, torch.bfloat16).to(dev)
    rw, rids = moe.route(x)
    out = moe(x)
    torch.cuda.synchronize()
    wn, idn = rw.cpu().numpy(), rids.cpu().numpy()
    sums = {}
    for e, v in zip(idn.reshape(-1).tolist(), wn.reshape(-1).tolist()):
        sums[e] = sums.get(e, 0.0) + v
    kept = [e for e, _ in sorted(sums.items(), key=lambda kv: -kv[1])][:2]
    ids_drop = np.where(np.isin(idn, kept), idn, -1)
    ref = oracle.fused_experts(x.cpu(), w1, w2, wn, ids_drop)
    assert oracle.max_rel(out.float().cpu().numpy(), ref) <= 2e-2
    assert moe._cache.resident_set() >= frozenset(kept)


@pytest.mark.parametrize("env", [{"RE_MAX_PACK": "1"}, {"RE_CHUNK_SIZE": "1"}])
def test_offload_steps_with_fewer_experts_than_top_k(env, dev, monkeypatch):
    """A truncated step keeping one expert (RE_MAX_PACK=1) and streaming
    chunks of one expert (RE_CHUNK_SIZE=1) hand the kernels fewer bank rows
    than top_k = 2: the dropped or other-chunk slots are renamed to -1 and
    the output must equal the oracle with exactly those slots removed."""
    monkeypatch.delenv("RE_CHUNK_SIZE", raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    banner(f"offload with fewer experts than top_k: {env}")
    E, K, H, I, T = 8, 2, 256, 512, 5
    moe = _build(E, K, H, I, torch.bfloat16, gate_sigma=0.2)
    w1 = [p.detach().clone() for p in moe.experts_w1]
    w2 = [p.detach().clone() for p in moe.experts_w2]
    moe.gate.data = moe.gate.data.to(dev)
    moe.build_offload_cache(dev, lru_capacity=2)
    x = synth.make_tokens(T, H, torch.bfloat16, seed=4).to(dev)
    rw, rids = moe.route(x)
    out = moe(x)
    torch.cuda.synchronize()
    wn, idn = rw.cpu().numpy(), rids.cpu().numpy()
    if "RE_MAX_PACK" in env:
        sums = {}
        for e, v in zip(idn.reshape(-1).tolist(), wn.reshape(-1).tolist()):
            sums[e] = sums.get(e, 0.0) + v
        kept = max(sums, key=lambda e: sums[e])
        idn = np.where(idn == kept, idn, -1)
    ref = oracle.fused_experts(x.cpu(), w1, w2, wn, idn)
    assert oracle.max_rel(out.float().cpu().numpy(), ref) <= 2e-2


def test_streaming_offload_equals_resident(dev, monkeypatch):
    banner("streaming offload == resident")
    E, K, H, I, T = 8, 2, 512, 512, 40
    ref_moe = _build(E, K, H, I, torch.bfloat16).to(dev)
    x = synth.make_tokens(T, H, torch.bfloat16).to(dev)
    want = ref_moe(x).float()
    moe = _build(E, K, H, I, torch.bfloat16)
    moe.gate.data = moe.gate.data.to(dev)
    moe.build_offload_cache(dev, lru_capacity=3)
    monkeypatch.setenv("RE_CHUNK_SIZE", "3")
    got = moe(x).float()
    torch.cuda.synchronize()
    err = (got - want).abs().max().item() / want.abs().max().item()
    assert err <= 1e-2
    st = moe._cache.stats
    assert st.misses >= E - 3 and st.transfers_bytes > 0


def _routed_moe(dev, E=8):
    """Diagonal gate: a token spiked at dim d routes (top-1) to expert d
    (restates tests/test_moe_prefetch.py:198-218)."""
    torch.manual_seed(0)
    mlp = FusedMoE(num_experts=E, top_k=1, hidden_size=16, intermediate_size=8,
                   dtype=torch.float16)
    with torch.no_grad():
        mlp.gate.fill_(0.0)
        for e in range(E):
            mlp.gate[e, e] = 10.0
        for p in list(mlp.experts_w1) + list(mlp.experts_w2):
            p.normal_(0, 0.1)
    mlp.gate.data = mlp.gate.data.to(dev)
    return mlp


def test_forward_drives_lookahead_reserve(dev):
    banner("lookahead via forward")
    mlp = _routed_moe(dev)
    cache = mlp.build_offload_cache(dev, lru_capacity=4)
    mlp.attach_predictor(window=8)
    cache._bw_gb_s = None  # cap by LRU room only, as on the reference's CPU test box
    assert mlp._predictor is not None and cache._predictor is mlp._predictor

    def spike(d):
        x = torch.zeros(1, 16, dtype=torch.float16, device=dev)
        x[0, d] = 5.0
        return x

    for d in range(5):
        out = mlp(spike(d))
        assert out.shape == (1, 16)
    torch.cuda.synchronize()
    assert cache._next_reserve == frozenset({0})
    assert 0 in cache._lru and 4 in cache._lru
    assert cache.stats.predicts >= 1


def test_forward_prefill_does_not_lookahead(dev):
    banner("prefill resets history")
    mlp = _routed_moe(dev)
    cache = mlp.build_offload_cache(dev, lru_capacity=8)
    mlp.attach_predictor(window=8)
    x = torch.zeros(4, 16, dtype=torch.float16, device=dev)
    for d in range(4):
        x[d, d] = 5.0
    mlp(x)
    torch.cuda.synchronize()
    assert list(mlp._predictor._history) == []
    assert cache.stats.predicts == 0


def test_offload_slot_reuse_keeps_results_correct(dev, monkeypatch):
    """Many steps through a 2-slot cache: evicted slots are refilled while
    earlier kernels may still run; every step must match the resident layer."""
    monkeypatch.delenv("RE_CHUNK_SIZE", raising=False)
    monkeypatch.setenv("RE_MAX_PACK", "8")
    banner("slot reuse under eviction")
    E, K, H, I = 8, 2, 256, 256
    ref = _build(E, K, H, I, torch.bfloat16, seed=3).to(dev)
    moe = _build(E, K, H, I, torch.bfloat16, seed=3)
    moe.gate.data = moe.gate.data.to(dev)
    cache = moe.build_offload_cache(dev, lru_capacity=2)
    cache.measure_bandwidth()
    assert cache._bw_gb_s is None or cache._bw_gb_s > 0
    outs, wants = [], []
    for step in range(12):
        x = synth.make_tokens(1, H, torch.bfloat16, seed=step).to(dev)
        outs.append(moe(x))
        wants.append(ref(x))
    torch.cuda.synchronize()
    for o, w in zip(outs, wants):
        assert torch.allclose(o.float(), w.float(), rtol=0, atol=1e-3 * w.float().abs().max().item())
    assert cache.stats.evictions > 0 and cache._n_slots <= 4


def _build_shared(E, K, H, I, dtype, n_shared=0, shared_I=None, seed=0):
    """A layer with shared experts loaded from the merged HF tensors."""
    moe = FusedMoE(num_experts=E, top_k=K, hidden_size=H, intermediate_size=I, dtype=dtype,
                   n_shared_experts=n_shared, shared_intermediate_size=shared_I)
    layer = synth.make_layer(synth.MoEShape("t", H, E, K, I), dtype, seed=seed, sigma_w=0.02)
    Is = shared_I or n_shared * I
    sh = synth.make_shared(1, H, Is, dtype, seed=seed)
    sd = {"gate.weight": layer["gate"]}
    for e in range(E):
        sd[f"experts.{e}.gate_proj.weight"] = layer["w1"][e][:I]
        sd[f"experts.{e}.up_proj.weight"] = layer["w1"][e][I:]
        sd[f"experts.{e}.down_proj.weight"] = layer["w2"][e]
    sd["shared_experts.gate_proj.weight"] = sh["gate_proj"]
    sd["shared_experts.up_proj.weight"] = sh["up_proj"]
    sd["shared_experts.down_proj.weight"] = sh["down_proj"]
    moe.load_state_dict(sd)
    return moe, layer, sh


@pytest.mark.parametrize("n_shared,shared_I,T", [(2, None, 100), (0, 384, 100), (2, None, 3)])
def test_shared_experts_add_dense_swiglu(n_shared, shared_I, T, dev):
    """out = routed sum + down(silu(x gate^T) * (x up^T)) over every token
    (litemoe/src/litemoe/model/model.py:192-195): folded as extra experts when
    the shared width is a multiple of the expert width (2 x 256), as a second
    fp32-accumulated call otherwise (384)."""
    banner(f"shared experts n={n_shared} Is={shared_I} T={T}")
    E, K, H, I = 16, 4, 512, 256
    moe, layer, sh = _build_shared(E, K, H, I, torch.bfloat16, n_shared, shared_I)
    assert moe._shared_folded == (shared_I is None)
    moe = moe.to(dev)
    x = synth.make_tokens(T, H, torch.bfloat16, seed=5)
    out = moe(x.to(dev))
    rw, rids = moe.route(x.to(dev))
    torch.cuda.synchronize()
    wn, idn = rw.cpu().numpy(), rids.cpu().numpy()
    routed = oracle.fused_experts(x, layer["w1"], layer["w2"], wn, idn, inter_round=ROUND[torch.bfloat16])
    shared = oracle.fused_experts(x, sh["w1"], sh["w2"], np.ones((T, 1), np.float32),
                                  np.zeros((T, 1), np.int64), inter_round=ROUND[torch.bfloat16])
    err = oracle.max_rel(out.float().cpu().numpy(), routed + shared)
    print(f"  max_rel {err:.2e}", flush=True)
    assert err <= 2e-2
    # the shared part is really there: without it the output is far off
    assert oracle.max_rel(out.float().cpu().numpy(), routed) > 0.1


def test_shared_experts_with_streaming_offload(dev, monkeypatch):
    banner("shared experts + streaming offload")
    E, K, H, I, T = 8, 2, 512, 256, 24
    ref_moe, _, _ = _build_shared(E, K, H, I, torch.bfloat16, n_shared=2)
    ref_moe = ref_moe.to(dev)
    x = synth.make_tokens(T, H, torch.bfloat16, seed=2).to(dev)
    want = ref_moe(x).float()
    moe, _, _ = _build_shared(E, K, H, I, torch.bfloat16, n_shared=2)
    moe.gate.data = moe.gate.data.to(dev)
    for p in list(moe.shared_w1) + list(moe.shared_w2):
        p.data = p.data.to(dev)
    moe.build_offload_cache(dev, lru_capacity=3)
    monkeypatch.setenv("RE_CHUNK_SIZE", "3")
    got = moe(x).float()
    monkeypatch.delenv("RE_CHUNK_SIZE")
    monkeypatch.setenv("RE_MAX_PACK", "8")
    got_pack = moe(x).float()
    torch.cuda.synchronize()
    for g in (got, got_pack):
        err = (g - want).abs().max().item() / want.abs().max().item()
        assert err <= 1e-2


def test_checkpoint_loaded_layer_matches_resident_and_offload(dev, tmp_path, monkeypatch):
    """Mixtral-named safetensors -> FusedMoE (resident) and -> pinned pool
    (offload, streamed per expert); both forwards agree with the oracle."""
    from safetensors.torch import save_file

    from reframework_amd.checkpoint import SafetensorsIndex, load_moe_layer, load_moe_layer_offload

    banner("checkpoint adapter on the GPU")
    E, K, H, I, T = 8, 2, 512, 256, 32
    layer = synth.make_layer(synth.MoEShape("t", H, E, K, I), torch.bfloat16, seed=7)
    p = "model.layers.5.block_sparse_moe"
    sd = {f"{p}.gate.weight": layer["gate"]}
    for e in range(E):
        sd[f"{p}.experts.{e}.w1.weight"] = layer["w1"][e][:I].contiguous()
        sd[f"{p}.experts.{e}.w3.weight"] = layer["w1"][e][I:].contiguous()
        sd[f"{p}.experts.{e}.w2.weight"] = layer["w2"][e]
    save_file(sd, str(tmp_path / "model.safetensors"))
    idx = SafetensorsIndex(tmp_path)
    res = FusedMoE(E, K, H, I, dtype=torch.bfloat16)
    assert not load_moe_layer(idx, res, "model.layers.5.mlp").missing
    res = res.to(dev)
    off = FusedMoE(E, K, H, I, dtype=torch.bfloat16)
    off.gate.data = off.gate.data.to(dev)
    cache, rep = load_moe_layer_offload(idx, off, "model.layers.5.mlp", dev, lru_capacity=8)
    assert not rep.missing and cache._pinned
    off.gate.data = off.gate.data.to(dev)
    x = synth.make_tokens(T, H, torch.bfloat16, seed=3).to(dev)
    monkeypatch.setenv("RE_CHUNK_SIZE", "4")
    a, b = res(x), off(x)
    rw, rids = res.route(x)
    torch.cuda.synchronize()
    ref = oracle.fused_experts(x.cpu(), layer["w1"], layer["w2"], rw.cpu().numpy(),
                               rids.cpu().numpy())
    assert oracle.max_rel(a.float().cpu().numpy(), ref) <= 2e-2
    assert oracle.max_rel(b.float().cpu().numpy(), ref) <= 2e-2


def test_shared_pool_across_layers_matches_resident(dev, monkeypatch):
    """Three layers share a 3-slot HBM pool; every step of a chained decode
    must equal the resident layers while slots move between layers."""
    from reframework_amd.moe import ExpertPool

    monkeypatch.delenv("RE_CHUNK_SIZE", raising=False)
    monkeypatch.setenv("RE_MAX_PACK", "8")
    banner("shared expert pool across layers")
    E, K, H, I = 8, 2, 256, 256
    pool = ExpertPool(capacity=3)
    refs, layers = [], []
    for li in range(3):
        refs.append(_build(E, K, H, I, torch.bfloat16, seed=10 + li, gate_sigma=0.2).to(dev))
        m = _build(E, K, H, I, torch.bfloat16, seed=10 + li, gate_sigma=0.2)
        m.gate.data = m.gate.data.to(dev)
        m.build_offload_cache(dev, lru_capacity=2, pool=pool)
        layers.append(m)
    outs, wants = [], []
    for step in range(8):
        x = synth.make_tokens(1, H, torch.bfloat16, seed=100 + step).to(dev)
        y, z = x, x
        for m, r in zip(layers, refs):
            y = m(y)
            z = r(z)
        outs.append(y)
        wants.append(z)
    torch.cuda.synchronize()
    for o, w in zip(outs, wants):
        assert torch.allclose(o.float(), w.float(), rtol=0, atol=2e-3 * w.float().abs().max().item())
    ev = sum(m._cache.stats.evictions for m in layers)
    assert ev > 0 and pool.n_slots <= 3 + 2 and len(pool) <= 3 + 2


def test_layers_sharing_host_pools_match_resident(dev, monkeypatch):
    """Four offloaded layers on two staged host pools (layers 2 and 3 borrow
    the pools of layers 0 and 1 through host_from, each with its own router and
    HBM window): a chained decode equals resident layers that hold the pool
    owners' experts and their own gates."""
    monkeypatch.delenv("RE_CHUNK_SIZE", raising=False)
    monkeypatch.setenv("RE_MAX_PACK", "8")
    banner("offloaded layers sharing host pools")
    E, K, H, I = 8, 2, 256, 256
    refs, layers = [], []
    for li in range(4):
        owner = li % 2
        r = _build(E, K, H, I, torch.bfloat16, seed=20 + owner, gate_sigma=0.2)
        r.gate.data = _build(E, K, H, I, torch.bfloat16, seed=30 + li, gate_sigma=0.2).gate.data
        refs.append(r.to(dev))
        if li < 2:
            m = _build(E, K, H, I, torch.bfloat16, seed=20 + owner, gate_sigma=0.2)
            m.build_offload_cache(dev, lru_capacity=2)
        else:
            m = FusedMoE(num_experts=E, top_k=K, hidden_size=H, intermediate_size=I,
                         dtype=torch.bfloat16)
            m.build_offload_cache(dev, lru_capacity=2, host_from=layers[owner]._cache)
        m.gate.data = refs[li].gate.data.clone()
        layers.append(m)
    assert layers[2]._cache._host_buf is layers[0]._cache._host_buf
    outs, wants = [], []
    for step in range(6):
        x = synth.make_tokens(2, H, torch.bfloat16, seed=200 + step).to(dev)
        y, z = x, x
        for m, r in zip(layers, refs):
            y = m(y)
            z = r(z)
        outs.append(y)
        wants.append(z)
    torch.cuda.synchronize()
    for o, w in zip(outs, wants):
        assert torch.allclose(o.float(), w.float(), rtol=0, atol=2e-3 * w.float().abs().max().item())
    assert all(m._cache.stats.misses > 0 for m in layers)


def test_substitute_aliases_hbm_slot_then_refills(dev, monkeypatch):
    """Similarity substitution on HBM slots (reference: offload_cache.py:713-
    732): a miss served by the most similar resident expert makes the kernels
    read that expert's slot under the missing id (two LRU entries, one slot,
    two references). Once every entry aliasing the slot is evicted, the slot
    goes back to the free list and is refilled with another expert, which the
    kernels then read. Steps are queued without host synchronisation, so the
    refill must wait for the kernels that read the alias; every step's output
    is checked against the oracle with the expert each step really ran."""
    monkeypatch.delenv("RE_CHUNK_SIZE", raising=False)
    monkeypatch.setenv("RE_MAX_PACK", "8")
    banner("substitution aliases an HBM slot, then the slot is refilled")
    E, H, I, T = 8, 256, 512, 4
    layer = synth.make_layer(synth.MoEShape("t", H, E, 1, I), torch.bfloat16, seed=21)
    moe = FusedMoE(num_experts=E, top_k=1, hidden_size=H, intermediate_size=I,
                   dtype=torch.bfloat16)
    sd = {"gate.weight": torch.zeros(E, H, dtype=torch.bfloat16)}
    for e in range(E):
        sd["gate.weight"][e, e] = 10.0  # a token spiked at dim d routes to expert d
        sd[f"experts.{e}.gate_proj.weight"] = layer["w1"][e][:I]
        sd[f"experts.{e}.up_proj.weight"] = layer["w1"][e][I:]
        sd[f"experts.{e}.down_proj.weight"] = layer["w2"][e]
    moe.load_state_dict(sd)
    moe.gate.data = moe.gate.data.to(dev)
    cache = moe.build_offload_cache(dev, lru_capacity=2)

    def tokens(d, seed):
        x = synth.make_tokens(T, H, torch.bfloat16, seed=seed).float() * 0.05
        x[:, d] = 5.0
        return x.to(torch.bfloat16).to(dev)

    sim = torch.zeros(E, E)
    sim[1, 0] = 1.0               # expert 1's miss takes expert 0's slot
    sim[2, 0], sim[2, 1] = 0.5, 0.9  # expert 2's takes expert 1's entry (expert 0's slot)
    # (routed expert, expert whose weights the step runs, sim table on?)
    plan = [(0, 0, False), (1, 0, True), (2, 0, True), (3, 3, False), (4, 4, False),
            (5, 5, False), (1, 1, False), (5, 5, False)]
    outs, xs = [], []
    slot_a = None
    for step, (d, _, use_sim) in enumerate(plan):
        cache.sim_table = sim if use_sim else None
        x = tokens(d, seed=step)
        xs.append(x)
        outs.append(moe(x))
        if step == 0:
            slot_a = cache._slot_of[0]
        if step == 2:
            # entries 1 and 2 alias expert 0's slot; entry 0 was evicted
            assert cache._slot_of[2] is slot_a and slot_a.refs == 2 and 0 not in cache._lru
        if step == 4:
            # the last alias (entry 2) is evicted before the miss is copied,
            # so expert 4 is copied into the same slot; the layer never holds
            # more than its 2 slots
            assert cache._slot_of[4] is slot_a and slot_a.refs == 1
            assert cache._n_slots == 2
    torch.cuda.synchronize()
    assert cache.stats.subs == 2
    for step, (d, ran, _) in enumerate(plan):
        x = xs[step].cpu()
        ref = oracle.fused_experts(x, [layer["w1"][ran]], [layer["w2"][ran]],
                                   np.ones((T, 1), np.float32), np.zeros((T, 1), np.int64))
        err = oracle.max_rel(outs[step].float().cpu().numpy(), ref)
        print(f"  step {step}: routed {d}, ran expert {ran}: max_rel {err:.2e}", flush=True)
        assert err <= 2e-2


def test_shared_pool_with_lookahead_matches_resident(dev, monkeypatch):
    """Layers sharing one small ExpertPool, each with a predictor: the
    lookahead loads experts on its layer's copy stream, and the next layer's
    requests evict many of them from the pool before anything reads them;
    their slots are then refilled on another layer's copy stream. Each refill
    must wait for the copy still filling the slot as well as for the slot's
    readers: every step of a chained decode must equal the resident layers."""
    from reframework_amd.moe import ExpertPool

    monkeypatch.delenv("RE_CHUNK_SIZE", raising=False)
    monkeypatch.setenv("RE_MAX_PACK", "8")
    banner("shared pool + lookahead across layers")
    E, K, H, I, n_layers = 8, 2, 1024, 1024, 3
    pool = ExpertPool(capacity=4)
    refs, layers = [], []
    for li in range(n_layers):
        refs.append(_build(E, K, H, I, torch.bfloat16, seed=30 + li, gate_sigma=0.2).to(dev))
        m = _build(E, K, H, I, torch.bfloat16, seed=30 + li, gate_sigma=0.2)
        m.gate.data = m.gate.data.to(dev)
        m.build_offload_cache(dev, lru_capacity=2, pool=pool)
        m.attach_predictor(window=4)
        m._cache._bw_gb_s = None  # lookahead bounded by pool room only
        layers.append(m)
    outs, wants = [], []
    for step in range(16):
        x = synth.make_tokens(1, H, torch.bfloat16, seed=200 + step).to(dev)
        y, z = x, x
        for m, r in zip(layers, refs):
            y = m(y)
            z = r(z)
        outs.append(y)
        wants.append(z)
    torch.cuda.synchronize()
    predicts = sum(m._cache.stats.predicts for m in layers)
    evictions = sum(m._cache.stats.evictions for m in layers)
    print(f"  predicts {predicts}, evictions {evictions}, slots {pool.n_slots}", flush=True)
    assert predicts > 0 and evictions > 0
    for o, w in zip(outs, wants):
        assert torch.allclose(o.float(), w.float(), rtol=0, atol=2e-3 * w.float().abs().max().item())


@pytest.mark.parametrize("mode", ["resident", "offload", "streaming", "split", "split_int8",
                                  "with_norm"])
def test_zero_tokens_on_every_forward_path(mode, dev, monkeypatch):
    """An empty batch [0, H] gives an empty [0, H] output on every forward
    path, as the reference's does (its route, top-k and per-expert loop run
    on empty tensors: moe_layer.py:320-344, 451-519, 523-627), and a batch
    after it is still right."""
    banner(f"zero tokens, {mode}")
    E, K, H, I = 8, 2, 256, 512
    dtype = torch.bfloat16
    monkeypatch.setenv("RE_MAX_PACK", "2")
    monkeypatch.delenv("RE_CHUNK_SIZE", raising=False)
    moe = _build(E, K, H, I, dtype)
    w1 = [p.detach().clone() for p in moe.experts_w1]
    w2 = [p.detach().clone() for p in moe.experts_w2]
    if mode in ("resident", "with_norm"):
        moe = moe.to(dev)
    else:
        moe.gate.data = moe.gate.data.to(dev)
        moe.build_offload_cache(dev, lru_capacity=8)
        if mode == "streaming":
            monkeypatch.setenv("RE_CHUNK_SIZE", "4")
        if mode.startswith("split"):
            moe.enable_cpu_split(int8=mode.endswith("int8"))
    x0 = torch.empty(0, H, dtype=dtype, device=dev)
    if mode == "with_norm":
        from reframework_amd.layers import RMSNorm
        norm = RMSNorm(H, 1e-6).to(dev)
        out, res = moe.forward_with_norm(x0, torch.empty_like(x0), norm)
        assert res.shape == (0, H)
    else:
        out = moe(x0)
    torch.cuda.synchronize()
    assert out.shape == (0, H) and out.dtype == dtype
    # the layer still works on the next batch: with every expert resident
    # (capacity 8) the output is the full layer's
    x = synth.make_tokens(5, H, dtype, seed=4)
    if mode.startswith("split") or mode in ("offload", "streaming"):
        monkeypatch.setenv("RE_MAX_PACK", "8")
    rw, rids = moe.route(x.to(dev))
    got = moe(x.to(dev)).float().cpu().numpy()
    assert got.shape == (5, H)
    if mode == "split_int8":
        return  # host experts on int8 codes: checked against the int8 oracle in test_gpu_split
    ref = oracle.fused_experts(x, w1, w2, rw.cpu().numpy(), rids.cpu().numpy())
    assert oracle.max_rel(got, ref) <= TOL[dtype]


@pytest.mark.parametrize("E,K,renorm,T", [(128, 8, True, 300), (128, 8, False, 5), (256, 8, True, 64)])
def test_many_experts_layer_matches_oracle(E, K, renorm, T, dev):
    """Many small experts with top-8 (Qwen3-MoE's 128, the library's maximum
    of 256), with and without renormalised weights, through FusedMoE.forward:
    routing bit-exact on the layer's own fp32 logits except near-ties, output
    within the bf16 bar of the oracle on the layer's routing."""
    banner(f"FusedMoE E={E} K={K} renorm={renorm} T={T}")
    H, I, dtype = 512, 256, torch.bfloat16
    moe = FusedMoE(num_experts=E, top_k=K, hidden_size=H, intermediate_size=I, dtype=dtype,
                   renormalize=renorm)
    layer = synth.make_layer(synth.MoEShape("t", H, E, K, I), dtype, seed=E + T, sigma_w=0.02)
    sd = {"gate.weight": layer["gate"]}
    for e in range(E):
        sd[f"experts.{e}.gate_proj.weight"] = layer["w1"][e][:I]
        sd[f"experts.{e}.up_proj.weight"] = layer["w1"][e][I:]
        sd[f"experts.{e}.down_proj.weight"] = layer["w2"][e]
    moe.load_state_dict(sd)
    gate = moe.gate.detach().clone()
    moe = moe.to(dev)
    x = synth.make_tokens(T, H, dtype, seed=T)
    out = moe(x.to(dev))
    rw, rids = moe.route(x.to(dev))
    torch.cuda.synchronize()
    lg = oracle.router_logits(x, gate, None, round_mode=1)
    ow, oids = oracle.topk(lg, K, renorm)
    assert (rids.cpu().numpy() == oids).all(1).mean() > 0.95
    if not renorm:
        # softmax over all experts, not renormalised: the kept weights sum below 1
        assert float(rw.sum(1).max()) < 1.0
    ref = oracle.fused_experts(x, layer["w1"], layer["w2"], rw.cpu().numpy(), rids.cpu().numpy())
    err = oracle.max_rel(out.float().cpu().numpy(), ref)
    print(f"  max_rel {err:.2e}", flush=True)
    assert err <= TOL[dtype]
