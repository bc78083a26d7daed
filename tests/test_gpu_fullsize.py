"""GPU parity of the 256-token-tile grouped GEMM at full size and on the
shapes whose last round is split along K.

Reference: fused_experts (reframework/moe/fused.py:49-87). The tiled gate_up
and down run their items on one workgroup per CU; the items of a last,
partly filled round are cut along K over the idle CUs, their fp32 partial
tiles summed (and activated, for gate_up) by a fix-up kernel. These tests
build routings whose tile counts put that split on (checked with the host
replica of its rule), and compare sampled tokens with the fp64 oracle: the
tokens at the first, middle and last row of every token tile of the tile map
(the tiles' rows and heights by the permute's rules, which
test_gpu_experts.py checks against the map the kernel writes), so every tile
of every launch is checked, plus a few random tokens:
  * <= 2e-2 max-relative against the fp64 oracle;
  * against the oracle that rounds the intermediate (and, for the tiled
    paths with one down K-split, y) like the kernels: every element within
    its own output rounding plus 1e-3 (bf16) / 5e-4 (f16) of the largest
    output; and the output follows that rounding of y, not the other one.
The full-size cases are the Mixtral-8x7B layer (H=4096, I=14336, E=8, K=2) at
T=4096 and 256, the Phi-3.5-MoE layer at T=2048 with Zipf-skewed routing, and
the fine-grained layer (64 experts top-6 plus 2 shared) at T=4096 and 8, and
the Mixtral decode sizes T=1 and 16 on the weight-streaming path (K-split down
projection; at T=1 the gate_up workgroups group the slots themselves): the
shapes the throughput figures are quoted on. The Mixtral cases route with the
router kernel on the biased logits of the throughput workload, its ids checked
bit-exact on its own fp32 logits, so the whole path of each figure is checked.
Each comparison also asserts which rounding of y the plan's kernels apply.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import (ROUND, assert_matches_rounded, assert_y_rounding, banner, gpu_fused,
                      read_ws, tile_height, tiled_down_split, tiled_gate_up_split, y_round_of)
from oracle import oracle
from reframework_amd import _capi, synth

pytestmark = pytest.mark.gpu


def _bank(E, H, I, dtype, seed, dev, used=None, scale=0.05):
    """Per-expert CPU weights; experts outside `used` are zeros (never read
    by a correct kernel). Generated on the GPU for speed."""
    g = torch.Generator(device=dev).manual_seed(seed)
    w1, w2 = [], []
    for e in range(E):
        if used is not None and e not in used:
            w1.append(torch.zeros(2 * I, H, dtype=dtype))
            w2.append(torch.zeros(H, I, dtype=dtype))
            continue
        w1.append((torch.randn(2 * I, H, generator=g, device=dev) * scale).to(dtype).cpu())
        w2.append((torch.randn(H, I, generator=g, device=dev) * scale).to(dtype).cpu())
    return w1, w2


@pytest.fixture(scope="module")
def mixtral(dev):
    """The Mixtral-8x7B layer of the throughput workload: H=4096, I=14336,
    E=8, K=2, bf16 weights N(0, 0.02), router gate N(0, 0.02) with the fixed
    per-expert logit bias N(0, 0.5^2); CPU copies for the oracle, device
    copies for the kernels, shared by the Mixtral tests of this module."""
    H, I, E, K = 4096, 14336, 8, 2
    w1, w2 = _bank(E, H, I, torch.bfloat16, seed=13, dev=dev, scale=0.02)
    gate = (torch.randn(E, H, generator=torch.Generator().manual_seed(14)) * 0.02).to(
        torch.bfloat16)
    bias = synth.mixtral_router_bias(E)
    m = {"H": H, "I": I, "E": E, "K": K, "w1": w1, "w2": w2, "gate": gate, "bias": bias,
         "w1d": [w.to(dev) for w in w1], "w2d": [w.to(dev) for w in w2],
         "gate_d": gate.to(dev), "bias_d": bias.to(dev)}
    yield m
    m.clear()
    torch.cuda.empty_cache()


def _route_biased(m, x_d):
    """Router kernel on the throughput workload's biased logits (logits
    rounded to bf16, as the reference's F.linear returns them, then the fp32
    bias; softmax top-2, renormalised): (w, ids int32, logits) on the device.
    Checks the logits against the fp64 oracle and the ids bit-exact against
    the oracle's top-k on the kernel's own logits."""
    T = x_d.shape[0]
    w = torch.empty(T, m["K"], dtype=torch.float32, device=x_d.device)
    ids = torch.empty(T, m["K"], dtype=torch.int32, device=x_d.device)
    lg = torch.empty(T, m["E"], dtype=torch.float32, device=x_d.device)
    _capi.router_topk(x_d, m["gate_d"], m["bias_d"], m["K"], True, True, 0, w, ids, logits_out=lg)
    torch.cuda.synchronize()
    lg_h = lg.cpu().numpy()
    ref = oracle.router_logits(x_d.cpu(), m["gate"], m["bias"], round_mode=1)
    pre = ref - m["bias"].numpy()[None, :]
    # fp32 sums that straddle a bf16 rounding boundary may land one unit apart
    ulp = np.abs(pre) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(lg_h - ref) <= 1.01 * ulp + 1e-6)
    assert np.mean(lg_h == ref) > 0.99
    ow, oids = oracle.topk(lg_h, m["K"], True)
    assert np.array_equal(ids.cpu().numpy(), oids)
    assert np.max(np.abs(w.cpu().numpy() - ow)) <= 1e-6
    return w, ids, lg


def _ids_from_counts(counts, experts, seed):
    """[T,1] ids: counts[i] tokens on experts[i], in shuffled token order."""
    ids = np.concatenate([np.full(c, e, dtype=np.int64) for c, e in zip(counts, experts)])
    np.random.default_rng(seed).shuffle(ids)
    return ids[:, None]


def _sample_tokens(ids, n_random, seed, tile_rows=256):
    """The tokens whose rows sit at the first, middle and last position of
    every token tile of the tile map (``tile_rows``-row map: an expert of n
    rows has ceil(n / tile_rows) tiles ``tile_height`` rows apart, the last
    one ending at its n-th row), plus ``n_random`` random tokens. Rows map to
    tokens through the stable grouping (expert ascending, token ascending)."""
    T = ids.shape[0]
    E = int(ids.max()) + 1
    offsets, _, src = oracle.permute(ids, E)
    pick, n_tiles = set(), 0
    for e in range(E):
        n = int(offsets[e + 1] - offsets[e])
        if n == 0:
            continue
        h = tile_height(n, tile_rows)
        for j in range(-(-n // tile_rows)):
            lo, hi = j * h, min((j + 1) * h, n) - 1
            assert lo <= hi, (e, n, j, h)
            n_tiles += 1
            for r in (lo, (lo + hi) // 2, hi):
                pick.add(int(src[offsets[e] + r]))
    pick.update(int(t) for t in np.random.default_rng(seed).choice(T, n_random, replace=False))
    print(f"  {n_tiles} token tiles of {tile_rows} rows: {len(pick)} tokens checked", flush=True)
    return sorted(pick)


def _check_sampled(out, x, w1, w2, w, ids, tokens, act=0, path=-1):
    """Sampled tokens against the fp64 oracle (<= 2e-2) and against the oracle
    that rounds the intermediate, and y where the plan's kernels do (each
    element within its output rounding plus the oracle's fp32 bound); plus
    which rounding of y the output follows."""
    dt = w1[0].dtype
    plan = _capi.make_plan(x.shape[0], x.shape[1], w1[0].shape[0] // 2, len(w1), ids.shape[1],
                           _capi.dtype_code(dt), path)
    yr = y_round_of(plan, dt)
    got = out.float().cpu().numpy().astype(np.float64)[tokens]
    exact = oracle.fused_experts(x, w1, w2, w, ids, activation=act, tokens=tokens)[tokens]
    rounded, allow = oracle.fused_experts_bound(x, w1, w2, w, ids, act, ROUND[dt], y_round=yr,
                                                tokens=tokens)
    rounded, allow = rounded[tokens], allow[tokens]
    other = oracle.fused_experts(x, w1, w2, w, ids, activation=act, inter_round=ROUND[dt],
                                 y_round=0 if yr else ROUND[dt], tokens=tokens)[tokens]
    e1 = oracle.max_rel(got, exact)
    e2 = oracle.max_rel(got, rounded)
    print(f"  {len(tokens)} tokens, path {plan.path} splits {plan.down_splits}: max_rel vs fp64 "
          f"{e1:.2e}, vs the oracle rounding inter{' and y' if yr else ''} {e2:.2e}", flush=True)
    assert e1 <= 2e-2
    assert_matches_rounded(got, rounded, allow, dt)
    assert_y_rounding(got, rounded, other, dt)


SPLIT_CASES = [
    # name, H, I, E, counts, experts, dtype, act, expected S of gate_up and of down
    ("no_full_round_s8", 4096, 256, 64, [256, 256, 256, 256], [3, 17, 40, 63], "bf16", 0, (8, 1)),
    ("ragged_s8", 4096, 256, 64, [300, 200, 256, 268], [5, 17, 40, 63], "bf16", 0, (8, 1)),
    ("full_round_then_tail", 1024, 2048, 8, [512] * 7 + [520], list(range(8)), "bf16", 0, (4, 1)),
    ("f16_gelu", 4096, 256, 64, [256, 256, 256, 256], [0, 1, 2, 3], "f16", 1, (8, 1)),
    # 17 token tiles x 16 weight tiles: 272 down items, a 16-item last round cut 4 ways
    ("down_tail_s4", 4096, 2048, 8, [512] * 7 + [700], list(range(8)), "bf16", 0, (8, 4)),
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: c[0])
def test_tail_split_matches_oracle(case, dev):
    name, H, I, E, counts, experts, dts, act, want_s = case
    dt = torch.bfloat16 if dts == "bf16" else torch.float16
    ids = _ids_from_counts(counts, experts, seed=H + I)
    T = ids.shape[0]
    # forced: the automatic choice sees 16 rows per expert on average
    plan = _capi.make_plan(T, H, I, E, 1, _capi.dtype_code(dt), path=_capi.PATH_MFMA_TILED)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    S = (tiled_gate_up_split(plan, counts, cus), tiled_down_split(plan, counts, cus))
    banner(f"tail split {name} T={T} H={H} I={I} E={E} path={plan.path} S={S} cus={cus}")
    assert plan.path == _capi.PATH_MFMA_TILED
    if cus == 256:
        assert S == want_s
    w1, w2 = _bank(E, H, I, dt, seed=T, dev=dev, used=set(experts))
    x = (torch.randn(T, H, generator=torch.Generator().manual_seed(2)) * 0.5).to(dt)
    w = np.random.default_rng(4).random((T, 1)).astype(np.float32)
    out = gpu_fused(x, w1, w2, w, ids, act=act, path=_capi.PATH_MFMA_TILED)
    _check_sampled(out, x, w1, w2, w, ids, _sample_tokens(ids, 24, seed=T), act=act,
                   path=_capi.PATH_MFMA_TILED)


def test_tail_split_is_deterministic(dev):
    """The partial tiles are summed in a fixed order: two runs agree bit for bit."""
    ids = _ids_from_counts([300, 200, 256, 268], [5, 17, 40, 63], seed=1)
    T, H, I, E = ids.shape[0], 4096, 256, 64
    w1, w2 = _bank(E, H, I, torch.bfloat16, seed=9, dev=dev, used={5, 17, 40, 63})
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    w = np.ones((T, 1), dtype=np.float32)
    a = gpu_fused(x, w1, w2, w, ids, path=_capi.PATH_MFMA_TILED)
    b = gpu_fused(x, w1, w2, w, ids, path=_capi.PATH_MFMA_TILED)
    assert torch.equal(a, b)


def test_mixtral_prefill_t4096_sampled_tokens(mixtral, dev):
    """Mixtral-8x7B layer, T=4096, random top-2 routing: sampled tokens of the
    full-size grouped GEMM against the oracle."""
    m = mixtral
    T, H, I, E, K = 4096, m["H"], m["I"], m["E"], m["K"]
    rng = np.random.default_rng(11)
    ids = np.argsort(rng.random((T, E)), axis=1)[:, :K].astype(np.int64)
    counts = np.bincount(ids.ravel(), minlength=E)
    plan = _capi.make_plan(T, H, I, E, K, _capi.BF16)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    S = tiled_gate_up_split(plan, counts, cus)
    Sd = tiled_down_split(plan, counts, cus)
    banner(f"mixtral T={T} path={plan.path} down_splits={plan.down_splits} gate_up tail S={S} "
           f"down tail S={Sd}")
    assert plan.path == _capi.PATH_MFMA_TILED
    if cus == 256:
        # 35 token tiles: 3920 gate_up items (80 in the last round) cut in two
        # along K; one down split, 560 items (48 in the last round) cut in four
        assert (S, Sd) == (2, 4) and plan.down_splits == 1
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    w = rng.random((T, K)).astype(np.float32)
    out = gpu_fused(x, m["w1"], m["w2"], w, ids)
    _check_sampled(out, x, m["w1"], m["w2"], w, ids, _sample_tokens(ids, 6, seed=5))


def test_mixtral_t4096_end_to_end_biased_router(mixtral, dev):
    """The throughput workload as the bench runs it: 4096 tokens N(0,1), the
    router kernel (its MFMA form at this size) on the biased bf16 logits, then
    one fused_experts call on the router's own outputs. Ids bit-exact on the
    kernel's logits; sampled tokens of the output against the oracle."""
    m = mixtral
    T = 4096
    banner(f"mixtral end to end T={T} (router with bias -> fused_experts)")
    x = synth.make_tokens(T, m["H"], torch.bfloat16, seed=7)
    x_d = x.to(dev)
    w, ids, _ = _route_biased(m, x_d)
    counts = np.bincount(ids.cpu().numpy().ravel(), minlength=m["E"])
    print(f"  routed counts {counts.tolist()}", flush=True)
    out = torch.empty(T, m["H"], dtype=torch.bfloat16, device=dev)
    plan = _capi.make_plan(T, m["H"], m["I"], m["E"], m["K"], _capi.BF16)
    assert plan.path == _capi.PATH_MFMA_TILED and plan.down_splits == 1
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=dev)
    _capi.fused_experts(x_d, [t.data_ptr() for t in m["w1d"]], [t.data_ptr() for t in m["w2d"]],
                        m["I"], w, ids, 0, out, ws)
    torch.cuda.synchronize()
    ids_h = ids.cpu().numpy().astype(np.int64)
    _check_sampled(out.cpu(), x, m["w1"], m["w2"], w.cpu().numpy(), ids_h,
                   _sample_tokens(ids_h, 6, seed=8))


@pytest.mark.parametrize("T,splits", [(1, 8), (16, 4)])
def test_mixtral_decode_full_size(T, splits, mixtral, dev):
    """Mixtral-8x7B decode at 1 and 16 tokens through moe355_fused_experts,
    routed by the router kernel on the biased logits: the weight-streaming
    path with its K-split down projection (8 splits at one token, 4 at 16);
    at both sizes (2 and 32 slots) the gate_up workgroups group the slots
    themselves. Grouping bit-exact, every token's output against the oracle
    (y stays fp32 on this path)."""
    m = mixtral
    H, I, E, K = m["H"], m["I"], m["E"], m["K"]
    plan = _capi.make_plan(T, H, I, E, K, _capi.BF16)
    self_grouping = plan.rows <= 64
    banner(f"mixtral decode T={T} path={plan.path} down_splits={plan.down_splits} "
           f"grouping in gate_up={self_grouping}")
    assert plan.path == _capi.PATH_MFMA_SKINNY and plan.down_splits == splits
    assert self_grouping
    x = synth.make_tokens(T, H, torch.bfloat16, seed=T)
    x_d = x.to(dev)
    w, ids, _ = _route_biased(m, x_d)
    ws = torch.full((plan.workspace_bytes,), 0x5A, dtype=torch.uint8, device=dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    _capi.fused_experts(x_d, [t.data_ptr() for t in m["w1d"]], [t.data_ptr() for t in m["w2d"]],
                        I, w, ids, 0, out, ws)
    torch.cuda.synchronize()
    ids_h = ids.cpu().numpy().astype(np.int64)
    offsets, s2r, src = oracle.permute(ids_h, E)
    assert np.array_equal(read_ws(plan, ws, plan.off_offsets, E + 1), offsets)
    assert np.array_equal(read_ws(plan, ws, plan.off_slot_to_row, T * K), s2r)
    assert np.array_equal(read_ws(plan, ws, plan.off_row_src, T * K), src)
    _check_sampled(out.cpu(), x, m["w1"], m["w2"], w.cpu().numpy(), ids_h, list(range(T)))


def test_mixtral_t256_sampled_tokens(mixtral, dev):
    """Mixtral-8x7B layer, T=256 (~64 rows per expert): the automatic plan
    takes the 256-row kernel on 128-row token tiles with a 2-way K-split down
    projection, and the 112 x 8 gate_up items leave a 128-item last round
    that is cut along K."""
    m = mixtral
    T, H, I, E, K = 256, m["H"], m["I"], m["E"], m["K"]
    rng = np.random.default_rng(17)
    ids = np.argsort(rng.random((T, E)), axis=1)[:, :K].astype(np.int64)
    counts = np.bincount(ids.ravel(), minlength=E)
    plan = _capi.make_plan(T, H, I, E, K, _capi.BF16)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    S = tiled_gate_up_split(plan, counts, cus)
    banner(f"mixtral T={T} path={plan.path} down_splits={plan.down_splits} gate_up tail S={S}")
    assert plan.path == _capi.PATH_MFMA_TILED128
    if cus == 256:
        assert S == 2 and plan.down_splits == 2
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    w = rng.random((T, K)).astype(np.float32)
    out = gpu_fused(x, m["w1"], m["w2"], w, ids)
    _check_sampled(out, x, m["w1"], m["w2"], w, ids,
                   _sample_tokens(ids, 8, seed=6, tile_rows=plan.tile_rows))


def test_phi35_t2048_sampled_tokens(dev):
    """Phi-3.5-MoE-shape layer (H=4096, I=6400, E=16, K=2) at 2048 tokens with
    Zipf-skewed routing: the ragged groups of the bench's Phi config (some
    experts a fraction of a 256-row tile, others several tiles)."""
    T, H, I, E, K = 2048, 4096, 6400, 16, 2
    rng = np.random.default_rng(21)
    pop = 1.0 / np.arange(1, E + 1) ** 1.1
    scores = np.log(pop)[None, :] + rng.gumbel(size=(T, E))
    ids = np.argsort(-scores, axis=1)[:, :K].astype(np.int64)
    counts = np.bincount(ids.ravel(), minlength=E)
    plan = _capi.make_plan(T, H, I, E, K, _capi.BF16)
    banner(f"phi-3.5 T={T} path={plan.path} counts={counts.tolist()}")
    assert plan.path == _capi.PATH_MFMA_TILED
    w1, w2 = _bank(E, H, I, torch.bfloat16, seed=23, dev=dev, scale=0.02)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    w = rng.random((T, K)).astype(np.float32)
    out = gpu_fused(x, w1, w2, w, ids)
    _check_sampled(out, x, w1, w2, w, ids, _sample_tokens(ids, 8, seed=7))


def test_finegrained_t4096_with_shared_columns_sampled_tokens(dev):
    """Fine-grained layer (H=2048, I=1408, 64 routed experts top-6 plus 2
    shared experts folded in as two always-routed columns) at 4096 tokens."""
    T, H, I, E, K = 4096, 2048, 1408, 66, 8
    rng = np.random.default_rng(31)
    routed = np.argsort(rng.random((T, 64)), axis=1)[:, :6]
    ids = np.concatenate([routed, np.full((T, 1), 64), np.full((T, 1), 65)], axis=1).astype(np.int64)
    plan = _capi.make_plan(T, H, I, E, K, _capi.BF16)
    banner(f"fine-grained T={T} path={plan.path} down_splits={plan.down_splits}")
    assert plan.path == _capi.PATH_MFMA_TILED
    w1, w2 = _bank(E, H, I, torch.bfloat16, seed=33, dev=dev, scale=0.02)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    w = np.concatenate([rng.random((T, 6)), np.ones((T, 2))], axis=1).astype(np.float32)
    out = gpu_fused(x, w1, w2, w, ids)
    _check_sampled(out, x, w1, w2, w, ids, _sample_tokens(ids, 8, seed=9))


def test_finegrained_t8_layer_forward(dev):
    """Fine-grained layer (H=2048, I=1408, 64 routed experts top-6
    renormalised, plus 2 always-on shared experts of 1408) at decode batch 8,
    through FusedMoE.forward as a model calls it: the router kernel, then one
    fused_experts call with the shared experts folded in as two extra experts
    of weight 1 (64 slots over up to 38 experts: the weight-streaming path
    after a permute launch). Ids bit-exact on the router's own logits; every
    token against the oracle (routed sum plus the dense shared SwiGLU)."""
    from reframework_amd.moe import FusedMoE

    T, H, I, E, K, ns = 8, 2048, 1408, 64, 6, 2
    plan = _capi.make_plan(T, H, I, E + ns, K + ns, _capi.BF16)
    banner(f"fine-grained layer T={T} path={plan.path} down_splits={plan.down_splits}")
    assert plan.path == _capi.PATH_MFMA_SKINNY
    w1, w2 = _bank(E, H, I, torch.bfloat16, seed=41, dev=dev, scale=0.02)
    sh1, sh2 = _bank(1, H, ns * I, torch.bfloat16, seed=42, dev=dev, scale=0.02)
    gate = (torch.randn(E, H, generator=torch.Generator().manual_seed(43)) * 0.02).to(
        torch.bfloat16)
    sd = {"gate.weight": gate,
          "shared_experts.gate_proj.weight": sh1[0][:ns * I],
          "shared_experts.up_proj.weight": sh1[0][ns * I:],
          "shared_experts.down_proj.weight": sh2[0]}
    for e in range(E):
        sd[f"experts.{e}.gate_proj.weight"] = w1[e][:I]
        sd[f"experts.{e}.up_proj.weight"] = w1[e][I:]
        sd[f"experts.{e}.down_proj.weight"] = w2[e]
    moe = FusedMoE(E, K, H, I, dtype=torch.bfloat16, n_shared_experts=ns)
    moe.load_state_dict(sd)
    assert moe._shared_folded
    moe = moe.to(dev)
    x = synth.make_tokens(T, H, torch.bfloat16, seed=9)
    x_d = x.to(dev)
    out = moe(x_d)
    rw, rids = moe.route(x_d)
    lw = torch.empty(T, K, dtype=torch.float32, device=dev)
    lids = torch.empty(T, K, dtype=torch.int32, device=dev)
    lg = torch.empty(T, E, dtype=torch.float32, device=dev)
    _capi.router_topk(x_d, gate.to(dev), None, K, True, True, 0, lw, lids, logits_out=lg)
    torch.cuda.synchronize()
    assert torch.equal(rids.cpu(), lids.long().cpu()) and torch.equal(rw.cpu(), lw.cpu())
    ow, oids = oracle.topk(lg.cpu().numpy(), K, True)
    assert np.array_equal(rids.cpu().numpy(), oids)
    wn, idn = rw.cpu().numpy(), rids.cpu().numpy()
    print(f"  {len(np.unique(idn))} routed experts", flush=True)
    ones, zeros = np.ones((T, 1), np.float32), np.zeros((T, 1), np.int64)
    got = out.float().cpu().numpy().astype(np.float64)

    def ref(inter_round, y_round):
        return (oracle.fused_experts(x, w1, w2, wn, idn, inter_round=inter_round, y_round=y_round)
                + oracle.fused_experts(x, sh1, sh2, ones, zeros, inter_round=inter_round,
                                       y_round=y_round))

    exact, other = ref(0, 0), ref(ROUND[torch.bfloat16], 1)
    r1, a1 = oracle.fused_experts_bound(x, w1, w2, wn, idn, 0, ROUND[torch.bfloat16])
    r2, a2 = oracle.fused_experts_bound(x, sh1, sh2, ones, zeros, 0, ROUND[torch.bfloat16])
    rounded, allow = r1 + r2, a1 + a2
    e1, e2 = oracle.max_rel(got, exact), oracle.max_rel(got, rounded)
    print(f"  max_rel vs fp64 {e1:.2e}, vs the oracle rounding inter {e2:.2e}", flush=True)
    assert e1 <= 2e-2
    assert_matches_rounded(got, rounded, allow, torch.bfloat16)
    assert_y_rounding(got, rounded, other, torch.bfloat16)
    # the shared experts are really in: the routed sum alone is far off
    assert oracle.max_rel(got, oracle.fused_experts(x, w1, w2, wn, idn)) > 0.1
