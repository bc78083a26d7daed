"""GPU parity of the 256-token-tile grouped GEMM at full size and on the
shapes whose last round is split along K.

Reference: fused_experts (reframework/moe/fused.py:49-87). The tiled gate_up
and down run their items on one workgroup per CU; the items of a last,
partly filled round are cut along K over the idle CUs, their fp32 partial
tiles summed (and activated, for gate_up) by a fix-up kernel. These tests
build routings whose tile counts put that split on (checked with the host
replica of its rule), and compare
sampled tokens (the first and last token of every expert group, whose rows
sit in the first and last tiles, plus random ones) with the fp64 oracle:
  * <= 2e-2 max-relative against the fp64 oracle;
  * <= 4e-3 against the oracle that rounds the intermediate (and, for the
    tiled paths with one down K-split, y) like the kernels.
The full-size cases are the Mixtral-8x7B layer (H=4096, I=14336, E=8, K=2) at
T=4096 and 256, the Phi-3.5-MoE layer at T=2048 with Zipf-skewed routing, and
the fine-grained layer (64 experts top-6 plus 2 shared) at T=4096: the shapes
the throughput figures are quoted on.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import ROUND, banner, gpu_fused, tiled_down_split, tiled_gate_up_split
from oracle import oracle
from reframework_amd import _capi

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


def _ids_from_counts(counts, experts, seed):
    """[T,1] ids: counts[i] tokens on experts[i], in shuffled token order."""
    ids = np.concatenate([np.full(c, e, dtype=np.int64) for c, e in zip(counts, experts)])
    np.random.default_rng(seed).shuffle(ids)
    return ids[:, None]


def _sample_tokens(ids, n_random, seed):
    """First and last token of every expert's group plus random tokens."""
    T = ids.shape[0]
    pick = set()
    for e in np.unique(ids):
        t = np.nonzero((ids == e).any(axis=1))[0]
        pick.update((int(t[0]), int(t[-1])))
    pick.update(int(t) for t in np.random.default_rng(seed).choice(T, n_random, replace=False))
    return sorted(pick)


def _check_sampled(out, x, w1, w2, w, ids, tokens, act=0):
    dt = w1[0].dtype
    got = out.float().cpu().numpy().astype(np.float64)[tokens]
    exact = oracle.fused_experts(x, w1, w2, w, ids, activation=act, tokens=tokens)[tokens]
    rounded = oracle.fused_experts(x, w1, w2, w, ids, activation=act, inter_round=ROUND[dt],
                                   tokens=tokens)[tokens]
    # tiled paths with one down K-split also round y to the layer dtype
    rounded_y = oracle.fused_experts(x, w1, w2, w, ids, activation=act, inter_round=ROUND[dt],
                                     y_round=ROUND[dt], tokens=tokens)[tokens]
    e1 = oracle.max_rel(got, exact)
    e2 = min(oracle.max_rel(got, rounded), oracle.max_rel(got, rounded_y))
    print(f"  {len(tokens)} tokens: max_rel vs fp64 {e1:.2e}, vs rounded intermediate (and y) "
          f"{e2:.2e}", flush=True)
    assert e1 <= 2e-2
    assert e2 <= (4e-3 if dt == torch.bfloat16 else 2e-3)


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
    _check_sampled(out, x, w1, w2, w, ids, _sample_tokens(ids, 24, seed=T), act=act)


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


def test_mixtral_prefill_t4096_sampled_tokens(dev):
    """Mixtral-8x7B layer, T=4096, random top-2 routing: sampled tokens of the
    full-size grouped GEMM against the oracle."""
    T, H, I, E, K = 4096, 4096, 14336, 8, 2
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
    w1, w2 = _bank(E, H, I, torch.bfloat16, seed=13, dev=dev, scale=0.02)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    w = rng.random((T, K)).astype(np.float32)
    out = gpu_fused(x, w1, w2, w, ids)
    _check_sampled(out, x, w1, w2, w, ids, _sample_tokens(ids, 6, seed=5))


def test_mixtral_t256_sampled_tokens(dev):
    """Mixtral-8x7B layer, T=256 (~64 rows per expert): the automatic plan
    takes the 256-row kernel on 128-row token tiles with a 2-way K-split down
    projection, and the 112 x 8 gate_up items leave a 128-item last round
    that is cut along K."""
    T, H, I, E, K = 256, 4096, 14336, 8, 2
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
    w1, w2 = _bank(E, H, I, torch.bfloat16, seed=19, dev=dev, scale=0.02)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    w = rng.random((T, K)).astype(np.float32)
    out = gpu_fused(x, w1, w2, w, ids)
    _check_sampled(out, x, w1, w2, w, ids, _sample_tokens(ids, 8, seed=6))


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
