"""Pins the oracle's expert FFN and grouping against closed forms (CPU).

The oracle restates fused_experts (reframework/moe/fused.py:49-87) in fp64.
It is checked against things it does not share code with:
  * E = K = 1 reduces to one dense gated MLP, computed here with
    torch.nn.functional (linear, silu, gelu) in float64;
  * hand-evaluated numbers on a 2-dimensional layer;
  * linearity in the routing weights, invariance under renaming experts,
    and token-subset consistency;
  * the grouping equals numpy's stable argsort.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle, ref_torch


def _layer(E, H, I, dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    w1 = [(torch.randn(2 * I, H, generator=g) * 0.1).to(dtype) for _ in range(E)]
    w2 = [(torch.randn(H, I, generator=g) * 0.1).to(dtype) for _ in range(E)]
    return w1, w2


@pytest.mark.parametrize("act,fn", [
    (0, lambda g: F.silu(g)),
    (1, lambda g: F.gelu(g)),
    (2, lambda g: F.gelu(g, approximate="tanh")),
])
def test_single_expert_is_dense_gated_mlp(act, fn):
    H, I, T = 48, 40, 9
    w1, w2 = _layer(1, H, I)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(3))
    ids = np.zeros((T, 1), np.int64)
    w = np.ones((T, 1), np.float32)
    out = oracle.fused_experts(x, w1, w2, w, ids, activation=act)
    xd, a, b = x.double(), w1[0].double(), w2[0].double()
    ref = F.linear(fn(F.linear(xd, a[:I])) * F.linear(xd, a[I:]), b)
    assert np.allclose(out, ref.numpy(), rtol=1e-12, atol=1e-12)


def test_hand_evaluated_two_dim_layer():
    # H=2, I=1: gate row [1,0], up row [0,1], down column [1,3]; x = [1,2].
    w1 = [torch.tensor([[1.0, 0.0], [0.0, 1.0]])]
    w2 = [torch.tensor([[1.0], [3.0]])]
    x = torch.tensor([[1.0, 2.0]])
    out = oracle.fused_experts(x, w1, w2, np.array([[0.5]], np.float32), np.zeros((1, 1), np.int64))
    inter = (1.0 / (1.0 + math.exp(-1.0))) * 2.0  # silu(1) * 2
    assert out[0].tolist() == pytest.approx([0.5 * inter, 1.5 * inter], rel=1e-15)


def test_linear_in_routing_weights_and_additive_over_slots():
    E, H, I, T, K = 4, 32, 24, 6, 2
    w1, w2 = _layer(E, H, I)
    x = torch.randn(T, H)
    rng = np.random.default_rng(0)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int64)
    w = rng.random((T, K)).astype(np.float32)
    full = oracle.fused_experts(x, w1, w2, w, ids)
    half = oracle.fused_experts(x, w1, w2, (w * 0.5).astype(np.float32), ids)
    assert np.allclose(half, 0.5 * full, rtol=1e-13, atol=1e-13)
    parts = sum(oracle.fused_experts(x, w1, w2, w[:, k:k + 1], ids[:, k:k + 1]) for k in range(K))
    assert np.allclose(parts, full, rtol=1e-12, atol=1e-12)


def test_renaming_experts_does_not_change_output():
    E, H, I, T, K = 6, 16, 8, 10, 2
    w1, w2 = _layer(E, H, I)
    x = torch.randn(T, H)
    rng = np.random.default_rng(1)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int64)
    w = rng.random((T, K)).astype(np.float32)
    perm = rng.permutation(E)  # new bank row j holds old expert perm[j]
    inv = np.argsort(perm)
    out_a = oracle.fused_experts(x, w1, w2, w, ids)
    out_b = oracle.fused_experts(x, [w1[p] for p in perm], [w2[p] for p in perm], w, inv[ids])
    assert np.array_equal(out_a, out_b)


def test_token_subset_matches_full_rows_and_dropped_slots():
    E, H, I, T, K = 4, 16, 8, 12, 2
    w1, w2 = _layer(E, H, I)
    x = torch.randn(T, H)
    rng = np.random.default_rng(2)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int64)
    w = rng.random((T, K)).astype(np.float32)
    full = oracle.fused_experts(x, w1, w2, w, ids)
    sub = oracle.fused_experts(x, w1, w2, w, ids, tokens=[3, 7, 11])
    assert np.array_equal(sub[[3, 7, 11]], full[[3, 7, 11]])
    assert not sub[[0, 1, 2]].any()
    ids2 = ids.copy()
    ids2[:, 1] = -1  # dropped slot contributes nothing
    only0 = oracle.fused_experts(x, w1, w2, w[:, :1], ids[:, :1])
    assert np.allclose(oracle.fused_experts(x, w1, w2, w, ids2), only0, rtol=0, atol=0)


def test_bf16_inputs_are_widened_exactly():
    E, H, I, T = 2, 32, 16, 5
    w1, w2 = _layer(E, H, I, dtype=torch.bfloat16)
    x = torch.randn(T, H).to(torch.bfloat16)
    ids = np.array([[0, 1]] * T, np.int64)
    w = np.full((T, 2), 0.5, np.float32)
    a = oracle.fused_experts(x, w1, w2, w, ids)
    b = oracle.fused_experts(x.float(), [t.float() for t in w1], [t.float() for t in w2], w, ids)
    assert np.array_equal(a, b)


def test_inter_rounding_modes_bound_the_difference():
    E, H, I, T = 3, 64, 48, 8
    w1, w2 = _layer(E, H, I)
    x = torch.randn(T, H)
    ids = np.array([[0, 2]] * T, np.int64)
    w = np.full((T, 2), 0.5, np.float32)
    exact = oracle.fused_experts(x, w1, w2, w, ids)
    rb = oracle.fused_experts(x, w1, w2, w, ids, inter_round=oracle.ROUND_BF16)
    rh = oracle.fused_experts(x, w1, w2, w, ids, inter_round=oracle.ROUND_F16)
    assert 0 < oracle.max_rel(rb, exact) < 2 ** -7
    assert 0 < oracle.max_rel(rh, exact) < 2 ** -10


def test_y_rounding_applies_per_slot_before_the_weight():
    """y_round rounds each slot's down-projection output, then weights it: with
    one slot, out = w * round(y), where y is the unweighted, unrounded output."""
    E, H, I, T = 3, 64, 48, 8
    w1, w2 = _layer(E, H, I)
    x = torch.randn(T, H)
    ids = np.array([[1]] * T, np.int64)
    y = oracle.fused_experts(x, w1, w2, np.ones((T, 1), np.float32), ids)
    wt = np.float32(0.3)
    for mode in (oracle.ROUND_BF16, oracle.ROUND_F16):
        got = oracle.fused_experts(x, w1, w2, np.full((T, 1), wt, np.float32), ids, y_round=mode)
        assert np.array_equal(got, float(wt) * oracle.round_array(y, mode))
        # rounding after the weight (or not at all) would differ
        assert not np.array_equal(got, oracle.round_array(float(wt) * y, mode))
    # two slots: the sum of the two rounded, weighted slot outputs
    ids2 = np.array([[1, 2]] * T, np.int64)
    w2s = np.array([[0.25, 0.75]] * T, np.float32)
    got = oracle.fused_experts(x, w1, w2, w2s, ids2, y_round=oracle.ROUND_BF16)
    ya = oracle.fused_experts(x, w1, w2, np.ones((T, 1), np.float32), ids2[:, :1])
    yb = oracle.fused_experts(x, w1, w2, np.ones((T, 1), np.float32), ids2[:, 1:])
    want = 0.25 * oracle.round_array(ya, oracle.ROUND_BF16) + 0.75 * oracle.round_array(yb, oracle.ROUND_BF16)
    assert np.allclose(got, want, rtol=0, atol=1e-15)


def test_round_array_matches_torch_casts():
    v = np.random.default_rng(4).normal(size=1000) * 10
    v32 = v.astype(np.float32).astype(np.float64)
    assert np.array_equal(oracle.round_array(v32, oracle.ROUND_BF16),
                          torch.from_numpy(v32).float().to(torch.bfloat16).double().numpy())
    assert np.array_equal(oracle.round_array(v32, oracle.ROUND_F16),
                          torch.from_numpy(v32).float().to(torch.float16).double().numpy())


def test_router_logits_closed_form_and_rounding():
    T, H, E = 7, 40, 5
    x = torch.randn(T, H)
    gate = torch.randn(E, H)
    bias = torch.randn(E)
    lg = oracle.router_logits(x, gate, bias)
    ref = (F.linear(x.double(), gate.double()).float() + bias).numpy()
    assert np.array_equal(lg, ref)
    xb, gb = x.to(torch.bfloat16), gate.to(torch.bfloat16)
    lgb = oracle.router_logits(xb, gb, None, round_mode=oracle.ROUND_BF16)
    refb = F.linear(xb.double(), gb.double()).float().to(torch.bfloat16).float().numpy()
    assert np.array_equal(lgb, refb)


@pytest.mark.parametrize("drop", [False, True])
def test_permute_is_stable_argsort(drop):
    rng = np.random.default_rng(5)
    T, K, E = 300, 3, 10
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int64)
    emap = None
    local = ids.reshape(-1).copy()
    if drop:
        emap = [-1 if e in (2, 7) else e for e in range(E)]
        local = np.array([emap[i] for i in local])
    offsets, s2r, src = oracle.permute(ids, E, emap)
    valid = np.nonzero(local >= 0)[0]
    order = valid[np.argsort(local[valid], kind="stable")]
    assert np.array_equal(src[:len(order)], order // K)
    assert np.array_equal(s2r[order], np.arange(len(order)))
    assert np.all(s2r[local < 0] == -1)
    counts = np.bincount(local[valid], minlength=E)
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(counts)]))


def test_ref_torch_fp32_agrees_with_fp64_oracle():
    E, H, I, T, K = 4, 64, 48, 20, 2
    w1, w2 = _layer(E, H, I)
    gate = torch.randn(E, H) * 0.3
    x = torch.randn(T, H)
    out = ref_torch.forward(x, gate, w1, w2, K)
    w, ids = ref_torch.route(x, gate, K, True, torch.float32)
    ref = oracle.fused_experts(x, w1, w2, w.numpy(), ids.numpy())
    assert oracle.max_rel(out.numpy(), ref) < 1e-5
