"""The oracle's per-element fp32 bound (oracle.fused_experts_bound), which the
GPU parity tests use as their tight bar: every output element within its own
rounding plus ``allow``.

Pinned on the CPU with an independent fp32 evaluation of the same
computation (torch float32 matmuls, the intermediate and, where the path does,
y rounded to the layer dtype; the kernels' arithmetic, with another summation
order): every element of it must fall inside the bound on random data of
several shapes, dtypes and K-splits; plausible mistakes planted into that
evaluation (a dropped slot, gate and up swapped, another expert's w2, w2 rows
shifted by one) must fall outside; and the bound must stay tight (its mean
below half the flat 1e-3 of the largest output it replaces), with ``out`` equal to
oracle.fused_experts bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import ROUND, make_bank, skewed_ids
from oracle import oracle

OUT_ROUND = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}


def fp32_eval(x, w1, w2, w, ids, dt, splits, y_round, plant=None):
    T, H = x.shape
    I = w1[0].shape[0] // 2
    E = len(w1)
    out = torch.zeros(T, H, dtype=torch.float32)
    xf = x.float()
    for e in range(E):
        rows = [(t, k) for t in range(T) for k in range(ids.shape[1]) if ids[t, k] == e]
        if not rows:
            continue
        tok = torch.tensor([r[0] for r in rows])
        gu = xf[tok] @ w1[e].float().T
        g, u = gu[:, :I], gu[:, I:]
        if plant == "swap_gate_up":
            g, u = u, g
        inter = (torch.nn.functional.silu(g) * u).to(dt).float()
        w2e = w2[(e + 1) % E if plant == "other_expert_w2" else e].float()
        if plant == "w2_rows_shifted":
            w2e = torch.roll(w2e, 1, dims=0)
        c = I // splits
        y = sum(inter[:, s * c:(s + 1) * c] @ w2e[:, s * c:(s + 1) * c].T for s in range(splits))
        if y_round:
            y = y.to(dt).float()
        for j, (t, k) in enumerate(rows):
            if plant == "drop_slot" and t == 1 and k == 0:
                continue
            out[t] += float(w[t, k]) * y[j]
    return out.to(dt).float().numpy().astype(np.float64)


def excess(got, ref, allow, dt):
    scale = float(np.max(np.abs(ref)))
    return float(np.max(np.abs(got - ref) - OUT_ROUND[dt] * np.abs(ref) - allow)) / scale


CASES = [
    # E, H, I, T, K, splits, y rounded, dtype
    (4, 256, 256, 130, 1, 4, False, torch.bfloat16),
    (8, 512, 384, 200, 2, 1, True, torch.bfloat16),
    (8, 512, 384, 200, 2, 2, False, torch.bfloat16),
    (8, 256, 256, 150, 2, 1, True, torch.float16),
    (16, 1024, 512, 40, 6, 1, True, torch.bfloat16),
]


def _data(E, H, I, T, K, dt, seed):
    w1, w2 = make_bank(E, H, I, dt, seed=H + I + E)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(seed)).to(dt)
    ids = skewed_ids(T, K, E, seed=seed, skew=1.0) if K > 1 else np.zeros((T, 1), np.int64)
    if K == 1:
        ids[-1, 0] = E - 1
    w = np.random.default_rng(seed).random((T, K)).astype(np.float32)
    return w1, w2, x, ids, w


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"E{c[0]}H{c[1]}I{c[2]}T{c[3]}K{c[4]}s{c[5]}y{int(c[6])}")
def test_fp32_evaluation_lies_inside_the_bound(case):
    E, H, I, T, K, splits, yr, dt = case
    for seed in range(4):
        w1, w2, x, ids, w = _data(E, H, I, T, K, dt, seed)
        ref, allow = oracle.fused_experts_bound(x, w1, w2, w, ids, 0, ROUND[dt],
                                                ROUND[dt] if yr else 0)
        assert np.array_equal(ref, oracle.fused_experts(x, w1, w2, w, ids, inter_round=ROUND[dt],
                                                        y_round=ROUND[dt] if yr else 0))
        assert (allow >= 0).all()
        assert excess(fp32_eval(x, w1, w2, w, ids, dt, splits, yr), ref, allow, dt) <= 1e-5
        # tight: on average well below the flat 1e-3 of max|ref| it replaces
        assert np.mean(allow) / np.max(np.abs(ref)) < 5e-4


@pytest.mark.parametrize("plant", ["drop_slot", "swap_gate_up", "other_expert_w2",
                                   "w2_rows_shifted"])
@pytest.mark.parametrize("case", CASES[:2] + CASES[3:4], ids=lambda c: f"E{c[0]}T{c[3]}")
def test_planted_mistakes_fall_outside_the_bound(case, plant):
    E, H, I, T, K, splits, yr, dt = case
    w1, w2, x, ids, w = _data(E, H, I, T, K, dt, 7)
    ref, allow = oracle.fused_experts_bound(x, w1, w2, w, ids, 0, ROUND[dt],
                                            ROUND[dt] if yr else 0)
    assert excess(fp32_eval(x, w1, w2, w, ids, dt, splits, yr, plant), ref, allow, dt) > 1e-2


def test_bound_flags_intermediates_on_a_rounding_boundary():
    """An intermediate exactly on a bf16 rounding boundary gets the other
    rounding allowed: x = 1, gate weight 30, up weight 30.0625 / silu(30), so
    v = silu(30) * u = 30.0625, the midpoint of the bf16 neighbours 30 and
    30.125; w2 = 1 (fp32 weights, so nothing else rounds). The allowance is
    one bf16 spacing at 30 (2^-3) plus the y accumulation term."""
    H, I = 1, 1
    x = torch.tensor([[1.0]])
    # bf16 values near 30 are spaced 2^-3; 30.0625 is the midpoint of 30 and 30.125
    g, u = 30.0, 30.0625 / (30.0 / (1.0 + np.exp(-30.0)))
    w1 = [torch.tensor([[g], [u]], dtype=torch.float32)]
    w2 = [torch.tensor([[1.0]], dtype=torch.float32)]
    ref, allow = oracle.fused_experts_bound(x, w1, w2, np.ones((1, 1), np.float32),
                                            np.zeros((1, 1), np.int64), 0, ROUND[torch.bfloat16])
    assert ref[0, 0] in (30.0, 30.125)
    assert 2.0 ** -3 <= allow[0, 0] < 2.0 ** -3 + 1e-4
    # a value far from any boundary gets only the accumulation term
    w1b = [torch.tensor([[g], [30.03 / (30.0 / (1.0 + np.exp(-30.0)))]], dtype=torch.float32)]
    _, allow_b = oracle.fused_experts_bound(x, w1b, w2, np.ones((1, 1), np.float32),
                                            np.zeros((1, 1), np.int64), 0, ROUND[torch.bfloat16])
    assert allow_b[0, 0] < 1e-4
