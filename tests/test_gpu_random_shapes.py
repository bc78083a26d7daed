"""GPU parity of fused_experts over 96 seeded random configurations
(tests/_random_shapes.py): 2-256 experts, top-1..8, 1-6000 tokens, hidden
256-2048, ffn 128-1408, bf16 / f16 / fp32, silu / gelu / gelu_tanh, skewed
and uniform routing, dropped slots through an expert map, int32 and int64
ids, so every kernel family meets shapes no hand-picked case names. Each
configuration's index math is replayed on the CPU first
(tests/test_kernel_index_math.py). Bar: max-relative error against the fp64
oracle <= 2e-2 (bf16, f16) or 1e-5 (fp32), on every token (a sample of 48
tokens for the configurations above 1024 tokens).

Reference: fused_experts (reframework/moe/fused.py:49-87).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _random_shapes
from _helpers import DT, banner, gpu_fused, make_bank, skewed_ids
from oracle import oracle

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


@pytest.mark.parametrize("c", _random_shapes.ALL, ids=_random_shapes.name)
def test_random_shape_matches_oracle(c, dev):
    T, K, E, H, I = c["T"], c["K"], c["E"], c["H"], c["I"]
    dt = DT[c["dt"]]
    banner(f"random shape {_random_shapes.name(c)} act={c['act']} ids64={c['ids64']}")
    w1, w2 = make_bank(E, H, I, dt, seed=c["seed"] % 100000)
    x = (torch.randn(T, H, generator=torch.Generator().manual_seed(c["seed"] % 9973)) * 0.7).to(dt)
    ids = skewed_ids(T, K, E, c["seed"], c["skew"])
    w = np.random.default_rng(c["seed"]).random((T, K)).astype(np.float32)
    out = gpu_fused(x, w1, w2, w, ids, act=c["act"], expert_map=c["emap"], ids64=c["ids64"])
    assert out.dtype == dt and out.shape == (T, H)
    got = out.float().cpu().numpy().astype(np.float64)
    ids_local = np.asarray(c["emap"])[ids] if c["emap"] else ids
    tokens = None
    if c["sample"]:
        rng = np.random.default_rng(c["seed"])
        tokens = sorted(rng.choice(T, size=min(T, 48), replace=False).tolist())
    ref = oracle.fused_experts(x, w1, w2, w, ids_local, activation=c["act"], tokens=tokens)
    if tokens is not None:
        got, ref = got[tokens], ref[tokens]
    assert np.isfinite(got).all()
    err = oracle.max_rel(got, ref)
    print(f"  max_rel {err:.2e}", flush=True)
    assert err <= TOL[dt]
