"""Seeded random fused_experts configurations for the random-shape tests (not
collected: no test_ prefix). Every configuration is one the library plans
(make_plan accepts it); the CPU test replays the kernels' index math on each,
the GPU test checks each against the oracle."""

from __future__ import annotations

from typing import Dict, List

import numpy as np

from reframework_amd import _capi

DTYPES = {"bf16": _capi.BF16, "f16": _capi.F16, "f32": _capi.F32}


def configs(seed: int, n: int, large: bool = False) -> List[Dict]:
    """n configurations: experts 2-256, top-1..8, ragged and skewed routing
    (Zipf exponent 0-2), some slots dropped through an expert map, int32 or
    int64 ids, all three activations and dtypes. ``large`` draws 1025-6000
    tokens (the output is then checked on a sample of tokens)."""
    rng = np.random.default_rng(seed)
    out: List[Dict] = []
    while len(out) < n:
        E = int(rng.choice([2, 3, 4, 5, 8, 12, 16, 32, 60, 64, 66, 100, 128, 200, 256]))
        K = int(rng.integers(1, min(E, 8) + 1))
        T = int(rng.choice([1025, 1500, 2500, 4096, 6000] if large else
                           [1, 2, 3, 5, 8, 13, 16, 31, 64, 100, 200, 333, 700, 1025, 1500, 2500]))
        H = int(rng.choice([256, 512, 768, 1024, 2048]))
        I = int(rng.choice([128, 256, 384, 512, 640, 1024, 1408]))
        dt = str(rng.choice(["bf16", "f16", "f32"], p=[0.6, 0.3, 0.1]))
        work = T * K * H * I
        if work > (2e10 if large else 6e8) or (dt == "f32" and work > 1.5e8):
            continue
        if E * 3 * H * I * 2 > 1.2e9:  # weights per configuration
            continue
        try:
            plan = _capi.make_plan(T, H, I, E, K, DTYPES[dt])
        except _capi.MoeLibError:
            continue
        emap = [(-1 if rng.random() < 0.25 else x) for x in range(E)] if rng.random() < 0.2 else None
        out.append(dict(T=T, K=K, E=E, H=H, I=I, dt=dt, skew=float(rng.choice([0.0, 0.8, 1.2, 2.0])),
                        seed=int(rng.integers(1 << 30)), emap=emap,
                        act=int(rng.choice([0, 0, 0, 1, 2])), ids64=bool(rng.random() < 0.3),
                        path=plan.path, sample=large))
    return out


SMALL = configs(123, 80) + configs(2024, 120)
LARGE = configs(7, 16, large=True) + configs(99, 24, large=True)
ALL = SMALL + LARGE


def name(c: Dict) -> str:
    return (f"T{c['T']}_K{c['K']}_E{c['E']}_H{c['H']}_I{c['I']}_{c['dt']}_p{c['path']}"
            f"{'_map' if c['emap'] else ''}")
