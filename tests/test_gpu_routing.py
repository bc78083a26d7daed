"""GPU parity of the router and top-k kernels against the oracle.

Bar: expert ids bit-exact on the same fp32 logits (ties to the lower id),
weights within 1e-6; router logits within fp32 accumulation error of the fp64
oracle (reference: reframework/moe/moe_layer.py:320-344,
reframework/moe/fused.py:32-46).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from _helpers import banner
from oracle import oracle
from reframework_amd import _capi
from reframework_amd.moe import torch_fused_topk

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "topk_golden.npz")


def _golden_cases():
    g = np.load(GOLDEN)
    names = sorted({k.split("__")[0] for k in g.files})
    return [(n, g[f"{n}__logits"], int(g[f"{n}__k"]), bool(g[f"{n}__renorm"])) for n in names]


@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: c[0])
def test_topk_from_logits_bit_exact(case, dev):
    name, logits, k, renorm = case
    banner(f"topk_from_logits {name} {logits.shape} k={k}")
    w, ids = torch_fused_topk(torch.from_numpy(logits).to(dev), k, renorm)
    ow, oids = oracle.topk(logits, k, renorm)
    assert ids.dtype == torch.int64 and w.dtype == torch.float32
    assert np.array_equal(ids.cpu().numpy(), oids)
    assert np.max(np.abs(w.cpu().numpy() - ow)) <= 1e-6


@pytest.mark.parametrize("E,K", [(8, 2), (16, 2), (64, 6), (256, 8), (5, 5), (3, 1)])
def test_topk_random_shapes(E, K, dev):
    banner(f"topk random E={E} K={K}")
    rng = np.random.default_rng(E + 7 * K)
    logits = (rng.normal(size=(333, E)) * 3).astype(np.float32)
    logits[::7, :] = np.round(logits[::7, :])  # plant exact ties on some rows
    for renorm in (True, False):
        w, ids = torch_fused_topk(torch.from_numpy(logits).to(dev), K, renorm)
        ow, oids = oracle.topk(logits, K, renorm)
        assert np.array_equal(ids.cpu().numpy(), oids)
        assert np.max(np.abs(w.cpu().numpy() - ow)) <= 1e-6


def _router(x, gate, bias, K, renorm, round_logits, kmin=0):
    T, E = x.shape[0], gate.shape[0]
    w = torch.empty((T, K), dtype=torch.float32, device=x.device)
    ids = torch.empty((T, K), dtype=torch.int32, device=x.device)
    lg = torch.empty((T, E), dtype=torch.float32, device=x.device)
    _capi.router_topk(x, gate, bias, K, renorm, round_logits, kmin, w, ids, logits_out=lg)
    torch.cuda.synchronize()
    return w.cpu().numpy(), ids.cpu().numpy(), lg.cpu().numpy()


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("T,H,E,K", [(1, 4096, 8, 2), (77, 4096, 8, 2), (64, 2048, 64, 6),
                                     (33, 1024, 16, 2), (5, 8192, 256, 8),
                                     # 4 and 8 tokens per workgroup, 8 or 16 experts per pass
                                     (300, 4096, 8, 2), (300, 2048, 64, 6), (1100, 1024, 8, 2),
                                     (1100, 512, 64, 6),
                                     # MFMA router: one 64-k batch per wave, a partial last
                                     # workgroup and 20 experts in two 16-row groups; an odd
                                     # batch count; 5 batches through a 4-buffer ring
                                     (1037, 1024 // 4, 20, 3), (1100, 768, 8, 2), (257, 1280, 40, 4)])
def test_router_topk(dtype, T, H, E, K, dev):
    banner(f"router dtype={dtype} T={T} H={H} E={E} K={K}")
    dt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    if dt == torch.float32 and H > 8192:
        pytest.skip("fp32 router holds H <= 8192")
    g = torch.Generator().manual_seed(T + H + E)
    x = torch.randn(T, H, generator=g).to(dt)
    gate = (torch.randn(E, H, generator=g) * 0.02).to(dt)
    bias = torch.randn(E, generator=g) * 0.5
    w, ids, lg = _router(x.to(dev), gate.to(dev), bias.to(dev), K, True, False)
    ref = oracle.router_logits(x, gate, bias)
    scale = (x.double().abs() @ gate.double().abs().t()).numpy()
    assert np.all(np.abs(lg - ref) <= 1e-5 * scale + 1e-6)
    # bit-exact selection on the kernel's own fp32 logits
    ow, oids = oracle.topk(lg, K, True)
    assert np.array_equal(ids, oids)
    assert np.max(np.abs(w - ow)) <= 1e-6


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_router_rounds_logits_to_model_dtype(dtype, dev):
    banner(f"router round_logits {dtype}")
    dt = {"bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    T, H, E, K = 256, 4096, 8, 2
    g = torch.Generator().manual_seed(11)
    x = torch.randn(T, H, generator=g).to(dt)
    gate = (torch.randn(E, H, generator=g) * 0.02).to(dt)
    w, ids, lg = _router(x.to(dev), gate.to(dev), None, K, True, True)
    ref = oracle.router_logits(x, gate, None, round_mode=1 if dtype == "bf16" else 2)
    # the kernel's logits are representable in the model dtype
    assert np.array_equal(torch.from_numpy(lg).to(dt).float().numpy(), lg)
    # fp32 sums that straddle a rounding boundary may land one unit apart
    ulp = np.abs(ref) * (2.0 ** -7 if dtype == "bf16" else 2.0 ** -10) + 1e-30
    assert np.all(np.abs(lg - ref) <= 1.01 * ulp)
    assert np.mean(lg == ref) > 0.99
    ow, oids = oracle.topk(lg, K, True)
    assert np.array_equal(ids, oids)


def test_router_entropy_adaptive_branch(dev):
    banner("router entropy-adaptive k")
    T, H, E, K = 128, 1024, 8, 4
    g = torch.Generator().manual_seed(5)
    x = torch.randn(T, H, generator=g)
    gate = torch.randn(E, H, generator=g) * torch.linspace(0.001, 0.2, T).mean()
    w, ids, lg = _router(x.to(dev), gate.to(dev), None, K, True, False, kmin=2)
    ow, oids = oracle.topk(lg, K, True, entropy_k_min=2)
    assert np.array_equal(ids, oids)
    assert np.max(np.abs(w - ow)) <= 1e-6
    assert np.allclose(w.sum(1), 1.0, atol=1e-6)


def test_router_rejects_bad_arguments(dev):
    x = torch.zeros(4, 64, device=dev)
    gate = torch.zeros(8, 64, device=dev)
    w = torch.empty(4, 2, device=dev)
    ids = torch.empty(4, 2, dtype=torch.int32, device=dev)
    with pytest.raises(_capi.MoeLibError, match="top-k"):
        _capi.router_topk(x, gate, None, 9, True, False, 0, w, ids)
    with pytest.raises(_capi.MoeLibError, match="entropy_k_min"):
        _capi.router_topk(x, gate, None, 2, True, False, 3, w, ids)


@pytest.mark.parametrize("T,E,K,n", [(1, 64, 6, 2), (300, 8, 2, 1), (1100, 16, 2, 3)])
def test_router_strided_output(T, E, K, n, dev):
    """moe355_router_topk_ld: token t's K results land at row t of [T, K+n]
    arrays, bit-equal to the unstrided router; columns K.. keep their values."""
    g = torch.Generator().manual_seed(T + E)
    x = torch.randn(T, 1024, generator=g).to(torch.bfloat16).to(dev)
    gate = (torch.randn(E, 1024, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    w0, ids0, _ = _router(x, gate, None, K, True, True)
    w = torch.full((T, K + n), -7.0, dtype=torch.float32, device=dev)
    ids = torch.full((T, K + n), -9, dtype=torch.int32, device=dev)
    _capi.router_topk(x, gate, None, K, True, True, 0, w, ids)
    torch.cuda.synchronize()
    w, ids = w.cpu().numpy(), ids.cpu().numpy()
    assert np.array_equal(ids[:, :K], ids0) and np.array_equal(w[:, :K], w0)
    assert (ids[:, K:] == -9).all() and (w[:, K:] == -7.0).all()


@pytest.mark.parametrize("T,H,E,K,kmin,ld", [(8, 2048, 64, 6, 0, 8), (1, 2048, 64, 6, 0, 6),
                                             (200, 1024, 32, 4, 0, 4), (16, 4096, 256, 8, 3, 8),
                                             (3, 512, 17, 2, 0, 3)])
def test_split_router_with_logits_buffer(T, H, E, K, kmin, ld, dev):
    """Few tokens over many experts with a logits buffer: the logits come from
    (token, 8-expert) workgroups and a second launch selects. Logits against
    the fp64 oracle (rounded to bf16, plus the bias), ids bit-exact and
    weights within 1e-6 on those logits, strided rows and the
    entropy-adaptive branch included."""
    banner(f"split router T={T} H={H} E={E} K={K} kmin={kmin} ld={ld}")
    g = torch.Generator().manual_seed(T * E + K)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    gate = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(E, generator=g) * 0.5
    w = torch.full((T, ld), -7.0, dtype=torch.float32, device=dev)
    ids = torch.full((T, ld), -9, dtype=torch.int32, device=dev)
    lg = torch.empty((T, E), dtype=torch.float32, device=dev)
    _capi.router_topk(x.to(dev), gate.to(dev), bias.to(dev), K, True, True, kmin, w, ids,
                      logits_out=lg)
    torch.cuda.synchronize()
    lg_h, w_h, ids_h = lg.cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy()
    ref = oracle.router_logits(x, gate, bias, round_mode=1)
    ulp = np.abs(ref - bias.numpy()[None, :]) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(lg_h - ref) <= 1.01 * ulp + 1e-6)
    ow, oids = oracle.topk(lg_h, K, True, entropy_k_min=kmin)
    assert np.array_equal(ids_h[:, :K], oids)
    assert np.max(np.abs(w_h[:, :K] - ow)) <= 1e-6
    assert (ids_h[:, K:] == -9).all() and (w_h[:, K:] == -7.0).all()
