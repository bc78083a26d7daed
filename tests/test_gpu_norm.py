"""GPU parity of the residual-add + RMSNorm kernel and the fused norm + router
entry against the oracle.

Reference: RMSNorm._forward / forward_add_residual
(reframework/layers/norm.py:27-53) and the decoder step that feeds the MoE
(reframework/models/base.py:135-136). Bars: the new residual is bit-exact (one
rounding of an exact fp32 sum); normed values are within one storage-dtype
step of the fp64 oracle (the kernel's fp32 sum of squares and square root may
round the scale differently); routing on the normed rows is checked like the
router itself.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import banner
from oracle import oracle
from reframework_amd import _capi, synth
from reframework_amd.layers import RMSNorm
from reframework_amd.moe import FusedMoE

pytestmark = pytest.mark.gpu

STEP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -22}
# spacing of the smallest (subnormal) values of each storage type
FLOOR = {torch.bfloat16: 2.0 ** -133, torch.float16: 2.0 ** -24, torch.float32: 2.0 ** -149}


def _within_one_step(got: torch.Tensor, ref: np.ndarray, dt, bias=None) -> float:
    """max over elements of |got - ref| / (one storage step of ref + the fp32
    rounding of the terms the reference also forms in fp32: r*inv*w and b,
    a few units of 2^-24 each, which dominates only where the bias cancels)."""
    g = got.double().cpu().numpy()
    err = np.abs(g - ref)
    b = 0.0 if bias is None else np.abs(bias.double().numpy())[None, :]
    terms = np.abs(ref) + 2.0 * b
    tol = np.abs(ref) * STEP[dt] + 8.0 * 2.0 ** -24 * terms + FLOOR[dt]
    return float((err / tol).max())


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("T,H", [(1, 1024), (7, 4096), (300, 2048), (3, 8192)])
@pytest.mark.parametrize("wdt,with_bias", [(torch.float32, False), ("same", True)])
def test_add_rmsnorm_matches_oracle(dt, T, H, wdt, with_bias, dev):
    banner(f"add_rmsnorm {dt} T={T} H={H} w={wdt} bias={with_bias}")
    if H * (4 if dt == torch.float32 else 2) > 8 * 256 * 16:
        pytest.skip("beyond the kernel's hidden-size limit for this dtype")
    g = torch.Generator().manual_seed(T + H)
    x = (torch.randn(T, H, generator=g) * 2).to(dt)
    r = torch.randn(T, H, generator=g).to(dt)
    wt = dt if wdt == "same" else wdt
    w = (torch.rand(H, generator=g) + 0.5).to(wt)
    b = torch.randn(H, generator=g).to(wt) * 0.1 if with_bias else None
    xd, rd = x.to(dev), r.to(dev)
    new_r = torch.empty_like(xd)
    out = torch.empty_like(xd)
    _capi.add_rmsnorm(xd, rd, new_r, w.to(dev), None if b is None else b.to(dev), 1e-5, out)
    torch.cuda.synchronize()
    ref_r, ref_n = oracle.add_rmsnorm(x, r, w, b, 1e-5)
    assert np.array_equal(new_r.double().cpu().numpy(), ref_r)
    assert _within_one_step(out, ref_n, dt, b) <= 1.0
    # plain norm, in place
    y = xd.clone()
    _capi.add_rmsnorm(y, None, None, w.to(dev), None if b is None else b.to(dev), 1e-5, y)
    torch.cuda.synchronize()
    _, ref_plain = oracle.add_rmsnorm(x, None, w, b, 1e-5)
    assert _within_one_step(y, ref_plain, dt, b) <= 1.0


def test_rmsnorm_layer_surface(dev):
    banner("RMSNorm layer")
    H = 512
    norm = RMSNorm(H, 1e-6).to(dev)
    with torch.no_grad():
        norm.weight.copy_(torch.linspace(0.5, 1.5, H))
    g = torch.Generator().manual_seed(47)
    x = torch.randn(6, H, generator=g).to(torch.bfloat16)
    r = torch.randn(6, H, generator=g).to(torch.bfloat16)
    xd, rd = x.to(dev), r.to(dev)
    f, new_r = norm.forward_add_residual(xd, rd)
    torch.cuda.synchronize()
    assert torch.equal(rd.cpu(), r) and torch.equal(xd.cpu(), x)  # inputs untouched
    ref_r, ref_n = oracle.add_rmsnorm(x, r, norm.weight.detach().cpu(), None, 1e-6)
    assert np.array_equal(new_r.double().cpu().numpy(), ref_r)
    assert _within_one_step(f, ref_n, torch.bfloat16) <= 1.0
    y = xd.clone()
    norm.forward_inplace(y)
    assert torch.equal(y, norm(xd))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        RMSNorm(H, 1e-6)(x)


@pytest.mark.parametrize("T", [1, 16, 300])
def test_forward_with_norm_equals_norm_then_layer(T, dev):
    banner(f"fused norm + router + experts T={T}")
    E, K, H, I = 8, 2, 1024, 512
    moe = FusedMoE(E, K, H, I, dtype=torch.bfloat16)
    layer = synth.make_layer(synth.MoEShape("t", H, E, K, I), torch.bfloat16, seed=T)
    sd = {"gate.weight": layer["gate"]}
    for e in range(E):
        sd[f"experts.{e}.gate_proj.weight"] = layer["w1"][e][:I]
        sd[f"experts.{e}.up_proj.weight"] = layer["w1"][e][I:]
        sd[f"experts.{e}.down_proj.weight"] = layer["w2"][e]
    moe.load_state_dict(sd)
    moe = moe.to(dev)
    norm = RMSNorm(H, 1e-5).to(dev)
    with torch.no_grad():
        norm.weight.uniform_(0.5, 1.5)
    g = torch.Generator().manual_seed(53)
    h = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    res = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    out, new_res = moe.forward_with_norm(h, res, norm)
    f, want_res = norm.forward_add_residual(h, res)
    want = moe(f)
    torch.cuda.synchronize()
    assert torch.equal(new_res, want_res)
    assert torch.equal(out, want)
