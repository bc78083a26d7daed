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

from _helpers import ROUND, assert_matches_rounded, banner
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


def _fused(x, r, nw, nb, gate, bias, K, logits=True, renorm=True):
    T, H = x.shape
    E = gate.shape[0]
    nr, normed = torch.empty_like(x), torch.empty_like(x)
    w = torch.full((T, K), -7.0, dtype=torch.float32, device=x.device)
    ids = torch.full((T, K), -9, dtype=torch.int32, device=x.device)
    lg = torch.empty((T, E), dtype=torch.float32, device=x.device) if logits else None
    _capi.add_rmsnorm_router_topk(x, r, nr, nw, nb, 1e-5, gate, bias, K, renorm, True, normed,
                                  w, ids, logits_out=lg)
    return nr, normed, lg, w, ids


@pytest.mark.parametrize("dt,T,H,E,K,with_res,wdt", [
    (torch.bfloat16, 1, 4096, 8, 2, True, "same"),        # Mixtral decode
    (torch.bfloat16, 16, 4096, 8, 2, True, torch.float32),
    (torch.bfloat16, 1023, 4096, 8, 2, True, "same"),     # two rows a workgroup, ragged last
    (torch.bfloat16, 512, 2048, 16, 2, True, "same"),     # two rows, 16 experts a pass
    (torch.float16, 7, 2048, 64, 6, True, torch.float32),  # four double-buffered passes
    (torch.bfloat16, 200, 1024, 33, 5, True, "same"),     # a one-expert last pass
    (torch.bfloat16, 5, 8192, 60, 4, False, "same"),      # widest rows, no residual
    (torch.bfloat16, 5, 512, 3, 3, True, "same"),         # K == E
    # past the VALU kernel's range (T * E > 8192): the one-launch MFMA kernel
    (torch.bfloat16, 4096, 1024, 16, 2, True, "same"),
    (torch.bfloat16, 4096, 4096, 8, 2, True, "same"),     # Mixtral prefill
    (torch.float16, 2060, 2048, 16, 8, True, torch.float32),  # ragged last workgroup
    (torch.bfloat16, 2100, 256, 5, 3, False, "same"),     # narrowest rows, no residual
    # norm, then the MFMA router (below the one-launch kernel's 2048 rows)
    (torch.bfloat16, 1030, 2048, 16, 2, True, "same"),
    # norm, then the MFMA router (H not a multiple of 256)
    (torch.bfloat16, 2048, 1032, 8, 2, True, "same"),
    (torch.float32, 9, 1024, 8, 2, True, torch.float32),  # fp32: norm, then router
    (torch.bfloat16, 9, 1024, 128, 8, True, "same"),      # E > 64: norm, then router
])
def test_fused_norm_router_matches_oracle(dt, T, H, E, K, with_res, wdt, dev):
    """The one-launch norm + router: new residual bit-exact against the
    oracle; normed rows bit for bit the standalone norm's; logits within one
    storage step of the fp64 oracle on those rows (rounded, plus the bias);
    ids bit-exact and weights within 1e-6 of the oracle's top-k on the
    kernel's own logits."""
    banner(f"fused norm+router {dt} T={T} H={H} E={E} K={K} residual={with_res} w={wdt}")
    g = torch.Generator().manual_seed(T * 7 + E)
    x = torch.randn(T, H, generator=g).to(dt)
    r = torch.randn(T, H, generator=g).to(dt) if with_res else None
    wt = dt if wdt == "same" else wdt
    nw = (torch.rand(H, generator=g) + 0.5).to(wt)
    nb = (torch.randn(H, generator=g) * 0.1).to(wt) if wdt == "same" else None
    gate = (torch.randn(E, H, generator=g) * 0.02).to(dt)
    bias = torch.randn(E, generator=g) * 0.5
    xd = x.to(dev)
    rd = None if r is None else r.to(dev)
    nwd, nbd = nw.to(dev), None if nb is None else nb.to(dev)
    nr, normed, lg, w, ids = _fused(xd, rd, nwd, nbd, gate.to(dev), bias.to(dev), K)
    want_r = torch.empty_like(xd) if with_res else None
    want_n = torch.empty_like(xd)
    _capi.add_rmsnorm(xd, rd, want_r, nwd, nbd, 1e-5, want_n)
    torch.cuda.synchronize()
    ref_r, _ = oracle.add_rmsnorm(x, r, nw, nb, 1e-5)
    if with_res:
        assert np.array_equal(nr.double().cpu().numpy(), ref_r)
    assert torch.equal(normed, want_n)
    mode = {torch.bfloat16: 1, torch.float16: 2, torch.float32: 0}[dt]
    ref = oracle.router_logits(normed.cpu(), gate, bias, round_mode=mode)
    lg_h = lg.cpu().numpy()
    scale = (normed.cpu().double().abs() @ gate.double().abs().t()).numpy()
    if dt == torch.float32:
        # nothing rounded: within the fp32 accumulation error, as the router
        assert np.all(np.abs(lg_h - ref) <= 1e-5 * scale + 1e-6)
    else:
        ulp = np.abs(ref - bias.numpy()[None, :]) * STEP[dt] + 1e-30
        assert np.all(np.abs(lg_h - ref) <= 1.01 * ulp + 1e-6)
    ow, oids = oracle.topk(lg_h, K, True)
    assert np.array_equal(ids.cpu().numpy(), oids)
    assert np.max(np.abs(w.cpu().numpy() - ow)) <= 1e-6
    # Without a logits buffer (the fused kernel for up to 64 experts, the
    # one-workgroup router past them): same normed rows, and the routing of
    # logits each within one step of the oracle's.
    _, normed2, _, w2, ids2 = _fused(xd, rd, nwd, nbd, gate.to(dev), bias.to(dev), K,
                                     logits=False)
    torch.cuda.synchronize()
    assert torch.equal(normed2, want_n)
    if dt == torch.float32:
        delta = (1e-5 * scale + 1e-6).max(axis=1)
    else:
        delta = np.abs(ref - bias.numpy()[None, :]).max(axis=1) * STEP[dt] * 1.01 + 1e-6
    _check_routing_near(ids2.cpu().numpy(), w2.cpu().numpy(), ref, delta, K)


def _check_routing_near(ids, w, ref, delta, K):
    """ids / weights of a router whose logits were not returned, against the
    oracle's top-k on the oracle's logits ``ref``, each kernel logit within
    ``delta`` (per row) of ``ref``: a row's ids may differ only where two of
    its K+1 largest oracle logits lie within 2 * delta (a rounding flip);
    elsewhere each weight is within 2.2 * delta relative (the renormalised
    softmax moves by at most twice the largest logit error)."""
    ow, oids = oracle.topk(ref.astype(np.float32), K, True)
    top = -np.sort(-ref, axis=1)[:, :K + 1]
    gap = np.min(np.abs(np.diff(top, axis=1)), axis=1) if top.shape[1] > 1 else np.inf
    differ = np.any(ids != oids, axis=1)
    assert np.all(gap[differ] <= 2 * delta[differ]), np.nonzero(differ)[0][:8]
    same = ~differ
    tol = 2.2 * delta[same, None] * ow[same] + 1e-6
    assert np.all(np.abs(w[same] - ow[same]) <= tol)


@pytest.mark.parametrize("T", [1, 16, 300, 1030])
def test_forward_with_norm_matches_oracle(T, dev):
    """FusedMoE.forward_with_norm: the new residual equals the norm layer's,
    and the output is the oracle's experts on the fused call's own normed rows
    and routing (within each element's rounding plus the fp32 bound)."""
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
    _, want_res = norm.forward_add_residual(h, res)
    nw, nb = norm._params(h)
    _, normed, _, w, ids = _fused(h, res, nw, nb, moe.gate.detach().to(torch.bfloat16).contiguous(),
                                  None, K, logits=False, renorm=moe.renormalize)
    torch.cuda.synchronize()
    assert torch.equal(new_res, want_res)
    wn, idn = w.cpu().numpy(), ids.cpu().numpy().astype(np.int64)
    xn = normed.cpu()
    stored = out.double().cpu().numpy()
    assert oracle.max_rel(stored, oracle.fused_experts(xn, layer["w1"], layer["w2"], wn, idn)) \
        <= 2e-2
    rounded, allow = oracle.fused_experts_bound(xn, layer["w1"], layer["w2"], wn, idn, 0,
                                                ROUND[torch.bfloat16])
    assert_matches_rounded(stored, rounded, allow, torch.bfloat16)


@pytest.mark.parametrize("dt,T,H,E,K,with_res,wdt", [
    (torch.bfloat16, 4096, 4096, 8, 2, True, "same"),
    (torch.bfloat16, 2050, 4096, 16, 4, True, torch.float32),
    (torch.float16, 2055, 2048, 12, 8, False, "same"),
    (torch.bfloat16, 2048, 512, 9, 2, True, torch.float16),
    (torch.bfloat16, 8197, 3072, 3, 1, True, "same"),
])
def test_prefill_norm_router_equals_two_kernels(dt, T, H, E, K, with_res, wdt, dev):
    """At prefill sizes the one-launch MFMA kernel keeps the normed rows in
    LDS; every output is bit for bit the two-kernel path's (the norm, then the
    router's MFMA kernel on the stored rows), logits included."""
    banner(f"prefill norm+router {dt} T={T} H={H} E={E} K={K} residual={with_res} w={wdt}")
    g = torch.Generator().manual_seed(T + H + E)
    x = torch.randn(T, H, generator=g).to(dt).to(dev)
    r = torch.randn(T, H, generator=g).to(dt).to(dev) if with_res else None
    wt = dt if wdt == "same" else wdt
    nw = (torch.rand(H, generator=g) + 0.5).to(wt).to(dev)
    nb = (torch.randn(H, generator=g) * 0.1).to(wt).to(dev) if wdt == "same" else None
    gate = (torch.randn(E, H, generator=g) * 0.02).to(dt).to(dev)
    bias = (torch.randn(E, generator=g) * 0.5).to(dev)
    nr, normed, lg, w, ids = _fused(x, r, nw, nb, gate, bias, K)
    want_r = torch.empty_like(x) if with_res else None
    want_n = torch.empty_like(x)
    _capi.add_rmsnorm(x, r, want_r, nw, nb, 1e-5, want_n)
    want_lg = torch.empty_like(lg)
    want_w = torch.full_like(w, -7.0)
    want_ids = torch.full_like(ids, -9)
    _capi.router_topk(want_n, gate, bias, K, True, True, 0, want_w, want_ids, logits_out=want_lg)
    torch.cuda.synchronize()
    if with_res:
        assert torch.equal(nr, want_r)
    assert torch.equal(normed, want_n)
    assert torch.equal(lg, want_lg)
    assert torch.equal(ids, want_ids) and torch.equal(w, want_w)
