"""GPU test of moe355_fused_experts_static, the entry point that allocates
nothing: its scratch is the library's static device array, not a workspace.

Called through the C ABI twice in a row on one stream (the second call with
fewer tokens, reading scratch the first call left behind), each output is
compared with moe355_fused_experts on its own workspace: bit for bit where the
static plan is the plan itself. Where the tiled paths had to drop their
down-projection partial tiles to fit (only the fp32 summation order of the
last round's items changes), every token is checked against the oracle that
rounds like the kernels: each element within its own bf16 rounding plus the
oracle's fp32 bound, and within 2e-2 max-relative of the workspace entry
point. A shape beyond the scratch size must fail with a clear error before
launching anything.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import ROUND, assert_matches_rounded, banner, skewed_ids, y_round_of
from oracle import oracle
from reframework_amd import _capi

pytestmark = pytest.mark.gpu


def _layer(H, I, E, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    w1 = [(torch.randn(2 * I, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
          for _ in range(E)]
    w2 = [(torch.randn(H, I, generator=g, device=dev) * 0.02).to(torch.bfloat16)
          for _ in range(E)]
    return w1, w2


def _inputs(T, H, E, K, seed, dev):
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
    ids = torch.from_numpy(skewed_ids(T, K, E, seed=seed, skew=1.1)).int()
    w = torch.from_numpy(np.random.default_rng(seed).random((T, K)).astype(np.float32))
    return x.to(dev), ids.to(dev), w.to(dev)


@pytest.mark.parametrize("H,I,E,K,T1,T2", [
    (1024, 2816, 8, 2, 16, 3),      # weight-streaming path, then its self-grouping form
    (2048, 1408, 64, 6, 64, 8),     # fine-grained decode, permute launch
    (1024, 2816, 8, 2, 512, 200),   # 256-row then 128-row token tiles, partial tiles dropped
])
def test_static_scratch_matches_workspace_entry_point(H, I, E, K, T1, T2, dev):
    w1, w2 = _layer(H, I, E, seed=H + E, dev=dev)
    p1, p2 = [t.data_ptr() for t in w1], [t.data_ptr() for t in w2]
    calls = []
    for T in (T1, T2):
        plan = _capi.make_plan(T, H, I, E, K, _capi.BF16)
        lean = plan.workspace_bytes > _capi.STATIC_SCRATCH_BYTES
        banner(f"fused_experts_static H={H} I={I} E={E} K={K} T={T} path={plan.path} "
               f"workspace={plan.workspace_bytes} lean={lean}")
        x, ids, w = _inputs(T, H, E, K, seed=T, dev=dev)
        out = torch.full((T, H), 7.0, dtype=torch.bfloat16, device=dev)
        _capi.fused_experts_static(x, p1, p2, I, w, ids, 0, out)
        calls.append((plan, lean, x, ids, w, out))
    torch.cuda.synchronize()
    for plan, lean, x, ids, w, out in calls:
        T = x.shape[0]
        ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=dev)
        want = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        _capi.fused_experts(x, p1, p2, I, w, ids, 0, want, ws)
        torch.cuda.synchronize()
        if not lean:
            assert torch.equal(out, want)
            continue
        a, b = out.float(), want.float()
        rel = ((a - b).abs().max() / b.abs().max()).item()
        print(f"  T={T}: max_rel against the workspace entry point {rel:.2e}", flush=True)
        assert rel <= 2e-2
        w1h, w2h = [t.cpu() for t in w1], [t.cpu() for t in w2]
        ids_h = ids.cpu().numpy().astype(np.int64)
        rounded, allow = oracle.fused_experts_bound(
            x.cpu(), w1h, w2h, w.cpu().numpy(), ids_h, 0, ROUND[torch.bfloat16],
            y_round=y_round_of(plan, torch.bfloat16))
        assert_matches_rounded(a.cpu().numpy().astype(np.float64), rounded, allow,
                               torch.bfloat16)


def test_static_scratch_accumulates_into_fp32(dev):
    """accumulate_f32 (the streaming layer's mode): the sum is added to out."""
    H, I, E, K, T = 1024, 2816, 8, 2, 4
    banner("fused_experts_static accumulate_f32")
    w1, w2 = _layer(H, I, E, seed=5, dev=dev)
    p1, p2 = [t.data_ptr() for t in w1], [t.data_ptr() for t in w2]
    x, ids, w = _inputs(T, H, E, K, seed=9, dev=dev)
    base = torch.randn(T, H, generator=torch.Generator().manual_seed(3)).to(dev)
    acc_s, acc_w = base.clone(), base.clone()
    _capi.fused_experts_static(x, p1, p2, I, w, ids, 0, acc_s, accumulate_f32=True)
    plan = _capi.make_plan(T, H, I, E, K, _capi.BF16)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=dev)
    _capi.fused_experts(x, p1, p2, I, w, ids, 0, acc_w, ws, accumulate_f32=True)
    torch.cuda.synchronize()
    assert torch.equal(acc_s, acc_w)


def test_static_scratch_rejects_oversize_shapes_before_launching(dev):
    """Mixtral's 4096-token plan needs ~300 MB of scratch: a clear error, and
    the output is left untouched (nothing was launched)."""
    H, I, E, K, T = 4096, 14336, 8, 2, 4096
    banner("fused_experts_static oversize")
    plan = _capi.make_plan(T, H, I, E, K, _capi.BF16)
    assert plan.off_part > _capi.STATIC_SCRATCH_BYTES
    w1 = [torch.empty(16, dtype=torch.bfloat16, device=dev) for _ in range(E)]
    x = torch.zeros(T, H, dtype=torch.bfloat16, device=dev)
    ids = torch.zeros(T, K, dtype=torch.int32, device=dev)
    w = torch.zeros(T, K, dtype=torch.float32, device=dev)
    out = torch.full((T, H), 3.0, dtype=torch.bfloat16, device=dev)
    with pytest.raises(_capi.MoeLibError, match="static"):
        _capi.fused_experts_static(x, [t.data_ptr() for t in w1], [t.data_ptr() for t in w1], I,
                                   w, ids, 0, out)
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())
