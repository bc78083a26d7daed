"""GPU parity of permute, grouped expert FFN and combine against the oracle.

Reference: fused_experts (reframework/moe/fused.py:49-87). Bars:
  * grouping (offsets, slot_to_row, row_src): bit-exact;
  * fp32 layers: max|out-ref|/max|ref| <= 1e-5 against the fp64 oracle;
  * bf16/f16 layers: <= 2e-2 against the fp64 oracle; and, a tighter check
    of the GEMMs, against the oracle that rounds the intermediate to the
    storage type like the kernels do, and y too where the plan's path does
    (the tiled paths with one down K-split, as the reference's matmul): every
    element within its own output rounding plus the oracle's fp32 bound (the
    accumulation error of y and the other rounding of any intermediate or y
    that fp32 evaluation may put across a rounding boundary) plus 1e-5 of the
    largest output; and the output follows that rounding of y, not the other
    one.
Every kernel family (256- and 128-token-tile MFMA, skinny MFMA with split-K,
fp32 SIMT) is driven, with ragged and empty expert groups, tile-boundary group
sizes, dropped slots and int64 ids; each MFMA family is also forced onto
shapes the automatic choice would give another one.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import (DT, ROUND, assert_matches_rounded, assert_y_rounding, banner, gpu_fused,
                      make_bank, read_ws, skewed_ids, tile_height, tile_order, y_round_of)
from oracle import oracle
from reframework_amd import _capi
from reframework_amd.moe import fused_experts

pytestmark = pytest.mark.gpu

TOL_EXACT = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _check(out: torch.Tensor, x, w1, w2, w, ids, act=0, tokens=None, path=-1):
    """Output against the fp64 oracle and against the oracle that rounds the
    intermediate, and y where the plan's kernels do (``path`` as given to
    gpu_fused: the plan is rebuilt here to know which rounding applies)."""
    dt = w1[0].dtype
    T, H = x.shape
    plan = _capi.make_plan(T, H, w1[0].shape[0] // 2, len(w1), ids.shape[1],
                           _capi.dtype_code(dt), path)
    yr = y_round_of(plan, dt)
    got = out.float().cpu().numpy().astype(np.float64)
    exact = oracle.fused_experts(x, w1, w2, w, ids, activation=act, tokens=tokens)
    rounded, allow = oracle.fused_experts_bound(x, w1, w2, w, ids, act, ROUND[dt], y_round=yr,
                                                tokens=tokens)
    other = oracle.fused_experts(x, w1, w2, w, ids, activation=act, inter_round=ROUND[dt],
                                 y_round=0 if yr else ROUND[dt], tokens=tokens)
    if tokens is not None:
        got, exact, rounded, other = got[tokens], exact[tokens], rounded[tokens], other[tokens]
        allow = allow[tokens]
    e1 = oracle.max_rel(got, exact)
    e2 = oracle.max_rel(got, rounded)
    print(f"  path {plan.path} splits {plan.down_splits}: max_rel vs fp64 {e1:.2e}, vs the "
          f"oracle rounding inter{' and y' if yr else ''} {e2:.2e}", flush=True)
    assert e1 <= TOL_EXACT[dt]
    if dt == torch.float32:
        assert e2 <= TOL_EXACT[dt]
        return
    assert_matches_rounded(got, rounded, allow, dt)
    assert_y_rounding(got, rounded, other, dt)


# ------------------------------------------------------------------ permute
@pytest.mark.parametrize("T,K,E,ids64,drop", [
    (1, 2, 8, False, False), (16, 2, 8, True, False), (700, 6, 64, False, False),
    (4096, 2, 8, False, True), (3000, 8, 256, True, False), (2048, 2, 16, False, True),
])
def test_permute_bit_exact(T, K, E, ids64, drop, dev):
    banner(f"permute T={T} K={K} E={E} ids64={ids64} drop={drop}")
    ids = skewed_ids(T, K, E, seed=T + E, skew=1.2)
    emap = [(-1 if e % 5 == 3 else e) for e in range(E)] if drop else None
    plan = _capi.make_plan(T, 256, 256, E, K, _capi.BF16)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=dev)
    idt = torch.from_numpy(ids).to(dev)
    idt = idt if ids64 else idt.int()
    _capi.permute(plan, idt, ws, expert_map=emap)
    torch.cuda.synchronize()
    R = T * K
    offsets, s2r, src = oracle.permute(ids, E, emap)
    assert np.array_equal(read_ws(plan, ws, plan.off_offsets, E + 1), offsets)
    assert np.array_equal(read_ws(plan, ws, plan.off_slot_to_row, R), s2r)
    n = offsets[-1]
    assert np.array_equal(read_ws(plan, ws, plan.off_row_src, R)[:n], src[:n])
    # tile map: ceil(m_e / tile_rows) tiles per expert, the expert's tile
    # height apart, experts in the interleaved size order
    tm = read_ws(plan, ws, plan.off_tile_map, 2 + 2 * plan.max_tiles)
    counts = np.diff(offsets)
    want = [(e, offsets[e] + j * tile_height(counts[e], plan.tile_rows)) for e in tile_order(counts)
            for j in range(-(-counts[e] // plan.tile_rows))]
    assert tm[0] == len(want) <= plan.max_tiles and tm[1] == plan.tile_rows
    assert [tuple(p) for p in tm[2:2 + 2 * len(want)].reshape(-1, 2)] == want


@pytest.mark.parametrize("T,K,E,ids64,drop", [
    # grouped inside gate_up (<= 64 routed slots)
    (1, 2, 8, False, False), (8, 2, 8, True, True), (4, 4, 32, False, True),
    (5, 3, 16, True, False), (2, 8, 32, False, False), (16, 2, 8, True, True),
    (32, 2, 8, False, False), (8, 6, 64, True, False), (8, 8, 256, True, True),
    (3, 6, 64, False, True), (64, 1, 8, False, False), (16, 4, 16, True, True),
    # permute launch (more than 64 slots), same checks
    (16, 6, 64, False, False), (12, 8, 256, True, True),
])
def test_decode_grouping_inside_gate_up_bit_exact(T, K, E, ids64, drop, dev):
    """At decode sizes (skinny path, <= 64 routed slots) fused_experts skips
    the permute launch: the gate_up workgroups group the slots themselves and
    workgroup 0 writes the permute's outputs. Those outputs must equal the
    oracle's grouping bit for bit, and the layer output (also accumulated into
    fp32) the staged path's (larger cases take the permute launch and are held
    to the same checks)."""
    H, I = 256, 256
    banner(f"decode grouping in gate_up T={T} K={K} E={E} ids64={ids64} drop={drop}")
    ids = skewed_ids(T, K, E, seed=T * E + K, skew=1.2)
    emap = [(-1 if e % 5 == 3 else e) for e in range(E)] if drop else None
    plan = _capi.make_plan(T, H, I, E, K, _capi.BF16)
    assert plan.path == _capi.PATH_MFMA_SKINNY
    w1, w2 = make_bank(E, H, I, torch.bfloat16, seed=T + E)
    w1d = [w.to(dev).contiguous() for w in w1]
    w2d = [w.to(dev).contiguous() for w in w2]
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16).to(dev)
    tw = torch.from_numpy(np.random.default_rng(T).random((T, K)).astype(np.float32)).to(dev)
    idt = torch.from_numpy(ids).to(dev)
    idt = idt if ids64 else idt.int()
    p1 = [w.data_ptr() for w in w1d]
    p2 = [w.data_ptr() for w in w2d]
    ws = torch.full((plan.workspace_bytes,), 0x5A, dtype=torch.uint8, device=dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    _capi.fused_experts(x, p1, p2, I, tw, idt, 0, out, ws, expert_map=emap)
    # the staged entry points: permute launch, then the plain gate_up
    staged = torch.empty_like(out)
    ws2 = torch.empty_like(ws)
    _capi.permute(plan, idt, ws2, expert_map=emap)
    _capi.gate_up(plan, x, p1, 0, ws2)
    _capi.down(plan, p2, ws2)
    _capi.combine(plan, tw, staged, False, ws2)
    torch.cuda.synchronize()
    R = T * K
    offsets, s2r, src = oracle.permute(ids, E, emap)
    assert np.array_equal(read_ws(plan, ws, plan.off_offsets, E + 1), offsets)
    assert np.array_equal(read_ws(plan, ws, plan.off_slot_to_row, R), s2r)
    n = offsets[-1]
    assert np.array_equal(read_ws(plan, ws, plan.off_row_src, R)[:n], src[:n])
    counts = np.diff(offsets)
    # the in-kernel grouping lists the experts by id, the permute launch in
    # the interleaved size order
    order = range(E) if R <= 64 else tile_order(counts)
    want = [(e, offsets[e] + j * tile_height(counts[e], plan.tile_rows)) for e in order
            for j in range(-(-counts[e] // plan.tile_rows))]
    tm = read_ws(plan, ws, plan.off_tile_map, 2 + 2 * plan.max_tiles)
    assert tm[0] == len(want) <= plan.max_tiles and tm[1] == plan.tile_rows
    assert [tuple(p) for p in tm[2:2 + 2 * len(want)].reshape(-1, 2)] == want
    assert torch.equal(out, staged)
    if not drop:
        _check(out, x.cpu(), w1, w2, tw.cpu().numpy(), ids)
    # accumulate into an fp32 output (the streaming layer's mode): the same sums
    base = torch.randn(T, H, generator=torch.Generator().manual_seed(7)).to(dev)
    acc_f, acc_s = base.clone(), base.clone()
    _capi.fused_experts(x, p1, p2, I, tw, idt, 0, acc_f, ws, expert_map=emap, accumulate_f32=True)
    _capi.permute(plan, idt, ws2, expert_map=emap)
    _capi.gate_up(plan, x, p1, 0, ws2)
    _capi.down(plan, p2, ws2)
    _capi.combine(plan, tw, acc_s, True, ws2)
    torch.cuda.synchronize()
    assert torch.equal(acc_f, acc_s)


# ------------------------------------------------------------ expert FFN
CASES = [
    # name, T, K, E, H, I, dtype, expected path
    ("decode_t1", 1, 2, 8, 512, 1024, "bf16", _capi.PATH_MFMA_SKINNY),
    ("decode_t16", 16, 2, 8, 1024, 2048, "bf16", _capi.PATH_MFMA_SKINNY),
    ("decode_f16", 8, 2, 8, 512, 512, "f16", _capi.PATH_MFMA_SKINNY),
    ("finegrained_t8", 8, 6, 64, 256, 128, "bf16", _capi.PATH_MFMA_SKINNY),
    ("half_tiles_ragged", 150, 2, 8, 512, 384, "bf16", _capi.PATH_MFMA_TILED128),
    ("half_tiles_f16", 80, 2, 4, 256, 256, "f16", _capi.PATH_MFMA_TILED128),
    ("half_tiles_e16", 300, 2, 16, 512, 256, "bf16", _capi.PATH_MFMA_TILED128),
    ("prefill_ragged", 700, 2, 8, 512, 384, "bf16", _capi.PATH_MFMA_TILED),
    ("prefill_tiled", 1200, 2, 4, 512, 384, "bf16", _capi.PATH_MFMA_TILED),
    ("prefill_f16", 1000, 2, 4, 256, 256, "f16", _capi.PATH_MFMA_TILED),
    # over 512 rows per expert: the 256-row kernel's non-ragged f16 instance
    ("prefill_f16_tall", 1400, 2, 4, 256, 256, "f16", _capi.PATH_MFMA_TILED),
    ("fp32_tiny", 96, 2, 8, 256, 352, "f32", _capi.PATH_SIMT),
    ("fp32_decode", 3, 2, 8, 128, 96, "f32", _capi.PATH_SIMT),
    ("bf16_unaligned", 40, 2, 4, 136, 200, "bf16", _capi.PATH_SIMT),
    ("decode_i1408", 6, 2, 8, 256, 1408, "bf16", _capi.PATH_MFMA_SKINNY),
    ("decode_unaligned_k", 4, 2, 4, 160, 96, "bf16", _capi.PATH_SIMT),
    # many small experts, top-8 (Qwen3-MoE 128 experts; 256 is the library's maximum)
    ("e128_k8_prefill", 2048, 8, 128, 512, 256, "bf16", _capi.PATH_MFMA_TILED),
    ("e128_k8_half_tiles", 600, 8, 128, 512, 256, "bf16", _capi.PATH_MFMA_TILED128),
    ("e256_k8_half_tiles", 1024, 8, 256, 256, 256, "bf16", _capi.PATH_MFMA_TILED128),
    ("e256_k8_decode", 4, 8, 256, 256, 128, "bf16", _capi.PATH_MFMA_SKINNY),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_fused_experts_paths(case, dev):
    name, T, K, E, H, I, dts, path = case
    dt = DT[dts]
    plan = _capi.make_plan(T, H, I, E, K, _capi.dtype_code(dt))
    banner(f"fused_experts {name} T={T} K={K} E={E} H={H} I={I} {dts} path={plan.path} "
           f"splits={plan.down_splits}")
    assert plan.path == path
    w1, w2 = make_bank(E, H, I, dt, seed=T + H)
    x = (torch.randn(T, H, generator=torch.Generator().manual_seed(1))).to(dt)
    ids = skewed_ids(T, K, E, seed=T, skew=1.0)
    w = np.random.default_rng(3).random((T, K)).astype(np.float32)
    out = gpu_fused(x, w1, w2, w, ids)
    assert out.dtype == dt and out.shape == (T, H)
    _check(out, x, w1, w2, w, ids)


def test_split_k_down_projection_is_exercised():
    plan = _capi.make_plan(1, 4096, 14336, 8, 2, _capi.BF16)
    assert plan.path == _capi.PATH_MFMA_SKINNY and plan.down_splits > 1


@pytest.mark.parametrize("act", [1, 2])
@pytest.mark.parametrize("T", [4, 400])
def test_gelu_activations(act, T, dev):
    banner(f"activation={act} T={T}")
    E, K, H, I = 8, 2, 256, 256
    w1, w2 = make_bank(E, H, I, torch.bfloat16, seed=act)
    g = torch.Generator().manual_seed(100 + 10 * act + T)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    ids = skewed_ids(T, K, E, seed=act)
    w = np.full((T, K), 0.5, np.float32)
    _check(gpu_fused(x, w1, w2, w, ids, act=act), x, w1, w2, w, ids, act=act)


@pytest.mark.parametrize("T,K,E,H,I,seed", [(700, 2, 8, 512, 384, 1), (333, 6, 18, 512, 256, 2),
                                            (1, 2, 8, 256, 256, 3), (2048, 2, 16, 512, 512, 4),
                                            (64, 1, 1, 256, 256, 5), (100, 2, 8, 256, 256, 6)])
@pytest.mark.parametrize("path", [_capi.PATH_MFMA_TILED, _capi.PATH_MFMA_TILED128,
                                  _capi.PATH_MFMA_SKINNY])
def test_every_mfma_family_on_every_shape(path, T, K, E, H, I, seed, dev):
    banner(f"forced path={path} T={T} K={K} E={E} H={H} I={I}")
    w1, w2 = make_bank(E, H, I, torch.bfloat16, seed=seed)
    x = (torch.randn(T, H, generator=torch.Generator().manual_seed(seed))).to(torch.bfloat16)
    ids = skewed_ids(T, K, E, seed=seed, skew=1.1)
    w = np.random.default_rng(seed).random((T, K)).astype(np.float32)
    out = gpu_fused(x, w1, w2, w, ids, path=path)
    _check(out, x, w1, w2, w, ids, path=path)


@pytest.mark.parametrize("path", [-1, _capi.PATH_MFMA_TILED, _capi.PATH_MFMA_TILED128,
                                  _capi.PATH_MFMA_SKINNY])
@pytest.mark.parametrize("m", [63, 64, 65, 127, 128, 129, 255, 256, 257, 512, 513])
def test_tile_boundary_group_sizes(m, path, dev):
    # all m tokens to expert 0 (K=1) plus one token on expert 3
    banner(f"tile boundary m={m} path={path}")
    E, H, I = 4, 256, 256
    T = m + 1
    ids = np.zeros((T, 1), np.int64)
    ids[-1, 0] = 3
    w1, w2 = make_bank(E, H, I, torch.bfloat16, seed=m)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(1000 + m)).to(torch.bfloat16)
    w = np.ones((T, 1), np.float32)
    _check(gpu_fused(x, w1, w2, w, ids, path=path), x, w1, w2, w, ids, path=path)


def _tile_blocks(n):
    """Token-block pairs J the 256-row kernel multiplies for every tile of an
    expert of n rows outside ragged launches: its tile height / 32."""
    return tile_height(n, 256) // 32


@pytest.mark.parametrize("counts,I", [
    # 8 experts, 385 rows on average (ragged instance, rotated slots):
    # heights of J = 5, 5, 6, 8, 7, 1, 1, 8; a K-split tail
    ([257, 300, 513, 700, 1025, 1, 32, 255], 2048),
    # the same with 3 x 1200 rows more (over 512 on average: the instance
    # that multiplies the blocks of each expert's height)
    ([257, 300, 513, 700, 1025, 1, 32, 255, 1200, 1200, 1200], 2048),
    # 16 experts of 192 rows on average (ragged instance)
    ([29, 94, 140, 187, 257, 281, 369, 514, 1, 33, 64, 97, 128, 160, 224, 500], 1536),
], ids=["e8", "e11", "e16"])
def test_balanced_tile_heights(counts, I, dev):
    E, H = len(counts), 512
    assert sorted({min(8, _tile_blocks(n)) for n in counts if n}) == (
        [1, 2, 3, 4, 5, 6, 7, 8] if E == 16 else [1, 5, 6, 7, 8])
    T = sum(counts)
    ids = np.repeat(np.arange(E), counts)[np.random.default_rng(E).permutation(T)][:, None]
    plan = _capi.make_plan(T, H, I, E, 1, _capi.BF16, _capi.PATH_MFMA_TILED)
    banner(f"balanced tiles E={E} T={T} I={I} tiles<={plan.max_tiles}")
    w1, w2 = make_bank(E, H, I, torch.bfloat16, seed=E + 40)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(E + 41)).to(torch.bfloat16)
    w = np.random.default_rng(E + 42).random((T, 1)).astype(np.float32)
    out = gpu_fused(x, w1, w2, w, ids.astype(np.int64), path=_capi.PATH_MFMA_TILED)
    _check(out, x, w1, w2, w, ids.astype(np.int64), path=_capi.PATH_MFMA_TILED)


def test_dropped_slots_and_expert_map(dev):
    banner("expert_map drop/rename")
    T, K, Eg, H, I = 200, 2, 8, 256, 256
    ids = skewed_ids(T, K, Eg, seed=9)
    kept = [1, 4, 6]  # global ids kept; local rows 0..2
    emap = [kept.index(e) if e in kept else -1 for e in range(Eg)]
    w1, w2 = make_bank(len(kept), H, I, torch.bfloat16, seed=9)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    w = np.random.default_rng(9).random((T, K)).astype(np.float32)
    out = gpu_fused(x, w1, w2, w, ids, expert_map=emap, ids64=True)
    local = np.array([[emap[e] for e in row] for row in ids], np.int64)
    _check(out, x, w1, w2, w, local)


def test_all_slots_dropped_gives_zeros(dev):
    banner("all dropped")
    T, K, H, I = 5, 2, 256, 256
    w1, w2 = make_bank(2, H, I, torch.bfloat16, seed=1)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(17)).to(torch.bfloat16)
    ids = np.full((T, K), 7, np.int64)
    out = gpu_fused(x, w1, w2, np.ones((T, K), np.float32), ids, expert_map=[-1] * 8)
    assert torch.count_nonzero(out).item() == 0


def test_fused_experts_api_with_stacked_bank(dev):
    banner("fused_experts public API, stacked bank, fp32 hidden with bf16 experts")
    T, K, E, H, I = 64, 2, 8, 256, 256
    w1, w2 = make_bank(E, H, I, torch.bfloat16, seed=2)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(23))
    ids = skewed_ids(T, K, E, seed=2)
    w = np.random.default_rng(2).random((T, K)).astype(np.float32)
    out = fused_experts(x.to(dev), torch.stack(w1).to(dev), torch.stack(w2).to(dev),
                        torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev), "silu")
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    _check(out.to(torch.bfloat16), x.to(torch.bfloat16), w1, w2, w, ids)
    with pytest.raises(ValueError, match="unknown gated activation"):
        fused_experts(x.to(dev), torch.stack(w1).to(dev), torch.stack(w2).to(dev),
                      torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev), "relu")


def test_outputs_are_deterministic(dev):
    banner("determinism")
    T, K, E, H, I = 512, 2, 8, 512, 512
    w1, w2 = make_bank(E, H, I, torch.bfloat16, seed=4)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(31)).to(torch.bfloat16)
    ids = skewed_ids(T, K, E, seed=4)
    w = np.random.default_rng(4).random((T, K)).astype(np.float32)
    a = gpu_fused(x, w1, w2, w, ids)
    b = gpu_fused(x, w1, w2, w, ids)
    assert torch.equal(a, b)


@pytest.mark.parametrize("T", [4, 40, 700, 2048])
def test_zero_weight_slots_are_dropped(T, dev):
    """The reference's expert-parallel layer (parallel/ep.py:137-143) keeps
    the experts 2-5 of 8 on this rank, maps the others to local row 0 and
    zeroes their weights. fused_experts drops slots of weight 0: the output
    equals the oracle's with those slots removed, and expert 0's rows are its
    own slots only (the grouping inside gate_up at 4 tokens; the one-block
    permute with 128-row tiles at 40; the multi-block permute with 256-row
    tiles at 700 and 2048)."""
    E_all, K, H, I = 8, 2, 256, 512
    lo, hi = 2, 6
    E = hi - lo
    banner(f"zero-weight slots T={T}")
    ids_g = skewed_ids(T, K, E_all, seed=T, skew=0.5)
    local = (ids_g >= lo) & (ids_g < hi)
    ids = np.where(local, ids_g - lo, 0).astype(np.int64)
    w = np.random.default_rng(T).random((T, K)).astype(np.float32)
    w_masked = np.where(local, w, 0.0).astype(np.float32)
    w1, w2 = make_bank(E, H, I, torch.bfloat16, seed=T + 1)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    plan = _capi.make_plan(T, H, I, E, K, _capi.BF16)
    ws = torch.full((plan.workspace_bytes,), 0x5A, dtype=torch.uint8, device=dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    w1d = [t.to(dev).contiguous() for t in w1]
    w2d = [t.to(dev).contiguous() for t in w2]
    _capi.fused_experts(x.to(dev), [t.data_ptr() for t in w1d], [t.data_ptr() for t in w2d], I,
                        torch.from_numpy(w_masked).to(dev), torch.from_numpy(ids).to(dev), 0, out, ws)
    torch.cuda.synchronize()
    counts = np.diff(read_ws(plan, ws, plan.off_offsets, E + 1))
    want = np.bincount((ids_g[local] - lo).reshape(-1), minlength=E)
    assert np.array_equal(counts, want)
    ids_dropped = np.where(local, ids, -1)
    _check(out, x, w1, w2, w_masked, ids_dropped)
