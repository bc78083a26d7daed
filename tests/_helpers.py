"""Helpers shared by the GPU parity tests (not collected: no test_ prefix)."""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

from reframework_amd import _capi
from reframework_amd.moe.fused import run_experts

DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
ROUND = {torch.bfloat16: 1, torch.float16: 2, torch.float32: 3}


def banner(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def make_bank(E: int, H: int, I: int, dtype: torch.dtype, seed: int, scale: float = 0.05):
    """Per-expert CPU tensors w1 [2I,H], w2 [H,I] of `dtype`."""
    g = torch.Generator().manual_seed(seed)
    w1 = [(torch.randn(2 * I, H, generator=g) * scale).to(dtype) for _ in range(E)]
    w2 = [(torch.randn(H, I, generator=g) * scale).to(dtype) for _ in range(E)]
    return w1, w2


def skewed_ids(T: int, K: int, E: int, seed: int, skew: float = 1.0) -> np.ndarray:
    """[T,K] distinct expert ids per token with a Zipf-like popularity."""
    rng = np.random.default_rng(seed)
    p = (np.arange(1, E + 1, dtype=np.float64)) ** (-skew)
    p /= p.sum()
    perm = rng.permutation(E)
    out = np.empty((T, K), dtype=np.int64)
    for t in range(T):
        out[t] = perm[rng.choice(E, size=K, replace=False, p=p)]
    return out


def gpu_fused(x: torch.Tensor, w1: Sequence[torch.Tensor], w2: Sequence[torch.Tensor],
              topk_w: np.ndarray, ids: np.ndarray, act: int = 0,
              expert_map: Optional[List[int]] = None, ids64: bool = False,
              path: int = -1) -> torch.Tensor:
    """libmoe355 fused_experts on cuda:0 tensors; returns the device output."""
    dev = torch.device("cuda:0")
    xd = x.to(dev).contiguous()
    w1d = [w.to(dev).contiguous() for w in w1]
    w2d = [w.to(dev).contiguous() for w in w2]
    idt = torch.from_numpy(np.ascontiguousarray(ids)).to(dev)
    idt = idt.long() if ids64 else idt.int()
    tw = torch.from_numpy(np.ascontiguousarray(topk_w, dtype=np.float32)).to(dev)
    I = w1[0].shape[0] // 2
    out = run_experts(xd, [w.data_ptr() for w in w1d], [w.data_ptr() for w in w2d], I, tw, idt,
                      act, expert_map=expert_map, path=path)
    torch.cuda.synchronize()
    return out


def tile_height(n: int, tile_rows: int) -> int:
    """Rows per token tile of an expert of n rows in the tile map (the
    kernels' tile_height): 256-row maps share the rows evenly over ceil(n/256)
    tiles, the height rounded up to 32 rows; other maps are tile_rows apart."""
    if tile_rows != 256 or n <= 0:
        return tile_rows
    nt = -(-n // 256)
    return -(-(-(-n // nt)) // 32) * 32


def tile_order(counts) -> List[int]:
    """Experts in the order the permute lists their tiles: by row count,
    largest, smallest, second largest, second smallest, ... (ties by id)."""
    E = len(counts)
    by = sorted(range(E), key=lambda e: (-int(counts[e]), e))
    order = [0] * E
    for r, e in enumerate(by):
        order[2 * r if 2 * r < E else 2 * (E - 1 - r) + 1] = e
    return order


def read_ws(plan: _capi.Plan, ws: torch.Tensor, off: int, n: int) -> np.ndarray:
    """int32 array of n entries at byte offset `off` of the workspace."""
    return ws[off:off + 4 * n].cpu().view(torch.int32).numpy().copy()


def tail_split(n_work: int, G: int, nk: int, cap: int) -> Tuple[int, int, int]:
    """(n_full, n_units, S) of the tiled kernels' tail split, as the kernel
    derives it (reframework_amd/csrc/dma_pipe.h, work_split): lets a test
    state which shapes run the K-split tail and its fix-up."""
    R = n_work // G if G > 0 else 0
    tail = n_work - R * G
    if cap <= 0 or tail == 0:
        return n_work, 0, 1
    cap = min(cap, G)
    best, S, s = 14 * nk, 1, 2
    while s <= 16 and s * tail <= cap and nk % s == 0:
        c = 14 * nk // s + s * tail
        if c < best:
            best, S = c, s
        s *= 2
    return (R * G, tail * S, S) if S > 1 else (n_work, 0, 1)


def tiled_down_split(plan: _capi.Plan, counts: Sequence[int], cus: int) -> int:
    """S of the tiled down projection's tail split for per-expert row counts
    `counts` on `cus` CUs (1: no split); its partial tiles live at off_part."""
    n_t = sum(-(-int(c) // plan.tile_rows) for c in counts)
    n_wtiles = plan.H // 256
    G = min(n_wtiles * plan.max_tiles * plan.down_splits, cus)
    cap = (plan.workspace_bytes - plan.off_part) // (256 * 256 * 4)
    nk = plan.I // plan.down_splits // 64
    return tail_split(n_wtiles * n_t * plan.down_splits, G, nk, cap)[2]


def tiled_gate_up_split(plan: _capi.Plan, counts: Sequence[int], cus: int) -> int:
    """S of the tiled gate_up for per-expert row counts `counts` on `cus` CUs
    (1: no split)."""
    n_t = sum(-(-int(c) // plan.tile_rows) for c in counts)
    n_wtiles = plan.I // 128
    G = min(n_wtiles * plan.max_tiles, cus)
    cap = (plan.workspace_bytes - plan.off_y) // (256 * 256 * 4)
    return tail_split(n_wtiles * n_t, G, plan.H // 64, min(cap, 4096))[2]


def y_round_of(plan: _capi.Plan, dt: torch.dtype) -> int:
    """Rounding mode of each slot's down-projection output y under ``plan``:
    the layer dtype on the tiled paths with one K-split (the reference's
    model-dtype ``inter @ w2[e].t()``), none (fp32 y) on every other path."""
    tiled = plan.path in (_capi.PATH_MFMA_TILED, _capi.PATH_MFMA_TILED128)
    return ROUND[dt] if tiled and plan.down_splits == 1 and dt != torch.float32 else 0


def _round_to(a: np.ndarray, dt: torch.dtype) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dt).float().numpy()


def assert_y_rounding(got: np.ndarray, ref_expected: np.ndarray, ref_other: np.ndarray,
                      dt: torch.dtype) -> None:
    """The output follows the oracle with the plan's rounding of y, not the
    other one: its RMS distance to ``ref_expected`` is below 0.95x that to
    ``ref_other`` (an independent rounding of y adds a second error term of
    about the size of the output's own rounding, ~0.7x expected). Skipped
    where the two oracles round to the same outputs in the layer dtype (one
    slot of weight 1 per token: rounding y and then the output is rounding
    once)."""
    if dt == torch.float32:
        return
    differ = np.mean(_round_to(ref_expected, dt) != _round_to(ref_other, dt))
    if differ < 0.2:
        return
    d_exp = float(np.sqrt(np.mean((got - ref_expected) ** 2)))
    d_oth = float(np.sqrt(np.mean((got - ref_other) ** 2)))
    print(f"  y rounding: rms to expected {d_exp:.3e}, to the other {d_oth:.3e} "
          f"(ratio {d_exp / max(d_oth, 1e-300):.3f}, outputs differing {differ:.2f})", flush=True)
    assert d_exp < 0.95 * d_oth


# Half an ulp of the output's own rounding (relative to the value) and the
# noise allowed beyond it (relative to the largest output) in the tight check;
# with y rounded, one ulp of a slot's y more (2^-7 bf16, 2^-10 f16 of it).
_OUT_ROUND = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}
_NOISE = 1e-5  # of max|ref|: the fp32 sum of a token's slots in the combine


def assert_matches_rounded(got: np.ndarray, ref: np.ndarray, allow: np.ndarray,
                           dt: torch.dtype) -> float:
    """Tight check against the oracle that rounds the intermediate (and y)
    like the kernels, ``(ref, allow) = oracle.fused_experts_bound(...)``: every
    output element within its own rounding to ``dt`` (<= 2^-8 |v| for bf16,
    2^-11 |v| for f16) plus ``allow`` — the fp32 accumulation error of its
    slots' y, and the other rounding of every intermediate (and y, where
    rounded) that an fp32 evaluation may put on the other side of a rounding
    boundary — plus 1e-5 of the largest output. Returns the excess over that
    bound, relative to max |ref|."""
    scale = float(np.max(np.abs(ref))) or 1.0
    excess = float(np.max(np.abs(got - ref) - _OUT_ROUND[dt] * np.abs(ref) - allow)) / scale
    print(f"  beyond the output's own rounding and the fp32 bound: {max(excess, 0.0):.2e} of "
          f"max|ref| (bar {_NOISE:.0e}; bound mean {np.mean(allow) / scale:.1e}, max "
          f"{np.max(allow) / scale:.1e})", flush=True)
    assert excess <= _NOISE
    return excess
