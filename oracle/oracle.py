"""Python side of the CPU oracle (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the oracle results are compared against (or the
timed CPU baseline). The product
package never imports it.

``moe_oracle.c`` holds the fp64 restatement of the reference algorithm; this
module loads ``_build/libmoe_oracle.so`` (``make -C oracle``) and wraps it for
numpy / torch CPU tensors. ``ref_torch.py`` holds the reference's torch-CPU
forward restated with the reference's own dtype roundings.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libmoe_oracle.so")

F32, BF16, F16 = 0, 1, 2
ROUND_NONE, ROUND_BF16, ROUND_F16, ROUND_F32 = 0, 1, 2, 3
_TYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: run `make -C {HERE}`")
        h = ctypes.CDLL(LIB_PATH)
        P, I = ctypes.c_void_p, ctypes.c_int
        h.oracle_router_logits.argtypes = [P, P, I, P, I, I, I, I, P]
        h.oracle_router_logits.restype = None
        h.oracle_topk.argtypes = [P, I, I, I, I, I, P, P]
        h.oracle_topk.restype = I
        h.oracle_permute.argtypes = [P, I, I, I, P, I, P, P, P]
        h.oracle_permute.restype = I
        h.oracle_fused_experts.argtypes = [P, I, ctypes.POINTER(P), ctypes.POINTER(P), I, P, P,
                                           I, I, I, I, I, I, I, I, P, I, P]
        h.oracle_fused_experts.restype = I
        h.oracle_fused_experts_bound.argtypes = [P, I, ctypes.POINTER(P), ctypes.POINTER(P), I, P,
                                                 P, I, I, I, I, I, I, I, I, P, I, P, P]
        h.oracle_fused_experts_bound.restype = I
        h.oracle_round.argtypes = [P, ctypes.c_size_t, I]
        h.oracle_round.restype = None
        h.oracle_add_rmsnorm.argtypes = [P, P, I, P, P, ctypes.c_double, I, I, P, P]
        h.oracle_add_rmsnorm.restype = None
        h.oracle_quantize_int8.argtypes = [P, ctypes.c_size_t, P]
        h.oracle_quantize_int8.restype = ctypes.c_float
        h.oracle_experts_int8.argtypes = [P, I, I, I, I, I, ctypes.POINTER(P), ctypes.POINTER(P),
                                          P, P, P, P, P, I, P]
        h.oracle_experts_int8.restype = I
        _lib = h
    return _lib


def _cpu(t: torch.Tensor) -> torch.Tensor:
    return t.detach().cpu().contiguous()


def _raw(t: torch.Tensor):
    """(contiguous CPU tensor, oracle type code) for fp32/bf16/f16 tensors."""
    t = _cpu(t)
    return t, _TYPES[t.dtype]


def round_array(a: np.ndarray, mode: int) -> np.ndarray:
    v = np.ascontiguousarray(a, dtype=np.float64).copy()
    lib().oracle_round(v.ctypes.data, v.size, mode)
    return v


def router_logits(x: torch.Tensor, gate: torch.Tensor, bias: Optional[torch.Tensor] = None,
                  round_mode: int = ROUND_NONE) -> np.ndarray:
    """fp32 logits [T,E] of x [T,H] and gate [E,H] (same storage dtype)."""
    xt, tx = _raw(x)
    gt, tg = _raw(gate)
    assert tx == tg
    T, H = xt.shape
    E = gt.shape[0]
    out = np.empty((T, E), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(_cpu(bias).numpy(), dtype=np.float32)
    lib().oracle_router_logits(xt.data_ptr(), gt.data_ptr(), tx,
                               None if b is None else b.ctypes.data, T, H, E, round_mode,
                               out.ctypes.data)
    return out


def topk(logits: np.ndarray, K: int, renormalize: bool, entropy_k_min: int = 0):
    """(weights fp32 [T,K], ids int32 [T,K]); lower id wins exact ties."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = lg.shape
    w = np.empty((T, K), dtype=np.float32)
    ids = np.empty((T, K), dtype=np.int32)
    rc = lib().oracle_topk(lg.ctypes.data, T, E, K, int(renormalize), entropy_k_min,
                           w.ctypes.data, ids.ctypes.data)
    if rc != 0:
        raise ValueError("oracle_topk: bad sizes")
    return w, ids


def permute(ids: np.ndarray, E: int, expert_map: Optional[Sequence[int]] = None):
    """(offsets [E+1], slot_to_row [T*K], row_src [T*K]) of a stable grouping."""
    a = np.ascontiguousarray(ids, dtype=np.int64)
    T, K = a.shape
    R = T * K
    offsets = np.empty(E + 1, dtype=np.int32)
    s2r = np.empty(max(R, 1), dtype=np.int32)
    src = np.empty(max(R, 1), dtype=np.int32)
    m = None if not expert_map else np.ascontiguousarray(expert_map, dtype=np.int32)
    lib().oracle_permute(a.ctypes.data, T, K, E, None if m is None else m.ctypes.data,
                         0 if m is None else len(m), offsets.ctypes.data, s2r.ctypes.data,
                         src.ctypes.data)
    return offsets, s2r[:R], src[:R]


def fused_experts(x: torch.Tensor, w1: Sequence[torch.Tensor], w2: Sequence[torch.Tensor],
                  topk_w: np.ndarray, ids: np.ndarray, activation: int = 0,
                  inter_round: int = ROUND_NONE,
                  tokens: Optional[Sequence[int]] = None,
                  y_round: int = ROUND_NONE) -> np.ndarray:
    """fp64 [T,H] output of the routed experts (rows outside ``tokens`` are 0).
    ``inter_round`` / ``y_round`` round the activated intermediate / each
    slot's down-projection output to a storage type, as the reference's
    model-dtype matmuls do (fused.py:80-83)."""
    xt, tx = _raw(x)
    w1c = [_raw(w)[0] for w in w1]
    w2c = [_raw(w)[0] for w in w2]
    tw = _TYPES[w1c[0].dtype]
    T, H = xt.shape
    I = w1c[0].shape[0] // 2
    E = len(w1c)
    tw_arr = np.ascontiguousarray(topk_w, dtype=np.float32)
    id_arr = np.ascontiguousarray(ids, dtype=np.int64)
    K = id_arr.shape[1]
    P = ctypes.c_void_p
    p1 = (P * E)(*[w.data_ptr() for w in w1c])
    p2 = (P * E)(*[w.data_ptr() for w in w2c])
    out = np.zeros((T, H), dtype=np.float64)
    tok = None if tokens is None else np.ascontiguousarray(tokens, dtype=np.int32)
    lib().oracle_fused_experts(xt.data_ptr(), tx, p1, p2, tw, tw_arr.ctypes.data,
                               id_arr.ctypes.data, T, H, I, E, K, activation, inter_round, y_round,
                               None if tok is None else tok.ctypes.data,
                               0 if tok is None else len(tok), out.ctypes.data)
    return out


def fused_experts_bound(x: torch.Tensor, w1: Sequence[torch.Tensor], w2: Sequence[torch.Tensor],
                        topk_w: np.ndarray, ids: np.ndarray, activation: int, inter_round: int,
                        y_round: int = ROUND_NONE, tokens: Optional[Sequence[int]] = None):
    """(out, allow): fused_experts with the given roundings, and per output
    element how far a correct fp32 evaluation may land from ``out`` beyond
    the output's own rounding — the fp32 accumulation error of each slot's y
    plus, for every intermediate (and y, where rounded) that may round to the
    neighbouring storage value once computed in fp32, the effect of that other
    rounding (moe_oracle.c: oracle_fused_experts_bound). A checker bound for
    the tests, not part of the reference's algorithm."""
    xt, tx = _raw(x)
    w1c = [_raw(w)[0] for w in w1]
    w2c = [_raw(w)[0] for w in w2]
    tw = _TYPES[w1c[0].dtype]
    T, H = xt.shape
    I = w1c[0].shape[0] // 2
    E = len(w1c)
    tw_arr = np.ascontiguousarray(topk_w, dtype=np.float32)
    id_arr = np.ascontiguousarray(ids, dtype=np.int64)
    K = id_arr.shape[1]
    P = ctypes.c_void_p
    p1 = (P * E)(*[w.data_ptr() for w in w1c])
    p2 = (P * E)(*[w.data_ptr() for w in w2c])
    out = np.zeros((T, H), dtype=np.float64)
    allow = np.zeros((T, H), dtype=np.float64)
    tok = None if tokens is None else np.ascontiguousarray(tokens, dtype=np.int32)
    lib().oracle_fused_experts_bound(xt.data_ptr(), tx, p1, p2, tw, tw_arr.ctypes.data,
                                     id_arr.ctypes.data, T, H, I, E, K, activation, inter_round,
                                     y_round, None if tok is None else tok.ctypes.data,
                                     0 if tok is None else len(tok), out.ctypes.data,
                                     allow.ctypes.data)
    return out, allow


def add_rmsnorm(x: torch.Tensor, residual: Optional[torch.Tensor], weight, bias, eps: float):
    """(new residual, normed), both fp64 [T,H] holding storage-dtype values,
    of reframework/layers/norm.py:27-53 (x and residual in one storage dtype;
    weight and bias any float arrays of length H)."""
    xt, tx = _raw(x)
    T, H = xt.shape
    rt = None
    if residual is not None:
        rt, tr = _raw(residual)
        assert tr == tx
    w = np.ascontiguousarray(_cpu(torch.as_tensor(weight)).double().numpy())
    b = None if bias is None else np.ascontiguousarray(_cpu(torch.as_tensor(bias)).double().numpy())
    r_out = np.empty((T, H), dtype=np.float64)
    n_out = np.empty((T, H), dtype=np.float64)
    lib().oracle_add_rmsnorm(xt.data_ptr(), None if rt is None else rt.data_ptr(), tx,
                             w.ctypes.data, None if b is None else b.ctypes.data, float(eps), T, H,
                             r_out.ctypes.data, n_out.ctypes.data)
    return r_out, n_out


def max_rel(out: np.ndarray, ref: np.ndarray) -> float:
    """max |out - ref| / max |ref| — the layer tolerance metric."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = float(np.max(np.abs(ref)))
    return float(np.max(np.abs(out - ref))) / (denom if denom > 0 else 1.0)


def quantize_int8(w) -> tuple:
    """(int8 codes, scale) of ``w`` (any shape; widened to fp32) by the
    reference's symmetric per-tensor rule."""
    v = np.ascontiguousarray(_cpu(w).float().numpy() if isinstance(w, torch.Tensor) else
                             np.asarray(w, dtype=np.float32))
    q = np.empty(v.shape, dtype=np.int8)
    scale = lib().oracle_quantize_int8(v.ctypes.data, v.size, q.ctypes.data)
    return q, float(scale)


def experts_int8(x: torch.Tensor, w1q: Sequence[np.ndarray], w2q: Sequence[np.ndarray],
                 s1: Sequence[float], s2: Sequence[float], slot_offsets: np.ndarray,
                 slot_tokens: np.ndarray, slot_weights: np.ndarray, act: int = 0) -> np.ndarray:
    """fp32 [T,H]: the reference's int8 host experts (fused_experts_cpu_int8)
    over the given slots, in the reference's own fp32 / integer steps."""
    xt, tx = _raw(x)
    T, H = xt.shape
    n = len(w1q)
    I = w2q[0].shape[1] if n else 1
    q1 = [np.ascontiguousarray(a, dtype=np.int8) for a in w1q]
    q2 = [np.ascontiguousarray(b, dtype=np.int8) for b in w2q]
    P = ctypes.c_void_p
    t1 = (P * max(n, 1))(*[a.ctypes.data for a in q1])
    t2 = (P * max(n, 1))(*[b.ctypes.data for b in q2])
    sc1 = np.ascontiguousarray(np.asarray(s1, dtype=np.float32).reshape(-1))
    sc2 = np.ascontiguousarray(np.asarray(s2, dtype=np.float32).reshape(-1))
    offs = np.ascontiguousarray(slot_offsets, dtype=np.int32)
    toks = np.ascontiguousarray(slot_tokens, dtype=np.int32)
    wts = np.ascontiguousarray(slot_weights, dtype=np.float32)
    out = np.zeros((T, H), dtype=np.float32)
    rc = lib().oracle_experts_int8(xt.data_ptr(), tx, T, H, I, n, t1, t2, sc1.ctypes.data,
                                   sc2.ctypes.data, offs.ctypes.data, toks.ctypes.data,
                                   wts.ctypes.data, int(act), out.ctypes.data)
    if rc != 0:
        raise ValueError("oracle_experts_int8: bad sizes")
    return out
