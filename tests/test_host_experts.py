"""The host half of the CPU/GPU split forward (libmoe355_host.so) against the
oracle, on the CPU.

Reference: the CPU half of FusedMoE._forward_split
(reframework/moe/moe_layer.py:523-627) and fused_experts_cpu_int8
(reframework/moe/fused.py:140-197). The reference multiplies int8-quantized
weights; this library multiplies the staged 16-bit weights with the device
kernels' numerics (fp32 gate|up, the intermediate rounded once to the weight
type, fp32 down projection), so it is held to the same bars as the device
kernels: each output element within its own rounding plus the oracle's fp32
bound (assert_matches_rounded) for bf16/f16, 1e-5 max-relative for fp32 and
2e-2 max-relative against the fp64 oracle that rounds nothing. Every slot
contributes to the token at its own (token, k) position (the reference's
split indexes tokens as if K were 1, F6).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from _helpers import ROUND, assert_matches_rounded
from oracle import oracle
from reframework_amd import _capi


def _slots(ids: np.ndarray, w: np.ndarray, experts):
    """Slot arrays of the host call: for each expert of ``experts`` (in that
    order) its (token, weight) pairs in token order."""
    offs, toks, wts = [0], [], []
    for e in experts:
        t, k = np.nonzero(ids == e)
        order = np.lexsort((k, t))
        toks.extend(t[order].tolist())
        wts.extend(w[t[order], k[order]].tolist())
        offs.append(len(toks))
    return (np.asarray(offs, np.int32), np.asarray(toks if toks else [0], np.int32),
            np.asarray(wts if wts else [0.0], np.float32))


def _case(T, H, I, E, K, dt, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(T, H, generator=g) * 0.7).to(dt)
    w1 = [(torch.randn(2 * I, H, generator=g) * 0.05).to(dt) for _ in range(E)]
    w2 = [(torch.randn(H, I, generator=g) * 0.05).to(dt) for _ in range(E)]
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.random((T, K)).astype(np.float32)
    return x, w1, w2, ids, w


@pytest.mark.parametrize("isa", ["avx2", "avx512", "avx512bf16"])
@pytest.mark.parametrize("dt,H,I,act", [
    (torch.bfloat16, 256, 384, 0), (torch.bfloat16, 200, 136, 1), (torch.float16, 512, 256, 2),
    (torch.float32, 192, 160, 0), (torch.bfloat16, 64, 40, 0)])
def test_host_experts_match_oracle(dt, H, I, act, isa, monkeypatch):
    """Random routing over 5 experts, 3 of them run on the host (the others
    marked -1 for the oracle), tails of 8/16-wide vectors included."""
    monkeypatch.setenv("MOE355_HOST_ISA", isa)
    T, E, K = 11, 5, 2
    x, w1, w2, ids, w = _case(T, H, I, E, K, dt, seed=H + I)
    host = [3, 0, 4]
    ids_h = np.where(np.isin(ids, host), ids, -1)
    offs, toks, wts = _slots(ids, w, host)
    out = torch.zeros(T, H, dtype=torch.float32)
    _capi.host_experts(x, [w1[e] for e in host], [w2[e] for e in host], offs, toks, wts, act, out)
    got = out.numpy().astype(np.float64)
    exact = oracle.fused_experts(x, w1, w2, w, ids_h, activation=act)
    if dt == torch.float32:
        assert oracle.max_rel(got, exact) <= 1e-5
        return
    assert oracle.max_rel(got, exact) <= 2e-2
    rounded, allow = oracle.fused_experts_bound(x, w1, w2, w, ids_h, act, ROUND[dt])
    # the host output stays fp32: compare its bf16/f16 rounding, as the layer stores it
    stored = torch.from_numpy(got).to(dt).double().numpy()
    assert_matches_rounded(stored, rounded, allow, dt)


def test_host_expert_mixtral_shape_decode():
    """One Mixtral-8x7B expert (H=4096, I=14336, bf16) for the 5 of 8 decode
    tokens routed to it, plus a second expert for 3 of them."""
    H, I, T = 4096, 14336, 8
    g = torch.Generator().manual_seed(3)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w1 = [(torch.randn(2 * I, H, generator=g) * 0.02).to(torch.bfloat16) for _ in range(2)]
    w2 = [(torch.randn(H, I, generator=g) * 0.02).to(torch.bfloat16) for _ in range(2)]
    ids = np.array([[0, 1], [0, -1], [1, 0], [-1, -1], [0, -1], [1, -1], [0, 1], [-1, -1]])
    w = np.random.default_rng(1).random((T, 2)).astype(np.float32)
    offs, toks, wts = _slots(ids, w, [0, 1])
    out = torch.zeros(T, H, dtype=torch.float32)
    _capi.host_experts(x, w1, w2, offs, toks, wts, 0, out)
    stored = out.to(torch.bfloat16).double().numpy()
    rounded, allow = oracle.fused_experts_bound(x, w1, w2, w, ids, 0, ROUND[torch.bfloat16])
    assert oracle.max_rel(stored, oracle.fused_experts(x, w1, w2, w, ids)) <= 2e-2
    assert_matches_rounded(stored, rounded, allow, torch.bfloat16)
    assert np.all(stored[[3, 7]] == 0)


def test_host_experts_rejects_bad_arguments():
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    w1, w2 = torch.zeros(32, 64, dtype=torch.bfloat16), torch.zeros(64, 16, dtype=torch.bfloat16)
    out = torch.zeros(2, 64)
    ok = (np.array([0, 1], np.int32), np.array([1], np.int32), np.array([1.0], np.float32))
    _capi.host_experts(x, [w1], [w2], *ok, 0, out)
    with pytest.raises(_capi.MoeLibError, match="out of range"):
        _capi.host_experts(x, [w1], [w2], ok[0], np.array([2], np.int32), ok[2], 0, out)
    with pytest.raises(_capi.MoeLibError, match="activation"):
        _capi.host_experts(x, [w1], [w2], *ok, 7, out)
    with pytest.raises(ValueError):
        _capi.host_experts(x, [w1.float()], [w2], *ok, 0, out)


def test_host_library_exports_every_declared_symbol():
    lib = _capi.host_lib()
    declared = _capi.header_symbols(_capi.HOST_HEADER_PATH)
    assert set(declared) == set(_capi._HOST_SIGNATURES)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.moe355_host_version() == 102


# ------------------------------------------------------------------- int8
# The int8 host experts restate the reference's fused_experts_cpu_int8
# (reframework/moe/fused.py:140-197) step for step: integer products are
# exact and the fp32 steps are the same operations in the same order as the
# oracle's restatement (tests/test_oracle_int8.py pins that), so the library
# must match the oracle bit for bit, on every instruction-set path.


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(40, 72), (256, 130), (3, 1)])
def test_host_quantize_int8_matches_oracle(dt, shape):
    g = torch.Generator().manual_seed(shape[0] + shape[1])
    w = (torch.randn(*shape, generator=g) * 0.03).to(dt)
    q, s, rs = _capi.host_quantize_int8(w)
    oq, os_ = oracle.quantize_int8(w)
    assert s == os_
    assert np.array_equal(q.numpy(), oq)
    assert np.array_equal(rs.numpy(), oq.astype(np.int64).sum(axis=1))
    z = torch.zeros(4, 9, dtype=dt)
    qz, sz, rz = _capi.host_quantize_int8(z)
    assert sz == 1.0 and not qz.any() and not rz.any()


def _int8_bank(w1, w2):
    bank = [(_capi.host_quantize_int8(a), _capi.host_quantize_int8(b)) for a, b in zip(w1, w2)]
    return ([b[0][0] for b in bank], [b[1][0] for b in bank], [b[0][1] for b in bank],
            [b[1][1] for b in bank], [b[0][2] for b in bank], [b[1][2] for b in bank])


@pytest.mark.parametrize("isa", ["avx2", "avx512"])
@pytest.mark.parametrize("dt,H,I,act,T", [
    (torch.bfloat16, 256, 384, 0, 11), (torch.bfloat16, 200, 136, 1, 9),
    (torch.float16, 512, 256, 2, 5), (torch.float32, 192, 160, 0, 13),
    (torch.bfloat16, 64, 40, 0, 1), (torch.bfloat16, 1100, 70, 0, 19)])
def test_host_experts_int8_match_oracle_bit_exact(dt, H, I, act, T, isa, monkeypatch):
    """Random routing over 5 experts, 3 on the host, with 64/16-wide tails
    and more than 8 tokens per expert (two token passes)."""
    monkeypatch.setenv("MOE355_HOST_ISA", isa)
    E, K = 5, 2
    x, w1, w2, ids, w = _case(T, H, I, E, K, dt, seed=H + I + T)
    host = [3, 0, 4]
    offs, toks, wts = _slots(ids, w, host)
    q1, q2, s1, s2, r1, r2 = _int8_bank([w1[e] for e in host], [w2[e] for e in host])
    out = torch.zeros(T, H, dtype=torch.float32)
    _capi.host_experts_int8(x, q1, q2, s1, s2, r1, r2, offs, toks, wts, act, out)
    want = oracle.experts_int8(x, [q.numpy() for q in q1], [q.numpy() for q in q2], s1, s2,
                               offs, toks, wts, act)
    assert np.array_equal(out.numpy(), want)
    # and the int8 path stays near the exact layer (the reference's quantization error)
    ids_h = np.where(np.isin(ids, host), ids, -1)
    exact = oracle.fused_experts(x, w1, w2, w, ids_h, activation=act)
    assert oracle.max_rel(out.numpy().astype(np.float64), exact) <= 0.1


def test_host_experts_int8_mixtral_shape_decode():
    """Two Mixtral-8x7B experts (H=4096, I=14336) for 8 decode tokens, bit
    for bit the oracle's, and the reference's ~4-5 % quantization error
    against the exact layer."""
    H, I, T = 4096, 14336, 8
    g = torch.Generator().manual_seed(11)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w1 = [(torch.randn(2 * I, H, generator=g) * 0.02).to(torch.bfloat16) for _ in range(2)]
    w2 = [(torch.randn(H, I, generator=g) * 0.02).to(torch.bfloat16) for _ in range(2)]
    ids = np.array([[0, 1], [0, -1], [1, 0], [-1, -1], [0, -1], [1, -1], [0, 1], [-1, -1]])
    w = np.random.default_rng(2).random((T, 2)).astype(np.float32)
    offs, toks, wts = _slots(ids, w, [0, 1])
    q1, q2, s1, s2, r1, r2 = _int8_bank(w1, w2)
    out = torch.zeros(T, H, dtype=torch.float32)
    _capi.host_experts_int8(x, q1, q2, s1, s2, r1, r2, offs, toks, wts, 0, out)
    want = oracle.experts_int8(x, [q.numpy() for q in q1], [q.numpy() for q in q2], s1, s2,
                               offs, toks, wts, 0)
    assert np.array_equal(out.numpy(), want)
    assert np.all(out.numpy()[[3, 7]] == 0)
    err = oracle.max_rel(out.numpy().astype(np.float64), oracle.fused_experts(x, w1, w2, w, ids))
    assert 1e-3 < err < 0.1


def test_host_experts_int8_rejects_bad_arguments():
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    q1, q2 = torch.zeros(32, 64, dtype=torch.int8), torch.zeros(64, 16, dtype=torch.int8)
    r1, r2 = torch.zeros(32, dtype=torch.int32), torch.zeros(64, dtype=torch.int32)
    out = torch.zeros(2, 64)
    ok = (np.array([0, 1], np.int32), np.array([1], np.int32), np.array([1.0], np.float32))
    _capi.host_experts_int8(x, [q1], [q2], [1.0], [1.0], [r1], [r2], *ok, 0, out)
    with pytest.raises(_capi.MoeLibError, match="out of range"):
        _capi.host_experts_int8(x, [q1], [q2], [1.0], [1.0], [r1], [r2], ok[0],
                                np.array([5], np.int32), ok[2], 0, out)
    with pytest.raises(ValueError):
        _capi.host_experts_int8(x, [q1.float()], [q2], [1.0], [1.0], [r1], [r2], *ok, 0, out)
    with pytest.raises(ValueError):
        _capi.host_experts_int8(x, [q1], [q2], [1.0], [1.0], [r1[:5]], [r2], *ok, 0, out)
    # K past 65536 would overflow the int32 sums: refused by the library itself
    lib = _capi.host_lib()
    one = (ctypes.c_void_p * 1)(q1.data_ptr())
    rc = lib.moe355_host_experts_int8(x.data_ptr(), 2, 70000, 16, _capi.BF16, 1, one, one,
                                      ok[2].ctypes.data, ok[2].ctypes.data, one, one,
                                      ok[0].ctypes.data, ok[1].ctypes.data, ok[2].ctypes.data, 0,
                                      0, out.data_ptr())
    assert rc == -1 and b"65536" in lib.moe355_host_last_error()
