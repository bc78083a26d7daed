"""The RMSNorm oracle against library routines and closed forms (CPU).

Reference: RMSNorm._forward / forward_add_residual
(reframework/layers/norm.py:27-53): residual = x + residual in the storage
dtype; normed = residual / sqrt(mean(residual^2) + eps) * w (+ b) in fp32,
rounded once.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle
from reframework_amd import _capi


def test_matches_torch_rms_norm_in_float64():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(9, 96, generator=g)
    w = torch.randn(96, generator=g)
    _, normed = oracle.add_rmsnorm(x, None, w, None, 1e-5)
    want = F.rms_norm(x.double(), (96,), w.double(), 1e-5).float().double().numpy()
    assert np.array_equal(normed, want)


def test_residual_add_rounds_like_torch_bf16_add_and_bias_is_added_last():
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(5, 64, generator=g) * 3).to(torch.bfloat16)
    r = (torch.randn(5, 64, generator=g) * 1e-2).to(torch.bfloat16)
    w = torch.rand(64, generator=g) + 0.5
    b = torch.randn(64, generator=g)
    new_r, normed = oracle.add_rmsnorm(x, r, w, b, 1e-6)
    s = x + r  # the reference's add: bf16 tensors
    assert np.array_equal(new_r, s.double().numpy())
    want = (F.rms_norm(s.double(), (64,), w.double(), 1e-6) + b.double()).to(torch.bfloat16)
    got = torch.from_numpy(normed)
    # one rounding of nearly the same fp64 value: equal, or one bf16 step apart
    diff = (got - want.double()).abs()
    ulp = want.double().abs() * 2.0 ** -7 + 1e-30
    assert bool((diff <= ulp).all())


def test_constant_rows_and_eps():
    x = torch.full((2, 8), 2.0)
    x[1] = -0.5
    _, normed = oracle.add_rmsnorm(x, None, torch.ones(8), None, 0.0)
    assert np.allclose(normed[0], 1.0) and np.allclose(normed[1], -1.0)
    eps = 0.75
    _, normed = oracle.add_rmsnorm(x, None, torch.ones(8), None, eps)
    assert np.allclose(normed[1], np.float32(-0.5 / np.sqrt(0.25 + eps)))


def test_scale_invariance_without_eps():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(4, 32, generator=g)
    _, a = oracle.add_rmsnorm(x, None, torch.ones(32), None, 0.0)
    _, b = oracle.add_rmsnorm(x * 8.0, None, torch.ones(32), None, 0.0)
    assert np.array_equal(a, b)  # power-of-two scaling is exact


@pytest.mark.parametrize("args,code,msg", [
    ((4, 100, _capi.BF16), -2, "norm needs"),
    ((4, 8 * 256 * 8 * 2, _capi.BF16), -2, "norm needs"),
    ((-1, 64, _capi.BF16), -1, "bad sizes"),
])
def test_norm_entry_rejects_bad_shapes(args, code, msg):
    T, H, dt = args
    lib = _capi.lib()
    rc = lib.moe355_add_rmsnorm(None, None, None, None, None, _capi.F32, ctypes.c_float(1e-6), T, H,
                                dt, None, None)
    assert rc == code and msg in lib.moe355_last_error().decode()


def test_norm_entry_rejects_null_and_missing_residual_out():
    lib = _capi.lib()
    assert lib.moe355_add_rmsnorm(None, None, None, None, None, _capi.F32, ctypes.c_float(1e-6), 0,
                                  64, _capi.BF16, None, None) == 0
    assert lib.moe355_add_rmsnorm(None, None, None, None, None, _capi.F32, ctypes.c_float(1e-6), 2,
                                  64, _capi.BF16, None, None) == -1
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) & ~15
    assert lib.moe355_add_rmsnorm(p, p, None, p, None, _capi.F32, ctypes.c_float(1e-6), 2, 64,
                                  _capi.BF16, p, None) == -1
    assert "residual_out" in lib.moe355_last_error().decode()
