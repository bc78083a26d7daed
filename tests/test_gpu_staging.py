"""GPU checks of the zero-copy staging the CPU/GPU split forward uses
(moe355_copy_to_host, moe355_merge_host_f32 on moe355_host_staging_alloc
memory). Reference: the split's host transfers `.tolist()` / `.cpu()` and the
merge `out.float() + cpu_out.to(dev)` then `.to(x2.dtype)`
(reframework/moe/moe_layer.py:550-551, 597-598; fused.py:175). Bytes must
arrive exactly; the merge must equal torch's fp32 add rounded once to the
layer dtype, bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import banner
from reframework_amd import _capi

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 70, 4096, 65536 + 48, 1 << 20])
def test_copy_to_host_moves_every_byte(nbytes, dev):
    banner(f"copy_to_host {nbytes} bytes")
    stg = _capi.HostStaging(2 << 20)
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8,
                        generator=torch.Generator().manual_seed(nbytes)).to(dev)
    host = stg.array(256, np.uint8, nbytes + 32)
    host[:] = 0xA5
    _capi.copy_to_host(stg.ptr + 256, src, nbytes)
    torch.cuda.synchronize()
    assert np.array_equal(host[:nbytes], src.cpu().numpy())
    assert np.all(host[nbytes:] == 0xA5)  # nothing past the end is written


@pytest.mark.parametrize("sizes", [(8, 8, 8192), (64, 64), (16,), (0, 48, 70, 1 << 16)])
def test_copy_to_host_multi_moves_every_region(sizes, dev):
    """One kernel for up to four regions (the split's ids, weights and hidden
    states), each landing at its own 16-byte aligned offset, nothing written
    between or past them."""
    banner(f"copy_to_host_multi {sizes}")
    stg = _capi.HostStaging(2 << 20)
    g = torch.Generator().manual_seed(sum(sizes))
    srcs = [torch.randint(0, 256, (max(n, 16),), dtype=torch.uint8, generator=g).to(dev)
            for n in sizes]
    offs, o = [], 256
    for n in sizes:
        offs.append(o)
        o += (n + 64 + 15) // 16 * 16  # a 64-byte gap after each region
    host = stg.array(0, np.uint8, o + 64)
    host[:] = 0xA5
    _capi.copy_to_host_multi(stg.ptr, [(t, off, n) for t, off, n in zip(srcs, offs, sizes)])
    torch.cuda.synchronize()
    written = np.zeros(o + 64, dtype=bool)
    for t, off, n in zip(srcs, offs, sizes):
        assert np.array_equal(host[off:off + n], t[:n].cpu().numpy())
        written[off:off + n] = True
    assert np.all(host[~written] == 0xA5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_merge_host_equals_fp32_add_rounded_once(dtype, dev):
    banner(f"merge_host_f32 {dtype}")
    T, H = 8, 4096
    g = torch.Generator().manual_seed(3)
    acc = (torch.randn(T, H, generator=g) * 3).to(dev)
    stg = _capi.HostStaging(1 << 20)
    host = torch.from_numpy(stg.array(512, np.float32, T * H)).reshape(T, H)
    host.copy_(torch.randn(T, H, generator=g))
    out = torch.empty(T, H, dtype=dtype, device=dev)
    _capi.merge_host_f32(acc, stg.ptr + 512, out)
    want = (acc + host.to(dev)).to(dtype)
    torch.cuda.synchronize()
    assert torch.equal(out, want)

