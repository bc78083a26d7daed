"""reframework_amd.moe.install(): the drop-in patch rebinds the reference
package's MoE names and the same names in its submodules (which other code
imports directly: parallel/ep.py:32, integrations/litemoe_adapter.py:39,
engine/engine.py:460), and changes nothing when the MI355X path is not
available. Checked on a stand-in package with the reference's layout
(reframework/moe/__init__.py:8-18); the reference itself is not imported."""

from __future__ import annotations

import importlib
import sys
import textwrap

import pytest

import reframework_amd.moe as amd_moe
from reframework_amd.moe import fused as amd_fused

FILES = {
    "__init__.py": "",
    "moe/__init__.py": """
        from standin.moe.fused import torch_fused_topk, fused_experts
        from standin.moe.moe_layer import FusedMoE
        from standin.moe.offload_cache import ExpertOffloadCache, OffloadStats
        """,
    "moe/fused.py": """
        def torch_fused_topk(*a): return "reference"
        def fused_experts(*a): return "reference"
        def fused_experts_masked(*a): return "reference"
        def fused_experts_cpu_int8(*a): return "reference"
        """,
    "moe/moe_layer.py": """
        class FusedMoE: pass
        class CpuShuttle: pass
        """,
    "moe/offload_cache.py": """
        class ExpertOffloadCache: pass
        class OffloadStats: pass
        class Prediction: pass
        """,
    "user.py": """
        from standin.moe.fused import fused_experts
        from standin.moe import FusedMoE
        """,
}


@pytest.fixture
def standin(tmp_path, monkeypatch):
    root = tmp_path / "standin"
    for rel, text in FILES.items():
        f = root / rel
        f.parent.mkdir(parents=True, exist_ok=True)
        f.write_text(textwrap.dedent(text))
    monkeypatch.syspath_prepend(str(tmp_path))
    for name in [m for m in sys.modules if m == "standin" or m.startswith("standin.")]:
        monkeypatch.delitem(sys.modules, name)
    yield importlib.import_module("standin.moe")
    for name in [m for m in sys.modules if m == "standin" or m.startswith("standin.")]:
        sys.modules.pop(name, None)


def test_install_is_a_no_op_without_the_gpu_path(standin, monkeypatch):
    monkeypatch.setattr(amd_moe, "available", lambda: False)
    assert amd_moe.install("standin.moe") is False
    assert standin.fused_experts() == "reference"
    assert importlib.import_module("standin.moe.fused").fused_experts() == "reference"


def test_install_rebinds_package_and_submodule_names(standin, monkeypatch):
    monkeypatch.setattr(amd_moe, "available", lambda: True)
    assert amd_moe.install("standin.moe") is True
    fused = importlib.import_module("standin.moe.fused")
    layer = importlib.import_module("standin.moe.moe_layer")
    cache = importlib.import_module("standin.moe.offload_cache")
    assert standin.fused_experts is amd_fused.fused_experts
    assert standin.torch_fused_topk is amd_fused.torch_fused_topk
    assert standin.FusedMoE is amd_moe.FusedMoE
    assert standin.ExpertOffloadCache is amd_moe.ExpertOffloadCache
    assert fused.fused_experts_masked is amd_fused.fused_experts_masked
    assert fused.fused_experts_cpu_int8 is amd_fused.fused_experts_cpu_int8
    assert layer.CpuShuttle is amd_moe.CpuShuttle
    assert cache.Prediction is amd_moe.Prediction
    # the reference's own functions stay reachable, also after a second call
    assert fused._reference_fused_experts() == "reference"
    amd_moe.install("standin.moe")
    assert fused._reference_fused_experts() == "reference"
    # code imported afterwards, importing from the submodule, gets this library
    user = importlib.import_module("standin.user")
    assert user.fused_experts is amd_fused.fused_experts and user.FusedMoE is amd_moe.FusedMoE


@pytest.mark.gpu
def test_install_on_the_gpu_routes_calls_to_the_library(standin, dev):
    """With a ROCm GPU visible, install() needs no help: code that imports
    fused_experts from the patched submodule runs the library's kernels."""
    import torch
    assert amd_moe.available()
    assert amd_moe.install("standin.moe") is True
    user = importlib.import_module("standin.user")
    g = torch.Generator().manual_seed(0)
    E, K, T, H, I = 8, 2, 16, 256, 512
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    w2 = (torch.randn(E, H, I, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    w, ids = amd_fused.torch_fused_topk(torch.randn(T, E, generator=g).to(dev), K, True)
    out = user.fused_experts(x, w1, w2, w, ids)
    torch.cuda.synchronize()
    assert torch.equal(out, amd_fused.fused_experts(x, w1, w2, w, ids))
