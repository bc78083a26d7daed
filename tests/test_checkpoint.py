"""Checkpoint adapter on the CPU: key translation, lazy per-layer loading into
FusedMoE parameters, and streaming routed experts into an offload pool.

Reference: reframework/checkpoint/loader.py:83-103 (PhiMoE translation; the
reference leaves Mixtral's names untranslated), :120-127 (load_weights), and
the HF names FusedMoE consumes (reframework/moe/moe_layer.py:631-660).
Checkpoints here are small synthetic safetensors files.
"""

from __future__ import annotations

import pytest
import torch
from safetensors.torch import save_file

from reframework_amd.checkpoint import (SafetensorsIndex, load_moe_layer, load_moe_layer_offload,
                                        translate_key)
from reframework_amd.moe import FusedMoE


@pytest.mark.parametrize("src,dst", [
    ("model.layers.3.block_sparse_moe.gate.weight", "model.layers.3.mlp.gate.weight"),
    ("model.layers.3.block_sparse_moe.experts.7.w1.weight",
     "model.layers.3.mlp.experts.7.gate_proj.weight"),
    ("model.layers.3.block_sparse_moe.experts.7.w3.weight",
     "model.layers.3.mlp.experts.7.up_proj.weight"),
    ("model.layers.3.block_sparse_moe.experts.7.w2.weight",
     "model.layers.3.mlp.experts.7.down_proj.weight"),
    ("model.layers.0.mlp.experts.1.down_proj.weight", "model.layers.0.mlp.experts.1.down_proj.weight"),
    ("model.layers.0.mlp.shared_expert.up_proj.weight",
     "model.layers.0.mlp.shared_experts.up_proj.weight"),
    ("model.layers.0.mlp.shared_experts.up_proj.weight",
     "model.layers.0.mlp.shared_experts.up_proj.weight"),
    ("model.layers.0.self_attn.q_proj.weight", "model.layers.0.self_attn.q_proj.weight"),
    ("model.layers.0.mlp.w1.weight", "model.layers.0.mlp.w1.weight"),  # dense MLP: untouched
])
def test_translate_key(src, dst):
    assert translate_key(src) == dst


def _mixtral_ckpt(tmp_path, L=2, E=4, H=16, I=8, dtype=torch.float32, shards=2, stored=None):
    g = torch.Generator().manual_seed(0)
    sd = {}
    for layer in range(L):
        p = f"model.layers.{layer}.block_sparse_moe"
        sd[f"{p}.gate.weight"] = torch.randn(E, H, generator=g).to(dtype)
        for e in range(E if stored is None else stored):
            sd[f"{p}.experts.{e}.w1.weight"] = torch.randn(I, H, generator=g).to(dtype)
            sd[f"{p}.experts.{e}.w3.weight"] = torch.randn(I, H, generator=g).to(dtype)
            sd[f"{p}.experts.{e}.w2.weight"] = torch.randn(H, I, generator=g).to(dtype)
        sd[f"model.layers.{layer}.input_layernorm.weight"] = torch.ones(H).to(dtype)
    keys = sorted(sd)
    for s in range(shards):
        part = {k: sd[k].contiguous() for k in keys[s::shards]}
        save_file(part, str(tmp_path / f"model-{s:05d}-of-{shards:05d}.safetensors"))
    return sd


def test_mixtral_layer_loads_lazily_into_fused_moe(tmp_path):
    sd = _mixtral_ckpt(tmp_path)
    idx = SafetensorsIndex(tmp_path)
    assert len(idx.files) == 2
    moe = FusedMoE(4, 2, 16, 8, dtype=torch.float32)
    rep = load_moe_layer(idx, moe, "model.layers.1.mlp")
    assert not rep.missing and not rep.unexpected and len(rep.loaded) == 1 + 3 * 4
    src = "model.layers.1.block_sparse_moe"
    assert torch.equal(moe.gate, sd[f"{src}.gate.weight"])
    for e in range(4):
        assert torch.equal(moe.experts_w1[e][:8], sd[f"{src}.experts.{e}.w1.weight"])
        assert torch.equal(moe.experts_w1[e][8:], sd[f"{src}.experts.{e}.w3.weight"])
        assert torch.equal(moe.experts_w2[e], sd[f"{src}.experts.{e}.w2.weight"])


def test_bf16_checkpoint_into_bf16_layer_and_missing_report(tmp_path):
    sd = _mixtral_ckpt(tmp_path, L=1, E=5, dtype=torch.bfloat16, shards=1, stored=4)
    idx = SafetensorsIndex(next(tmp_path.glob("*.safetensors")))
    moe = FusedMoE(5, 2, 16, 8, dtype=torch.bfloat16)  # the checkpoint lacks expert 4
    rep = load_moe_layer(idx, moe, "model.layers.0.mlp")
    assert len(rep.missing) == 3 and all(".experts.4." in k for k in rep.missing)
    assert torch.equal(moe.experts_w2[3], sd["model.layers.0.block_sparse_moe.experts.3.w2.weight"])


@pytest.mark.parametrize("name", ["shared_experts", "shared_expert"])
def test_shared_experts_from_deepseek_and_qwen_names(tmp_path, name):
    H, I, E = 16, 8, 4
    g = torch.Generator().manual_seed(1)
    p = "model.layers.0.mlp"
    sd = {f"{p}.gate.weight": torch.randn(E, H, generator=g)}
    for e in range(E):
        for n, shp in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            sd[f"{p}.experts.{e}.{n}.weight"] = torch.randn(*shp, generator=g)
    for n, shp in (("gate_proj", (2 * I, H)), ("up_proj", (2 * I, H)), ("down_proj", (H, 2 * I))):
        sd[f"{p}.{name}.{n}.weight"] = torch.randn(*shp, generator=g)
    save_file(sd, str(tmp_path / "m.safetensors"))
    moe = FusedMoE(E, 2, H, I, dtype=torch.float32, n_shared_experts=2)
    rep = load_moe_layer(SafetensorsIndex(tmp_path), moe, p)
    assert not rep.missing and not rep.unexpected
    back = moe.state_dict(prefix=p)
    for n in ("gate_proj", "up_proj", "down_proj"):
        assert torch.equal(back[f"{p}.shared_experts.{n}.weight"], sd[f"{p}.{name}.{n}.weight"])


def test_offload_load_streams_experts_into_host_pool(tmp_path):
    sd = _mixtral_ckpt(tmp_path, dtype=torch.bfloat16)
    idx = SafetensorsIndex(tmp_path)
    moe = FusedMoE(4, 2, 16, 8, dtype=torch.bfloat16)
    cache, rep = load_moe_layer_offload(idx, moe, "model.layers.0.mlp", "cpu", lru_capacity=2)
    assert not rep.missing and not rep.unexpected
    assert moe.uses_offload and len(moe.experts_w1) == 0 and cache.num_experts == 4
    src = "model.layers.0.block_sparse_moe"
    assert torch.equal(moe.gate, sd[f"{src}.gate.weight"])
    for e in range(4):
        w1, w2 = cache._host[e]
        assert torch.equal(w1[:8], sd[f"{src}.experts.{e}.w1.weight"])
        assert torch.equal(w1[8:], sd[f"{src}.experts.{e}.w3.weight"])
        assert torch.equal(w2, sd[f"{src}.experts.{e}.w2.weight"])


def test_offload_load_requires_every_routed_expert(tmp_path):
    _mixtral_ckpt(tmp_path, L=1, E=6, shards=1, stored=4)
    moe = FusedMoE(6, 2, 16, 8, dtype=torch.float32)
    with pytest.raises(KeyError, match="experts.4"):
        load_moe_layer_offload(SafetensorsIndex(tmp_path), moe, "model.layers.0.mlp", "cpu", 2)


def test_missing_checkpoint_is_an_error(tmp_path):
    with pytest.raises(FileNotFoundError):
        SafetensorsIndex(tmp_path)


@pytest.mark.parametrize("offload", [False, True])
def test_qwen2_moe_shared_expert_gate_is_refused(tmp_path, offload):
    """Qwen2-MoE gates its shared expert per token (sigmoid(x . g)); the
    layer's shared experts are ungated, so such a checkpoint must not load
    into it silently."""
    H, I, E = 16, 8, 4
    g = torch.Generator().manual_seed(2)
    p = "model.layers.0.mlp"
    sd = {f"{p}.gate.weight": torch.randn(E, H, generator=g),
          f"{p}.shared_expert_gate.weight": torch.randn(1, H, generator=g)}
    for e in range(E):
        for n, shp in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            sd[f"{p}.experts.{e}.{n}.weight"] = torch.randn(*shp, generator=g)
    for n, shp in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
        sd[f"{p}.shared_expert.{n}.weight"] = torch.randn(*shp, generator=g)
    save_file(sd, str(tmp_path / "m.safetensors"))
    moe = FusedMoE(E, 2, H, I, dtype=torch.float32, n_shared_experts=1)
    with pytest.raises(ValueError, match="shared_expert_gate"):
        if offload:
            load_moe_layer_offload(SafetensorsIndex(tmp_path), moe, p, "cpu", 2)
        else:
            load_moe_layer(SafetensorsIndex(tmp_path), moe, p)
