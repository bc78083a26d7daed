"""MoE checkpoint adapter: safetensors -> FusedMoE parameters or the offload pool.

The reference loads every tensor of a checkpoint into host memory
(reframework/checkpoint/loader.py:120-127), translates PhiMoE names
(``_translate_phimoe_keys``, loader.py:83-103) and leaves Mixtral's
``block_sparse_moe.experts.{e}.w1/w3/w2`` untranslated. Here one MoE layer is
read lazily, tensor by tensor, from the ``*.safetensors`` files:

  * ``translate_key`` maps Mixtral / PhiMoE (``block_sparse_moe``, ``w1`` gate,
    ``w3`` up, ``w2`` down) and Qwen2-MoE (``shared_expert``) names onto the
    names FusedMoE uses (moe/moe_layer.py:631-660, plus
    ``shared_experts.{gate,up,down}_proj`` for shared experts). A layer with
    Qwen2-MoE's per-token ``shared_expert_gate`` is refused: FusedMoE's shared
    experts are ungated, and loading it would silently drop the gate;
  * ``load_moe_layer`` copies one layer's router, experts and shared experts
    into a FusedMoE's parameters;
  * ``load_moe_layer_offload`` copies the router (and shared experts) into the
    module but streams the routed experts straight into the pinned host pool
    of an ExpertOffloadCache, so a checkpoint larger than HBM never
    materialises per-expert parameters.

Only ``safetensors`` files are read (no pickle-based formats).
"""

from __future__ import annotations

import os
import re
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple, Union

import torch

_EXPERT_PROJ = {".w1.weight": ".gate_proj.weight", ".w3.weight": ".up_proj.weight",
                ".w2.weight": ".down_proj.weight"}


def translate_key(key: str) -> str:
    """Checkpoint tensor name -> the name FusedMoE's state dict uses."""
    k = key.replace(".block_sparse_moe.", ".mlp.")
    if k.startswith("block_sparse_moe."):
        k = "mlp." + k[len("block_sparse_moe."):]
    if ".experts." in k or k.startswith("experts."):
        for src, dst in _EXPERT_PROJ.items():
            if k.endswith(src):
                k = k[:-len(src)] + dst
                break
    k = re.sub(r"\.shared_expert\.", ".shared_experts.", k)
    return k


class SafetensorsIndex:
    """Lazy view of a checkpoint: a ``.safetensors`` file or a directory of
    them, addressed by translated tensor names."""

    def __init__(self, path: Union[str, os.PathLike]) -> None:
        from safetensors import safe_open

        path = os.fspath(path)
        if os.path.isdir(path):
            files = sorted(os.path.join(path, f) for f in os.listdir(path)
                           if f.endswith(".safetensors"))
        else:
            files = [path]
        if not files:
            raise FileNotFoundError(f"no safetensors weights found under {path}")
        self.files = files
        self._handles = {f: safe_open(f, framework="pt", device="cpu") for f in files}
        self._where: Dict[str, Tuple[str, str]] = {}
        for f, h in self._handles.items():
            for k in h.keys():
                self._where[translate_key(k)] = (f, k)

    def __contains__(self, key: str) -> bool:
        return key in self._where

    def keys(self) -> List[str]:
        return list(self._where)

    def get(self, key: str) -> torch.Tensor:
        f, k = self._where[key]
        return self._handles[f].get_tensor(k)


@dataclass
class LayerLoadReport:
    prefix: str
    loaded: List[str] = field(default_factory=list)
    missing: List[str] = field(default_factory=list)      # FusedMoE expects, checkpoint lacks
    unexpected: List[str] = field(default_factory=list)   # under the prefix, not used

    def summary(self) -> str:
        return (f"{self.prefix}: loaded {len(self.loaded)} tensors; missing={len(self.missing)} "
                f"unexpected={len(self.unexpected)}")


def _layer_keys(index: SafetensorsIndex, prefix: str) -> List[str]:
    head = prefix + "." if prefix else ""
    return [k for k in index.keys() if k.startswith(head)]


def _expert_keys(prefix: str, e: int) -> Tuple[str, str, str]:
    p = f"{prefix}.experts.{e}" if prefix else f"experts.{e}"
    return (f"{p}.gate_proj.weight", f"{p}.up_proj.weight", f"{p}.down_proj.weight")


def _reject_gated_shared_expert(index: SafetensorsIndex, prefix: str) -> None:
    """Qwen2-MoE scales its shared expert's output per token by
    sigmoid(x . shared_expert_gate); FusedMoE adds its shared experts with
    weight 1 (the ungated form of litemoe/src/litemoe/model/model.py:192-195).
    Loading such a layer would run without the gate and give wrong outputs,
    so it is refused."""
    gated = [k for k in _layer_keys(index, prefix) if ".shared_expert_gate." in k]
    if gated:
        raise ValueError(f"{prefix}: {gated[0]} gates the shared expert per token "
                         "(Qwen2-MoE); FusedMoE adds shared experts ungated and cannot "
                         "load this layer")


def load_moe_layer(index: SafetensorsIndex, moe, prefix: str) -> LayerLoadReport:
    """Copy router, routed experts and shared experts of the layer at
    ``prefix`` (e.g. ``model.layers.3.mlp``) into ``moe``'s parameters, one
    tensor at a time."""
    _reject_gated_shared_expert(index, prefix)
    rep = LayerLoadReport(prefix)
    expected = list(moe.state_dict(prefix=prefix).keys())
    for key in expected:
        if key in index:
            moe.load_state_dict({key: index.get(key)}, prefix=prefix)
            rep.loaded.append(key)
        else:
            rep.missing.append(key)
    want = set(expected)
    rep.unexpected = sorted(k for k in _layer_keys(index, prefix) if k not in want)
    return rep


def load_moe_layer_offload(index: SafetensorsIndex, moe, prefix: str, device,
                           lru_capacity: int) -> Tuple["object", LayerLoadReport]:
    """Router and shared experts into ``moe``; routed experts straight from the
    checkpoint into a new ExpertOffloadCache's host pool (``moe`` then runs
    in offload mode). Returns (cache, report)."""
    _reject_gated_shared_expert(index, prefix)
    rep = LayerLoadReport(prefix)
    dense = [k for k in moe.state_dict(prefix=prefix).keys() if ".experts." not in k]
    for key in dense:
        if key in index:
            moe.load_state_dict({key: index.get(key)}, prefix=prefix)
            rep.loaded.append(key)
        else:
            rep.missing.append(key)
    E = moe.num_experts
    for e in range(E):
        for key in _expert_keys(prefix, e):
            (rep.loaded if key in index else rep.missing).append(key)
    if any(".experts." in k for k in rep.missing):
        raise KeyError(f"{prefix}: checkpoint lacks routed-expert tensors, e.g. "
                       f"{next(k for k in rep.missing if '.experts.' in k)}")

    def fetch(e: int):
        g, u, d = _expert_keys(prefix, e)
        return index.get(g), index.get(u), index.get(d)

    cache = moe.build_offload_cache(device, lru_capacity, source=fetch)
    used = set(rep.loaded)
    rep.unexpected = sorted(k for k in _layer_keys(index, prefix) if k not in used)
    return cache, rep


__all__ = ["translate_key", "SafetensorsIndex", "LayerLoadReport", "load_moe_layer",
           "load_moe_layer_offload"]
