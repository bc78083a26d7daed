"""FusedMoE host-side contract on the CPU (no kernels run): constructor,
``from_config``, HF-named state dict including shared experts.

Reference: FusedMoE (reframework/moe/moe_layer.py:135-169, 196-225, 631-660).
Shared experts are not in the reference; their names and semantics follow
litemoe (litemoe/src/litemoe/model/model.py:100-137, 192-195) and the HF
``mlp.shared_experts.{gate,up,down}_proj`` layout.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from reframework_amd import synth
from reframework_amd.moe import FusedMoE


def test_parameters_and_state_dict_names_match_reference():
    moe = FusedMoE(4, 2, 32, 16, dtype=torch.float32)
    assert tuple(moe.gate.shape) == (4, 32)
    assert all(tuple(p.shape) == (32, 32) for p in moe.experts_w1)
    assert all(tuple(p.shape) == (32, 16) for p in moe.experts_w2)
    sd = moe.state_dict(prefix="model.layers.0.mlp")
    assert "model.layers.0.mlp.gate.weight" in sd
    for e in range(4):
        for n in ("gate_proj", "up_proj", "down_proj"):
            assert f"model.layers.0.mlp.experts.{e}.{n}.weight" in sd
    assert not any("shared" in k for k in sd)


@pytest.mark.parametrize("n_shared,shared_I,pieces,piece", [(2, None, 2, 16), (0, 40, 1, 40),
                                                             (1, 32, 2, 16)])
def test_shared_expert_state_dict_round_trip(n_shared, shared_I, pieces, piece):
    H, I = 32, 16
    moe = FusedMoE(4, 2, H, I, dtype=torch.float32, n_shared_experts=n_shared,
                   shared_intermediate_size=shared_I)
    Is = shared_I or n_shared * I
    assert moe.shared_intermediate_size == Is
    assert len(moe.shared_w1) == pieces and moe._shared_piece == piece
    assert moe._shared_folded == (piece == I)
    g = torch.Generator().manual_seed(0)
    sd = {"mlp.shared_experts.gate_proj.weight": torch.randn(Is, H, generator=g),
          "mlp.shared_experts.up_proj.weight": torch.randn(Is, H, generator=g),
          "mlp.shared_experts.down_proj.weight": torch.randn(H, Is, generator=g)}
    moe.load_state_dict(sd, prefix="mlp")
    # piece j holds gate rows j*P.., then the matching up rows; down columns j*P..
    for j in range(pieces):
        rows = slice(j * piece, (j + 1) * piece)
        assert torch.equal(moe.shared_w1[j][:piece], sd["mlp.shared_experts.gate_proj.weight"][rows])
        assert torch.equal(moe.shared_w1[j][piece:], sd["mlp.shared_experts.up_proj.weight"][rows])
        assert torch.equal(moe.shared_w2[j], sd["mlp.shared_experts.down_proj.weight"][:, rows])
    back = moe.state_dict(prefix="mlp")
    for k, v in sd.items():
        assert torch.equal(back[k], v), k


def test_from_config_reads_reference_fields_and_optional_shared():
    cfg = SimpleNamespace(num_experts=8, num_experts_per_tok=2, hidden_size=64, moe_inter=32,
                          moe_activation="silu", moe_renormalize=True, dtype=torch.bfloat16)
    moe = FusedMoE.from_config(cfg)
    assert (moe.num_experts, moe.top_k, moe.hidden_size, moe.intermediate_size) == (8, 2, 64, 32)
    assert moe.dtype == torch.bfloat16 and len(moe.shared_w1) == 0
    cfg.n_shared_experts = 2
    moe = FusedMoE.from_config(cfg, dtype=torch.float16)
    assert moe.dtype == torch.float16 and len(moe.shared_w1) == 2


def test_synth_shared_pieces_match_merged_tensors():
    sh = synth.make_shared(2, 16, 8, torch.float32)
    assert tuple(sh["gate_proj"].shape) == (16, 16) and tuple(sh["down_proj"].shape) == (16, 16)
    assert torch.equal(sh["gate_proj"][8:], sh["w1"][1][:8])
    assert torch.equal(sh["up_proj"][:8], sh["w1"][0][8:])
    assert torch.equal(sh["down_proj"][:, 8:], sh["w2"][1])


def test_available_is_false_without_a_gpu_or_library(monkeypatch):
    """The drop-in import keeps the reference's modules where the MI355X path
    cannot run: no visible GPU (this host), or a library that fails to load."""
    import torch

    from reframework_amd import _capi, moe

    if not torch.cuda.is_available():
        assert moe.available() is False
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(_capi, "LIB_PATH", "/nonexistent/libmoe355.so")
    monkeypatch.setattr(_capi, "_lib", None)
    assert moe.available() is False


def test_offload_cache_host_from_shares_the_pool():
    a = FusedMoE(4, 2, 32, 16, dtype=torch.float32)
    with torch.no_grad():
        for e, p in enumerate(a.experts_w1):
            p.fill_(float(e))
    ca = a.build_offload_cache(torch.device("cpu"), lru_capacity=2)
    b = FusedMoE(4, 2, 32, 16, dtype=torch.float32)
    cb = b.build_offload_cache(torch.device("cpu"), lru_capacity=2, host_from=ca)
    assert cb is not ca and cb._host_buf is ca._host_buf and len(b.experts_w1) == 0
    w1, _, idx = cb.prefetch([3])
    assert torch.all(w1[idx[3]] == 3.0) and set(ca._lru) == set()
    other = FusedMoE(4, 2, 32, 24, dtype=torch.float32)
    with pytest.raises(ValueError):
        other.build_offload_cache(torch.device("cpu"), lru_capacity=2, host_from=ca)
