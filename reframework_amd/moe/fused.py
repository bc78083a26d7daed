"""Routing and grouped expert compute on libmoe355 (MI355X HIP kernels).

Same call surface as the reference's module (reframework/moe/fused.py):

  * ``torch_fused_topk(gating_output, topk, renormalize)`` -> (weights fp32
    [M,K], ids int64 [M,K]): softmax over experts, the K largest, optional
    renormalisation (fused.py:32-46).
  * ``fused_experts(hidden_states, w1, w2, topk_weights, topk_ids, activation)``
    -> [M,H] in the dtype of ``hidden_states`` (fused.py:49-87).
  * ``fused_experts_masked(..., active, activation)``: only the slots where
    ``active`` is set (the GPU half of the CPU/GPU split, fused.py:90-137).
  * ``fused_experts_cpu_int8(hidden_states, w1q, w2q, scales1, scales2,
    topk_weights, topk_ids, active, activation)`` -> fp32 [M,H] on the host:
    the split's CPU half on int8 banks (fused.py:140-197), run by
    libmoe355_host.

The reference loops over experts in Python (gather, two torch.mm, activation,
scale, index_add_). Here one C call runs the whole thing on the current HIP
stream: a stable counting sort of the routed slots, the grouped gate|up GEMM
with the activation fused, the grouped down GEMM, and a deterministic
weighted combine. Expert banks are passed as a table of per-expert device
pointers, so ``w1``/``w2`` may be a stacked ``[E,2I,H]`` tensor or a list of
per-expert tensors (the offload cache's HBM slots) without a stacking copy.
Exact ties in top-k go to the lower expert id.
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from reframework_amd import _capi
from reframework_amd.layers import activation_code

Bank = Union[torch.Tensor, Sequence[torch.Tensor]]


def require_gpu(t: torch.Tensor, what: str = "input") -> None:
    """The MoE kernels run only on a ROCm GPU; anything else is an error."""
    if t.device.type != "cuda":
        raise RuntimeError(
            f"reframework_amd MoE kernels run on a ROCm GPU; {what} is on {t.device}"
        )


def bank_pointers(bank: Bank) -> Tuple[List[int], Tuple[int, ...]]:
    """Per-expert device pointers of a stacked bank or a list of expert tensors.

    Returns (pointers, matrix shape). Every expert matrix must be contiguous.
    """
    if isinstance(bank, torch.Tensor):
        if bank.dim() != 3:
            raise ValueError(f"expected a stacked [E, rows, cols] bank, got {tuple(bank.shape)}")
        if not bank.is_contiguous():
            raise ValueError("stacked expert bank must be contiguous")
        base = bank.data_ptr()
        step = bank.stride(0) * bank.element_size()
        return [base + e * step for e in range(bank.shape[0])], tuple(bank.shape[1:])
    mats = list(bank)
    if not mats:
        raise ValueError("empty expert bank")
    shape = tuple(mats[0].shape)
    for m in mats:
        if tuple(m.shape) != shape or not m.is_contiguous():
            raise ValueError("per-expert tensors must be contiguous and share one shape")
    return [m.data_ptr() for m in mats], shape


def _bank_dtype(bank: Bank) -> torch.dtype:
    return bank.dtype if isinstance(bank, torch.Tensor) else bank[0].dtype


def torch_fused_topk(
    gating_output: torch.Tensor,
    topk: int,
    renormalize: bool,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Softmax over all experts, keep the top-k, renormalise the kept weights."""
    require_gpu(gating_output, "gating_output")
    E = gating_output.shape[-1]
    logits = gating_output.reshape(-1, E).float().contiguous()
    T = logits.shape[0]
    w = torch.empty((T, topk), dtype=torch.float32, device=logits.device)
    ids = torch.empty((T, topk), dtype=torch.int32, device=logits.device)
    _capi.topk_from_logits(logits, topk, renormalize, w, ids)
    shape = tuple(gating_output.shape[:-1]) + (topk,)
    return w.reshape(shape), ids.long().reshape(shape)


def run_experts(
    x: torch.Tensor,
    w1_ptrs: Sequence[int],
    w2_ptrs: Sequence[int],
    intermediate_size: int,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    act: int,
    out: Optional[torch.Tensor] = None,
    expert_map: Optional[Sequence[int]] = None,
    accumulate_f32: bool = False,
    path: int = -1,
) -> torch.Tensor:
    """One libmoe355 fused_experts call on the current stream.

    x [T,H] contiguous in the bank dtype; topk_weights [T,K] fp32; topk_ids
    [T,K] int32/int64; ids are local bank rows unless ``expert_map`` renames
    them. With ``accumulate_f32`` the result is added to the fp32 ``out``.
    ``path`` forces a kernel family (``_capi.PATH_*``); -1 lets the library
    choose from the shape.
    """
    T, H = x.shape
    if out is None:
        out = torch.empty((T, H), dtype=torch.float32 if accumulate_f32 else x.dtype,
                          device=x.device)
    if T == 0:
        return out
    K = topk_ids.shape[1]
    if len(w1_ptrs) < K:
        # Fewer bank rows than slots per token (a streaming chunk or a
        # truncated offload step holding fewer experts than top_k, the other
        # slots renamed to -1): the library plans for at least K experts, so
        # the tables are padded with a row no slot maps to.
        if not len(w1_ptrs):
            raise ValueError("run_experts needs at least one expert")
        w1_ptrs = list(w1_ptrs) + [w1_ptrs[-1]] * (K - len(w1_ptrs))
        w2_ptrs = list(w2_ptrs) + [w2_ptrs[-1]] * (K - len(w2_ptrs))
    stream = _capi.stream_handle(x.device)
    plan = _capi.make_plan(T, H, intermediate_size, len(w1_ptrs), topk_ids.shape[1],
                           _capi.dtype_code(x.dtype), path)
    ws = _capi.workspaces.get(x.device, stream, plan.workspace_bytes)
    _capi.fused_experts(x, w1_ptrs, w2_ptrs, intermediate_size, topk_weights, topk_ids, act, out,
                        ws, expert_map=expert_map, accumulate_f32=accumulate_f32, stream=stream,
                        plan=plan)
    return out


def fused_experts(
    hidden_states: torch.Tensor,
    w1: Bank,  # [E, 2I, H] gate|up rows (gate first), or E tensors [2I, H]
    w2: Bank,  # [E, H, I], or E tensors [H, I]
    topk_weights: torch.Tensor,  # [M, K] fp32
    topk_ids: torch.Tensor,  # [M, K] int64 (or int32)
    activation: str = "silu",
) -> torch.Tensor:
    """Run the routed experts and return the summed output ``[M, H]``."""
    act = activation_code(activation)
    require_gpu(hidden_states, "hidden_states")
    w1_ptrs, s1 = bank_pointers(w1)
    w2_ptrs, s2 = bank_pointers(w2)
    if len(w1_ptrs) != len(w2_ptrs):
        raise ValueError("w1 and w2 hold different expert counts")
    M, H = hidden_states.shape
    I = s1[0] // 2
    if s1 != (2 * I, H) or s2 != (H, I):
        raise ValueError(f"bank shapes {s1} / {s2} do not match hidden size {H}")
    dtype = _bank_dtype(w1)
    x = hidden_states.to(dtype).contiguous()
    ids = topk_ids if topk_ids.dtype in (torch.int32, torch.int64) else topk_ids.long()
    ids = ids.reshape(M, -1).contiguous()
    w = topk_weights.reshape(M, -1).float().contiguous()
    out = run_experts(x, w1_ptrs, w2_ptrs, I, w, ids, act)
    return out if out.dtype == hidden_states.dtype else out.to(hidden_states.dtype)


def fused_experts_masked(
    hidden_states: torch.Tensor,
    w1: Bank,  # [E, 2I, H], or E tensors [2I, H]: the experts this device holds
    w2: Bank,  # [E, H, I], or E tensors [H, I]
    topk_weights: torch.Tensor,  # [M, K] fp32
    topk_ids: torch.Tensor,  # [M, K], local rows of w1/w2
    active: torch.Tensor,  # [M, K] bool: the slots computed here
    activation: str = "silu",
) -> torch.Tensor:
    """fused_experts over the slots where ``active`` is set; the others add
    nothing (fused_experts_masked, reframework/moe/fused.py:90-137). The
    inactive slots are renamed to -1, which the permute drops, so the masked
    call is the same single library call. Each slot's output goes to its own
    token; the reference's ``arange(M).repeat(K)`` gives flat slot t*K+k the
    token (t*K+k) % M instead, which differs from it whenever K > 1 and a
    slot other than each token's first is active."""
    require_gpu(hidden_states, "hidden_states")
    M = hidden_states.shape[0]
    ids = topk_ids.reshape(M, -1)
    on = active.reshape(M, -1).to(device=ids.device, dtype=torch.bool)
    if on.shape != ids.shape:
        raise ValueError(f"active {tuple(active.shape)} does not match topk_ids {tuple(topk_ids.shape)}")
    ids = torch.where(on, ids, torch.full_like(ids, -1))
    return fused_experts(hidden_states, w1, w2, topk_weights, ids, activation)


def _group_active_slots(ids: np.ndarray, weights: np.ndarray, on: np.ndarray, E: int):
    """(experts used ascending, slot offsets, slot tokens, slot weights) of the
    active slots of [M, K] routing: per expert, its slots in ascending (t, k)
    order, each on its own token t."""
    K = ids.shape[1]
    flat = np.where(on, ids, -1).reshape(-1)
    chosen = flat[on.reshape(-1)]
    if chosen.size and (chosen.min() < 0 or chosen.max() >= E):
        raise ValueError(f"an active slot routes outside the {E} experts of the int8 bank")
    order = np.argsort(flat, kind="stable")
    order = order[flat[order] >= 0]
    used, counts = np.unique(flat[order], return_counts=True)
    offs = np.zeros(len(used) + 1, np.int32)
    np.cumsum(counts, out=offs[1:])
    toks = (order // K).astype(np.int32)
    sw = weights.reshape(-1)[order].astype(np.float32)
    return used, offs, toks, sw


def fused_experts_cpu_int8(
    hidden_states: torch.Tensor,  # [M, H], any device
    w1q: torch.Tensor,  # [E, 2I, H] int8 codes (symmetric, per-tensor scale)
    w2q: torch.Tensor,  # [E, H, I] int8
    scales1: torch.Tensor,  # [E] fp32
    scales2: torch.Tensor,  # [E] fp32
    topk_weights: torch.Tensor,  # [M, K] fp32
    topk_ids: torch.Tensor,  # [M, K], local rows of w1q/w2q
    active: torch.Tensor,  # [M, K] bool: the slots computed on the host
    activation: str = "silu",
    n_threads: int = 0,
) -> torch.Tensor:
    """The CPU half of the split on int8 banks (fused_experts_cpu_int8,
    reframework/moe/fused.py:140-197): an fp32 [M, H] host tensor, the sum
    over the active slots of weight * expert(x). Per expert its token rows
    (fp32) are quantized as one block, gate|up is the exact integer product
    dequantized by the two scales, act(g) * u runs in fp32, the intermediate
    is quantized the same way and the second product dequantized likewise,
    all in libmoe355_host (bit for bit the oracle's restatement of the
    reference's steps). Each slot's output goes to its own token, not the
    reference's (t*K+k) % M. Active slots must route inside the bank, where
    the reference's indexing would fail. ``n_threads`` 0 uses every OpenMP
    thread."""
    act = activation_code(activation)
    x = hidden_states.detach().to("cpu", torch.float32).contiguous()
    M, H = x.shape
    out = torch.zeros((M, H), dtype=torch.float32)
    if w1q.dim() != 3 or w2q.dim() != 3 or w1q.dtype != torch.int8 or w2q.dtype != torch.int8:
        raise ValueError("w1q / w2q must be int8 [E, 2I, H] / [E, H, I] banks")
    E, I = w1q.shape[0], w2q.shape[2]
    if tuple(w1q.shape) != (E, 2 * I, H) or tuple(w2q.shape) != (E, H, I):
        raise ValueError(f"int8 bank shapes {tuple(w1q.shape)} / {tuple(w2q.shape)} do not "
                         f"match hidden size {H}")
    ids = topk_ids.detach().cpu().long().reshape(M, -1).numpy()
    K = ids.shape[1]
    wts = topk_weights.detach().cpu().float().reshape(M, K).numpy()
    on = active.detach().cpu().reshape(M, K).numpy().astype(bool)
    used, offs, toks, sw = _group_active_slots(ids, wts, on, E)
    if not len(used):
        return out
    q1, q2 = w1q.detach().cpu().contiguous(), w2q.detach().cpu().contiguous()
    b1 = [q1[int(e)] for e in used]
    b2 = [q2[int(e)] for e in used]
    s1 = scales1.detach().cpu().float().reshape(-1)
    s2 = scales2.detach().cpu().float().reshape(-1)
    _capi.host_experts_int8(x, b1, b2, [float(s1[int(e)]) for e in used],
                            [float(s2[int(e)]) for e in used],
                            [_capi.host_int8_row_sums(b, n_threads) for b in b1],
                            [_capi.host_int8_row_sums(b, n_threads) for b in b2],
                            offs, toks, sw, act, out, n_threads)
    return out


__all__ = ["torch_fused_topk", "fused_experts", "fused_experts_masked", "fused_experts_cpu_int8",
           "run_experts", "bank_pointers", "require_gpu"]
