"""FusedMoE: the routed MoE block on libmoe355 (MI355X HIP kernels).

Drop-in for the reference's ``FusedMoE`` (reframework/moe/moe_layer.py:132-
660): same constructor, ``from_config`` fields, parameters (``gate [E,H]``,
``experts_w1[e] [2I,H]`` gate rows first, ``experts_w2[e] [H,I]``), HF-named
state dict, offload wiring (``build_offload_cache``, ``attach_predictor``,
``enable_cpu_split``, ``set_shuttle``) and forward semantics:

  * resident forward: route, then all routed experts (moe_layer.py:443-447,
    513). The reference stacks every expert into fresh ``[E,2I,H]``/``[E,H,I]``
    banks on each call; here the kernels read the parameters in place through
    a pointer table.
  * offload forward (``RE_CHUNK_SIZE`` unset or 0): experts ranked by summed
    routing weight, the first ``RE_MAX_PACK`` (default 2) kept and prefetched,
    the other slots dropped (weight 0), the routed set recorded for the
    lookahead, then the experts run (moe_layer.py:426-442, 477-513).
  * streaming offload (``RE_CHUNK_SIZE`` > 0): every routed expert, in chunks
    of that many experts, accumulated in fp32 (moe_layer.py:354-420). Chunk
    i+1's host->HBM copies are queued on the device's copy stream while chunk
    i's kernels run.
  * CPU/GPU split (``enable_cpu_split``, moe_layer.py:523-627): the experts
    the offload forward would run (``RE_MAX_PACK`` truncation, or every routed
    expert with ``RE_CHUNK_SIZE`` > 0) are split by residency. Resident ones
    run on the GPU into an fp32 accumulator while the host cores compute the
    others from the staged pool (libmoe355_host, 16-bit weights, the device
    kernels' numerics); the host half is added in fp32 and the sum cast once.
    Then, while fewer than ``RE_MOE_SPLIT_COPY_DEPTH`` copies are in flight,
    the host-computed experts are copied to device memory for later steps.

Optional shared experts (``n_shared_experts``; not in the reference, which
has none): the dense SwiGLU that fine-grained MoEs add to every token after
the routed sum, ``out += down(silu(x gate^T) * (x up^T))`` (the semantics of
litemoe/src/litemoe/model/model.py:192-195), stored under the HF names
``shared_experts.{gate,up,down}_proj.weight`` with width
``shared_intermediate_size`` (default ``n_shared_experts * intermediate_size``).
When that width is a multiple of ``intermediate_size`` it is kept as that many
expert-sized pieces and folded into the routed call as extra experts that
every token reaches with weight 1; otherwise it runs as a second call into the
same fp32 accumulator.

All device compute is in libmoe355: the router kernel (GEMV + softmax +
top-k) and one fused_experts call per forward (or per chunk). A CPU tensor is
an error, not a slower path; host compute happens only in the split forward,
which a caller turns on explicitly.
"""

from __future__ import annotations

import logging
import time
from collections import deque
from typing import Deque, Dict, List, Optional, Tuple

import numpy as np
import torch

from reframework_amd import _capi, env
from reframework_amd.layers import BaseOP, activation_code
from reframework_amd.moe.fused import require_gpu, run_experts
from reframework_amd.moe.offload_cache import ExpertOffloadCache, Prediction

logger = logging.getLogger(__name__)


class CpuShuttle:
    """Byte-accounting stand-in for a device-to-device token shuttle.

    ``send`` ages every in-flight transfer by one step and appends the new one;
    each transfer decays by ``bytes / n_steps`` per step, so it is visible to
    ``inflight_bytes`` for exactly ``n_steps`` reads (reference:
    moe_layer.py:58-129). No data moves: ``send`` returns a clone.
    """

    def __init__(self, n_steps: int = 2) -> None:
        self.n_steps = max(1, int(n_steps))
        self._transfers: Deque[Tuple[float, float]] = deque()

    def send(self, hidden: torch.Tensor, to: str = "") -> torch.Tensor:
        self.advance_step()
        if hidden is not None and hidden.numel() > 0:
            nbytes = float(hidden.numel() * hidden.element_size())
            self._transfers.append((nbytes, nbytes / self.n_steps))
        return hidden.clone() if hidden is not None else hidden

    def advance_step(self) -> None:
        self._transfers = deque((r - per, per) for r, per in self._transfers if r - per > 0.0)

    def inflight_bytes(self) -> float:
        return float(sum(r for r, _ in self._transfers))

    def sync(self) -> None:
        self._transfers.clear()


class FusedMoE(BaseOP):
    """A routed MoE block: ``gate`` -> top-k -> grouped SwiGLU experts."""

    def __init__(
        self,
        num_experts: int,
        top_k: int,
        hidden_size: int,
        intermediate_size: int,
        activation: str = "silu",
        renormalize: bool = True,
        dtype: torch.dtype = torch.float16,
        n_shared_experts: int = 0,
        shared_intermediate_size: Optional[int] = None,
    ) -> None:
        super().__init__()
        self.num_experts = num_experts
        self.top_k = top_k
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.activation = activation
        self.renormalize = renormalize
        self.dtype = dtype
        self.gate = torch.nn.Parameter(torch.empty(num_experts, hidden_size, dtype=dtype))
        self.experts_w1 = torch.nn.ParameterList([
            torch.nn.Parameter(torch.empty(2 * intermediate_size, hidden_size, dtype=dtype))
            for _ in range(num_experts)
        ])
        self.experts_w2 = torch.nn.ParameterList([
            torch.nn.Parameter(torch.empty(hidden_size, intermediate_size, dtype=dtype))
            for _ in range(num_experts)
        ])
        # Shared experts: width Is split into pieces of ``intermediate_size``
        # when it divides evenly (folded into the routed call), else one piece.
        shared_I = int(shared_intermediate_size or n_shared_experts * intermediate_size)
        if shared_I < 0:
            raise ValueError("shared_intermediate_size must be >= 0")
        self.n_shared_experts = int(n_shared_experts)
        self.shared_intermediate_size = shared_I
        if shared_I and shared_I % intermediate_size == 0:
            piece, n_pieces = intermediate_size, shared_I // intermediate_size
        else:
            piece, n_pieces = shared_I, (1 if shared_I else 0)
        self._shared_piece = piece
        self.shared_w1 = torch.nn.ParameterList([
            torch.nn.Parameter(torch.empty(2 * piece, hidden_size, dtype=dtype))
            for _ in range(n_pieces)
        ])
        self.shared_w2 = torch.nn.ParameterList([
            torch.nn.Parameter(torch.empty(hidden_size, piece, dtype=dtype))
            for _ in range(n_pieces)
        ])
        self._checked_tables: set = set()
        self._shared_cols = None  # cached (key, weights [T,K+n], ids [T,K+n]); see _route32
        self._logits = None  # cached (key, fp32 [T,E] router logits buffer); see _logits_buffer
        self._cache: Optional[ExpertOffloadCache] = None
        self._cpu_split_enabled: bool = False
        self._predictor: Optional[Prediction] = None
        self._shuttle: Optional[CpuShuttle] = None
        self._last_step_t: Optional[float] = None
        self.entropy_adaptive_k: bool = False
        self.entropy_k_min: int = 2

    # --------------------------------------------------------------- factories
    @classmethod
    def from_config(cls, cfg, dtype: Optional[torch.dtype] = None) -> "FusedMoE":
        """Build from a model config with the reference's MoE fields
        (num_experts, num_experts_per_tok, hidden_size, moe_inter,
        moe_activation, moe_renormalize, dtype; optional entropy_adaptive_k,
        entropy_k_min), honouring RE_ENTROPY_K / RE_ENTROPY_K_MIN. Optional
        ``n_shared_experts`` / ``shared_intermediate_size`` add shared experts."""
        moe = cls(
            num_experts=cfg.num_experts,
            top_k=cfg.num_experts_per_tok,
            hidden_size=cfg.hidden_size,
            intermediate_size=cfg.moe_inter,
            activation=cfg.moe_activation,
            renormalize=cfg.moe_renormalize,
            dtype=dtype or cfg.dtype,
            n_shared_experts=int(getattr(cfg, "n_shared_experts", 0) or 0),
            shared_intermediate_size=getattr(cfg, "shared_intermediate_size", None),
        )
        moe.entropy_adaptive_k = bool(getattr(cfg, "entropy_adaptive_k", False)) or env.get_entropy_k()
        moe.entropy_k_min = env.get_entropy_k_min(getattr(cfg, "entropy_k_min", 2))
        logger.info("[entropy] adaptive_k=%s k_min=%d top_k=%d num_experts=%d",
                    moe.entropy_adaptive_k, moe.entropy_k_min, moe.top_k, moe.num_experts)
        return moe

    # ----------------------------------------------------------- offload setup
    def build_offload_cache(self, device: torch.device, lru_capacity: int,
                            source=None, pool=None,
                            host_from: Optional[ExpertOffloadCache] = None) -> ExpertOffloadCache:
        """Stage this layer's experts into a pinned-host cache on ``device``
        and drop the per-expert parameters. ``source(e) -> (gate [I,H], up
        [I,H], down [H,I])``, when given, supplies the experts instead of the
        parameters (e.g. straight from a checkpoint). ``pool`` (an
        ExpertPool) shares one HBM slot pool and LRU with other layers
        instead of a per-layer window of ``lru_capacity`` experts.
        ``host_from`` (another layer's cache with the same expert shapes)
        lends its staged host pool instead: this layer's experts are then
        that layer's weights."""
        self._cache = ExpertOffloadCache(device=device, lru_capacity=lru_capacity, dtype=self.dtype,
                                         pool=pool)
        if host_from is not None:
            w1_shape = (2 * self.intermediate_size, self.hidden_size)
            if host_from.num_experts != self.num_experts or \
                    tuple(host_from._host[0][0].shape) != w1_shape:
                raise ValueError("host_from holds experts of another count or shape")
            self._cache.share_host(host_from)
        elif source is None:
            self._cache.load([{"w1": self.experts_w1[e], "w2": self.experts_w2[e]}
                              for e in range(self.num_experts)])
        else:
            self._cache.load_from(self.num_experts, self.hidden_size, self.intermediate_size,
                                  source)
        self.experts_w1 = torch.nn.ParameterList()
        self.experts_w2 = torch.nn.ParameterList()
        if torch.cuda.is_available():
            torch.cuda.empty_cache()
        return self._cache

    def attach_predictor(self, window: int = 32) -> None:
        if self._cache is None:
            return
        self._cache.attach_predictor(window=window)
        self._predictor = self._cache._predictor

    def enable_cpu_split(self, int8: Optional[bool] = None) -> None:
        """Turn on the CPU/GPU split forward for this offloaded layer
        (reference: moe_layer.py:263-282, 523-627): experts not resident in
        device memory are computed on the host cores while the GPU runs the
        resident ones. The host half multiplies the staged 16-bit weights
        with the device kernels' numerics, or, with ``int8`` (default:
        RE_MOE_SPLIT_INT8), the reference's per-tensor int8 bank with its
        int8 numerics (quantize_int8_host + fused_experts_cpu_int8), half
        the host bytes per expert. No-op for a layer without an offload
        cache."""
        if self._cache is None:
            return
        self._cache.enable_host_experts(int8=env.get_moe_split_int8() if int8 is None else int8)
        self._cpu_split_enabled = True

    def set_shuttle(self, shuttle: Optional[CpuShuttle]) -> None:
        self._shuttle = shuttle

    @property
    def cpu_split(self) -> bool:
        return self._cpu_split_enabled and self.uses_offload and self._cache.cpu_split

    @property
    def uses_offload(self) -> bool:
        return self._cache is not None

    def _since_last_step_ms(self) -> float:
        """Milliseconds since this layer's previous forward; 0.0 on the first."""
        t = time.perf_counter()
        prev, self._last_step_t = self._last_step_t, t
        return 0.0 if prev is None else max(0.0, (t - prev) * 1000.0)

    # ----------------------------------------------------------------- routing
    def _route32(self, xd: torch.Tensor,
                 with_shared_cols: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
        """Router kernel on ``xd`` ([T,H], model dtype, contiguous, on GPU):
        (weights fp32 [T,K], ids int32 [T,K]). With ``with_shared_cols`` (the
        shared experts folded in as extra experts) the router writes into
        [T, K+n] buffers whose last n columns already hold the shared ids E..
        with weight 1, so no concatenation follows; the buffers are cached per
        token count and stream, and reused by the next forward on that stream."""
        gate = self.gate.detach()
        if gate.device != xd.device:
            gate = gate.to(xd.device)
        gate = gate.to(self.dtype).contiguous()
        T = xd.shape[0]
        if with_shared_cols:
            n = len(self.shared_w1)
            # one pair per stream: forwards on different streams must not share
            key = (T, n, xd.device, _capi.stream_handle(xd.device))
            if self._shared_cols is None or self._shared_cols[0] != key:
                ids = torch.empty((T, self.top_k + n), dtype=torch.int32, device=xd.device)
                ids[:, self.top_k:] = torch.arange(self.num_experts, self.num_experts + n,
                                                   dtype=torch.int32, device=xd.device)
                w = torch.ones((T, self.top_k + n), dtype=torch.float32, device=xd.device)
                self._shared_cols = (key, w, ids)
            _, w, ids = self._shared_cols
        else:
            w = torch.empty((T, self.top_k), dtype=torch.float32, device=xd.device)
            ids = torch.empty((T, self.top_k), dtype=torch.int32, device=xd.device)
        kmin = 0
        if self.entropy_adaptive_k:
            if self.entropy_k_min < 1:
                raise ValueError("entropy-adaptive routing needs entropy_k_min >= 1")
            kmin = min(int(self.entropy_k_min), self.top_k)
        _capi.router_topk(xd, gate, None, self.top_k, self.renormalize, True, kmin, w, ids,
                          logits_out=self._logits_buffer(T, xd.device))
        return w, ids

    def _logits_buffer(self, T: int, device: torch.device) -> torch.Tensor:
        """fp32 [T, E] logits buffer. It lets the router spread few tokens
        over many experts across workgroups (it writes the logits there, then
        selects); one per token count and stream, reused by the next forward
        on that stream."""
        lkey = (T, device, _capi.stream_handle(device))
        if self._logits is None or self._logits[0] != lkey:
            self._logits = (lkey, torch.empty((T, self.num_experts), dtype=torch.float32,
                                              device=device))
        return self._logits[1]

    def route(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Return (topk_weights [M,K] fp32, topk_ids [M,K] int64) for ``x``."""
        x2 = x.reshape(-1, self.hidden_size)
        require_gpu(x2)
        w, ids = self._route32(x2.to(self.dtype).contiguous())
        return w, ids.long()

    def prefetch_ids(self, x: torch.Tensor) -> torch.Tensor:
        _, ids = self.route(x)
        return ids

    # ----------------------------------------------------------------- forward
    def _resident_banks(self) -> Tuple[List[int], List[int]]:
        if len(self.experts_w1) != self.num_experts:
            raise RuntimeError("expert parameters are not resident (offload cache built?)")
        return self._pointers(self.experts_w1, self.experts_w2)

    def _pointers(self, w1s, w2s) -> Tuple[List[int], List[int]]:
        """Device pointers of per-expert matrices. The checks (GPU, layer dtype,
        contiguous) run once per distinct pointer table; at decode sizes the
        per-parameter checks would otherwise cost more than the kernels."""
        p1 = list(w1s._parameters.values()) if isinstance(w1s, torch.nn.ParameterList) else list(w1s)
        p2 = list(w2s._parameters.values()) if isinstance(w2s, torch.nn.ParameterList) else list(w2s)
        w1p = [t.data_ptr() for t in p1]
        w2p = [t.data_ptr() for t in p2]
        key = (tuple(w1p), tuple(w2p))
        if key not in self._checked_tables:
            for t1, t2 in zip(p1, p2):
                if t1.device.type != "cuda" or t2.device.type != "cuda":
                    raise RuntimeError("expert parameters must be on the GPU")
                if t1.dtype != self.dtype or t2.dtype != self.dtype:
                    raise RuntimeError("expert parameters must be in the layer dtype")
                if not (t1.is_contiguous() and t2.is_contiguous()):
                    raise RuntimeError("expert parameters must be contiguous")
            if len(self._checked_tables) >= 16:
                self._checked_tables.clear()
            self._checked_tables.add(key)
        return w1p, w2p

    @property
    def _shared_folded(self) -> bool:
        return len(self.shared_w1) > 0 and self._shared_piece == self.intermediate_size

    def _experts(self, xd: torch.Tensor, w: torch.Tensor, ids: torch.Tensor, act: int,
                 w1p: List[int], w2p: List[int], expert_map: Optional[List[int]] = None,
                 out: Optional[torch.Tensor] = None, accumulate_f32: bool = False,
                 with_shared: bool = True) -> torch.Tensor:
        """Routed experts (bank pointers ``w1p``/``w2p``, ids renamed through
        ``expert_map`` when given), plus the shared experts when
        ``with_shared``: folded in as extra ids E.. with weight 1, or as a
        second call into an fp32 accumulator."""
        I = self.intermediate_size
        if not with_shared or not len(self.shared_w1):
            return run_experts(xd, w1p, w2p, I, w, ids, act, out=out, expert_map=expert_map,
                               accumulate_f32=accumulate_f32)
        s1, s2 = self._pointers(self.shared_w1, self.shared_w2)
        T, n = xd.shape[0], len(s1)
        if self._shared_folded:
            if ids.shape[1] == self.top_k + n:
                ids2, w2_ = ids, w  # routed with the shared columns (_route32)
            else:
                ids_x = torch.arange(self.num_experts, self.num_experts + n, dtype=ids.dtype,
                                     device=ids.device).expand(T, n)
                ids2 = torch.cat([ids, ids_x], dim=1)
                w2_ = torch.cat([w, torch.ones((T, n), dtype=torch.float32, device=ids.device)],
                                dim=1)
            base = len(w1p)
            if expert_map is None:
                emap = None if base == self.num_experts else \
                    list(range(base)) + [-1] * (self.num_experts - base) + [base + j for j in range(n)]
            else:
                emap = list(expert_map) + [-1] * (self.num_experts - len(expert_map)) + \
                    [base + j for j in range(n)]
            return run_experts(xd, w1p + s1, w2p + s2, I, w2_.contiguous(), ids2, act, out=out,
                               expert_map=emap, accumulate_f32=accumulate_f32)
        acc = out if accumulate_f32 else torch.zeros((T, self.hidden_size), dtype=torch.float32,
                                                     device=xd.device)
        run_experts(xd, w1p, w2p, I, w, ids, act, out=acc, expert_map=expert_map,
                    accumulate_f32=True)
        run_experts(xd, s1, s2, self._shared_piece,
                    torch.ones((T, 1), dtype=torch.float32, device=xd.device),
                    torch.zeros((T, 1), dtype=torch.int32, device=xd.device), act, out=acc,
                    accumulate_f32=True)
        if accumulate_f32:
            return acc
        res = out if out is not None else torch.empty((T, self.hidden_size), dtype=xd.dtype,
                                                      device=xd.device)
        _capi.cast_f32(acc, res)
        return res

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        M = x.shape[0] if x.dim() > 1 else x.numel()
        x2 = x.reshape(-1, self.hidden_size)
        require_gpu(x2)
        xd = x2.to(self.dtype).contiguous()
        # resident layer with folded shared experts: route straight into the
        # [T, K+n] arrays the expert call takes
        w, ids = self._route32(xd, with_shared_cols=not self.uses_offload and self._shared_folded)
        act = activation_code(self.activation)

        if self.cpu_split:
            out = self._forward_split(M, xd, w, ids, act)
        elif self.uses_offload and env.get_chunk_size(0) > 0:
            out = self._forward_streaming(xd, w, ids, act)
        elif self.uses_offload:
            out = self._forward_offload(M, xd, w, ids, act)
        else:
            w1p, w2p = self._resident_banks()
            out = self._experts(xd, w, ids, act, w1p, w2p)
        if out.dtype != x2.dtype:
            out = out.to(x2.dtype)
        return out.reshape(x.shape[:1] + (self.hidden_size,)) if x.dim() > 1 else out

    def forward_with_norm(self, x: torch.Tensor, residual: torch.Tensor,
                          norm) -> Tuple[torch.Tensor, torch.Tensor]:
        """``f, residual = norm.forward_add_residual(x, residual); f = self(f)``
        (reframework/models/base.py:135-136) with the residual add, the
        RMSNorm and the router in one library call; returns (output, new
        residual). ``norm`` is an RMSNorm (its weight, optional bias and eps)."""
        shape = x.shape
        x2 = x.reshape(-1, self.hidden_size)
        require_gpu(x2)
        xd = x2.to(self.dtype).contiguous()
        res = residual.reshape(-1, self.hidden_size).to(self.dtype).contiguous()
        T = xd.shape[0]
        normed = torch.empty_like(xd)
        new_res = torch.empty_like(xd)
        w = torch.empty((T, self.top_k), dtype=torch.float32, device=xd.device)
        ids = torch.empty((T, self.top_k), dtype=torch.int32, device=xd.device)
        gate = self.gate.detach()
        if gate.device != xd.device:
            gate = gate.to(xd.device)
        nw, nb = norm._params(xd)
        if self.entropy_adaptive_k:
            # the entropy-adaptive router is not fused: norm, then the router
            _capi.add_rmsnorm(xd, res, new_res, nw, nb, norm.eps, normed)
            w, ids = self._route32(normed)
        else:
            _capi.add_rmsnorm_router_topk(xd, res, new_res, nw, nb, norm.eps,
                                          gate.to(self.dtype).contiguous(), None, self.top_k,
                                          self.renormalize, True, normed, w, ids,
                                          logits_out=self._logits_buffer(T, xd.device))
        act = activation_code(self.activation)
        if self.cpu_split:
            out = self._forward_split(T, normed, w, ids, act)
        elif self.uses_offload and env.get_chunk_size(0) > 0:
            out = self._forward_streaming(normed, w, ids, act)
        elif self.uses_offload:
            out = self._forward_offload(T, normed, w, ids, act)
        else:
            w1p, w2p = self._resident_banks()
            out = self._experts(normed, w, ids, act, w1p, w2p)
        if out.dtype != x.dtype:
            out = out.to(x.dtype)
        return out.reshape(shape), new_res.reshape(shape).to(residual.dtype)

    def _forward_offload(self, M: int, xd: torch.Tensor, w: torch.Tensor, ids: torch.Tensor,
                         act: int) -> torch.Tensor:
        cache = self._cache
        ids_host, w_host, _ = self._routing_to_host(ids, w)
        kept = self._kept_experts(ids_host, w_host)
        w1s, w2s, local_index = cache.prefetch_slots(kept)
        # Dropped slots contribute nothing; in the routed set recorded for the
        # lookahead they read as the smallest kept id (moe_layer.py:479-486).
        expert_map = [-1] * self.num_experts
        for g, loc in local_index.items():
            expert_map[g] = loc
        if self._predictor is not None:
            fallback = next(iter(local_index)) if local_index else -1
            routed = [i if i in local_index else fallback for i in ids_host]
            self._predictor.record_step(routed, is_prefill=(M > 1),
                                        forward_ms=self._since_last_step_ms())
        w1p = [t.data_ptr() for t in w1s]
        w2p = [t.data_ptr() for t in w2s]
        if not w1p and not len(self.shared_w1):
            return torch.zeros_like(xd)
        out = self._experts(xd, w, ids, act, w1p, w2p, expert_map=expert_map)
        cache.mark_read(local_index)
        return out

    @staticmethod
    def _staged_layout(T: int, K: int, H: int, esz: int):
        """Byte offsets of ids, weights, hidden states and the host-half
        output in the staging buffer, and whether a step of this size fits."""
        def up(n: int) -> int:
            return (n + 255) & ~255
        o_w = up(T * K * 4)
        o_x = o_w + up(T * K * 4)
        o_out = o_x + up(T * H * esz)
        return o_w, o_x, o_out, o_out + T * H * 4 <= _capi.HostStaging.CAPACITY

    def _routing_to_host(self, ids: torch.Tensor, w: torch.Tensor,
                         xd: Optional[torch.Tensor] = None):
        """(ids list, weights list, staging buffer or None) of a step, read
        through the mapped staging buffer by a kernel on the compute stream
        (with xd too, when given) when the step fits it, else with
        synchronous copies. A copy through the DMA engines would wait behind
        expert copies in flight (lookahead loads, the split's background
        loads); the kernel does not."""
        T, K = ids.shape
        dev = ids.device
        o_w, o_x, _, fits = self._staged_layout(T, K, self.hidden_size,
                                                xd.element_size() if xd is not None else 2)
        ids32 = (ids if ids.dtype == torch.int32 else ids.int()).contiguous()
        w32 = w.contiguous()
        if not fits:
            return ids32.reshape(-1).tolist(), w32.reshape(-1).tolist(), None
        stream = _capi.stream_handle(dev)
        stg = _capi.staging(dev, stream)
        regions = [(ids32, 0, T * K * 4), (w32, o_w, T * K * 4)]
        if xd is not None:
            regions.append((xd, o_x, xd.numel() * xd.element_size()))
        _capi.copy_to_host_multi(stg.ptr, regions, stream)
        done = torch.cuda.Event()
        done.record(torch.cuda.current_stream(dev))
        done.synchronize()
        return (stg.array(0, np.int32, T * K).tolist(), stg.array(o_w, np.float32, T * K).tolist(),
                stg)

    @staticmethod
    def _kept_experts(ids_host: List[int], w_host: List[float]) -> List[int]:
        """Experts ranked by summed routing weight (ties: first appearance),
        the first RE_MAX_PACK kept (moe_layer.py:426-442)."""
        weight_sum: Dict[int, float] = {}
        for eid, wt in zip(ids_host, w_host):
            if eid >= 0:
                weight_sum[eid] = weight_sum.get(eid, 0.0) + wt
        kept = [eid for eid, _ in sorted(weight_sum.items(), key=lambda kv: -kv[1])]
        return kept[:env.get_max_pack(2)]

    def _forward_split(self, M: int, xd: torch.Tensor, w: torch.Tensor, ids: torch.Tensor,
                       act: int) -> torch.Tensor:
        """CPU/GPU split forward (moe_layer.py:523-627). The experts to run
        are the offload forward's (RE_MAX_PACK truncation, or all routed with
        RE_CHUNK_SIZE > 0); resident ones with their copy landed run on the
        GPU into an fp32 accumulator, the rest on the host cores from the
        staged pool while the GPU works; the host sum is added in fp32 and the
        total cast once (the host half on the int8 bank with the reference's
        int8 numerics when the split was enabled with int8). Each slot's
        output lands on its own token (the reference indexes tokens as if
        top_k were 1, F6). Afterwards the
        host-computed experts are copied to device memory while fewer than
        RE_MOE_SPLIT_COPY_DEPTH copies are in flight (the reference copies
        every one: reactive_load, moe_layer.py:601).

        The routing, the hidden states and the host half travel through a
        mapped pinned buffer that kernels on the compute stream read and
        write (moe355_copy_to_host / moe355_merge_host_f32): copies through
        the DMA engines would wait behind the expert copies in flight."""
        cache = self._cache
        T, K = ids.shape
        H = self.hidden_size
        dev = xd.device
        stream = _capi.stream_handle(dev)
        esz = xd.element_size()
        _, o_x, o_out, _ = self._staged_layout(T, K, H, esz)
        ids_host, w_host, stg = self._routing_to_host(ids, w, xd)
        if env.get_chunk_size(0) > 0:
            run = sorted({i for i in ids_host if i >= 0})
        else:
            run = self._kept_experts(ids_host, w_host)
        w1s, w2s, local_index, host_ids = cache.split_slots(run)
        expert_map = [-1] * self.num_experts
        for g, loc in local_index.items():
            expert_map[g] = loc
        if not host_ids and (w1s or len(self.shared_w1)):
            # every expert resident: the combine rounds the fp32 sum straight
            # into the output (0 + sum, the same single rounding as below)
            out = self._experts(xd, w, ids, act, [t.data_ptr() for t in w1s],
                                [t.data_ptr() for t in w2s], expert_map=expert_map)
            cache.mark_read(local_index)
            self._record_split(M, run, ids_host)
            return out
        acc = torch.zeros((T, H), dtype=torch.float32, device=dev)
        if w1s or len(self.shared_w1):
            self._experts(xd, w, ids, act, [t.data_ptr() for t in w1s],
                          [t.data_ptr() for t in w2s], expert_map=expert_map, out=acc,
                          accumulate_f32=True)
            cache.mark_read(local_index)
        out = torch.empty((T, H), dtype=xd.dtype, device=dev)
        if host_ids:
            offs, toks, wts = [0], [], []
            for e in host_ids:
                for j, eid in enumerate(ids_host):
                    if eid == e:
                        toks.append(j // K)
                        wts.append(w_host[j])
                offs.append(len(toks))
            if stg is not None:
                x_host = torch.from_numpy(stg.array(o_x, np.uint16, T * H)).view(
                    xd.dtype).reshape(T, H) if esz == 2 else \
                    torch.from_numpy(stg.array(o_x, np.float32, T * H)).reshape(T, H)
                host_out = torch.from_numpy(stg.array(o_out, np.float32, T * H)).reshape(T, H)
                host_out.zero_()
            else:
                x_host = xd.cpu()
                host_out = torch.zeros((T, H), dtype=torch.float32, pin_memory=cache._pinned)
            slots = (np.asarray(offs, np.int32), np.asarray(toks or [0], np.int32),
                     np.asarray(wts or [0.0], np.float32))
            if cache.host_int8:
                bank = [cache._int8_host[e] for e in host_ids]
                sums = [cache._int8_rowsums[e] for e in host_ids]
                _capi.host_experts_int8(x_host, [b[0] for b in bank], [b[1] for b in bank],
                                        [b[2] for b in bank], [b[3] for b in bank],
                                        [r[0] for r in sums], [r[1] for r in sums], *slots, act,
                                        host_out)
            else:
                _capi.host_experts(x_host, [cache._host[e][0] for e in host_ids],
                                   [cache._host[e][1] for e in host_ids], *slots, act, host_out)
            if stg is not None:
                _capi.merge_host_f32(acc, stg.ptr + o_out, out, stream)
            else:
                acc.add_(host_out.to(dev, non_blocking=cache._pinned))
                _capi.cast_f32(acc, out)
            cache.stats.host_experts += len(host_ids)
            cache.load_while_idle(host_ids, env.get_moe_split_copy_depth())
        else:
            _capi.cast_f32(acc, out)
        self._record_split(M, run, ids_host)
        return out

    def _record_split(self, M: int, run: List[int], ids_host: List[int]) -> None:
        """The split step's routed set for the lookahead predictor; dropped
        slots read as the first kept id, as in _forward_offload."""
        if self._predictor is not None:
            ran = set(run)
            fallback = min(run) if run else -1
            routed = [i if i in ran else fallback for i in ids_host]
            self._predictor.record_step(routed, is_prefill=(M > 1),
                                        forward_ms=self._since_last_step_ms())

    def _forward_streaming(self, xd: torch.Tensor, w: torch.Tensor, ids: torch.Tensor,
                           act: int) -> torch.Tensor:
        """Every routed expert, ``RE_CHUNK_SIZE`` experts at a time, summed in
        fp32 and cast once at the end (moe_layer.py:354-420); the shared
        experts join the first chunk."""
        cache = self._cache
        chunk_size = env.get_chunk_size(8)
        ids_host, _, _ = self._routing_to_host(ids, w)
        uniq = sorted({i for i in ids_host if i >= 0})
        acc = torch.zeros((xd.shape[0], self.hidden_size), dtype=torch.float32, device=xd.device)
        starts = list(range(0, len(uniq), chunk_size)) or [0]
        for n, start in enumerate(starts):
            chunk = uniq[start:start + chunk_size]
            w1s, w2s, local_index = cache.prefetch_slots(chunk)
            expert_map = [-1] * self.num_experts
            for g, loc in local_index.items():
                expert_map[g] = loc
            if not w1s and (n > 0 or not len(self.shared_w1)):
                continue
            self._experts(xd, w, ids, act, [t.data_ptr() for t in w1s],
                          [t.data_ptr() for t in w2s], expert_map=expert_map, out=acc,
                          accumulate_f32=True, with_shared=(n == 0))
            cache.mark_read(local_index)
        out = torch.empty((xd.shape[0], self.hidden_size), dtype=xd.dtype, device=xd.device)
        _capi.cast_f32(acc, out)
        return out

    # -------------------------------------------------------------- (de)serial
    def state_dict(self, *, prefix: str = "", result: Optional[dict] = None,
                   destination=None, keep_vars: bool = False) -> Dict[str, torch.Tensor]:
        result = destination if destination is not None else ({} if result is None else result)
        result[f"{prefix}.gate.weight" if prefix else "gate.weight"] = self.gate
        I = self.intermediate_size
        for e in range(len(self.experts_w1)):
            p = f"{prefix}.experts.{e}" if prefix else f"experts.{e}"
            result[f"{p}.gate_proj.weight"] = self.experts_w1[e][:I]
            result[f"{p}.up_proj.weight"] = self.experts_w1[e][I:]
            result[f"{p}.down_proj.weight"] = self.experts_w2[e]
        if len(self.shared_w1):
            p = f"{prefix}.shared_experts" if prefix else "shared_experts"
            P = self._shared_piece
            with torch.no_grad():
                result[f"{p}.gate_proj.weight"] = torch.cat([t[:P] for t in self.shared_w1])
                result[f"{p}.up_proj.weight"] = torch.cat([t[P:] for t in self.shared_w1])
                result[f"{p}.down_proj.weight"] = torch.cat(list(self.shared_w2), dim=1)
        return result

    def load_state_dict(self, state_dict: Dict[str, torch.Tensor], *, prefix: str = "",
                        strict: bool = True, assign: bool = False) -> None:
        with torch.no_grad():
            g = f"{prefix}.gate.weight" if prefix else "gate.weight"
            if g in state_dict:
                self.gate.copy_(state_dict[g].detach().to(dtype=self.dtype))
            I = self.intermediate_size
            for e in range(len(self.experts_w1)):
                p = f"{prefix}.experts.{e}" if prefix else f"experts.{e}"
                for name, param in (("gate_proj", self.experts_w1[e][:I]),
                                    ("up_proj", self.experts_w1[e][I:]),
                                    ("down_proj", self.experts_w2[e])):
                    key = f"{p}.{name}.weight"
                    if key in state_dict:
                        param.copy_(state_dict[key].detach().to(dtype=self.dtype))
            if len(self.shared_w1):
                p = f"{prefix}.shared_experts" if prefix else "shared_experts"
                P = self._shared_piece
                for j in range(len(self.shared_w1)):
                    cols = slice(j * P, (j + 1) * P)
                    for name, dst, src_slice in (("gate_proj", self.shared_w1[j][:P], cols),
                                                 ("up_proj", self.shared_w1[j][P:], cols)):
                        key = f"{p}.{name}.weight"
                        if key in state_dict:
                            dst.copy_(state_dict[key].detach()[src_slice].to(dtype=self.dtype))
                    key = f"{p}.down_proj.weight"
                    if key in state_dict:
                        self.shared_w2[j].copy_(
                            state_dict[key].detach()[:, cols].to(dtype=self.dtype))


__all__ = ["FusedMoE", "CpuShuttle"]
