"""Pinned-host expert pool with an HBM LRU window, for one MoE layer.

Drop-in for the reference's ``ExpertOffloadCache`` / ``Prediction`` /
``OffloadStats`` (reframework/moe/offload_cache.py:75-751): same constructor,
methods, counters, eviction policies (``RE_CACHE_POLICY`` = ``lru`` |
``least_stale``), two-tier hard/soft protection, lookahead ``reserve`` with a
bandwidth- and room-bounded dynamic k, and similarity substitution. The policy
is host bookkeeping and stays in Python, decision for decision the
reference's.

What changes on MI355X is how bytes move:

  * Resident experts live in fixed HBM *slots*, each one buffer holding w1
    ``[2I,H]`` followed by w2 ``[H,I]``. Evicted slots go to a free list and
    are reused; nothing is reallocated per miss.
  * A miss is one ``hipMemcpyAsync`` (libmoe355 ``moe355_h2d_async``) from the
    pinned pool into a slot on the device's copy stream (one per device,
    shared by every cache: per-cache streams beyond the process's hardware
    queues land on the compute stream's queue, whose kernels then wait for
    the copies), with an event recorded behind it.
    The host does not wait: compute streams wait on the slot's event right
    before the kernels that read it (:meth:`prefetch_slots`), so the copy of
    one expert overlaps whatever is already queued, e.g. the lookahead loads
    of ``reserve`` overlap the current step's expert FFN.
  * A freed slot remembers an event recorded on the compute stream at
    eviction time; the next copy into that slot waits for it, so an in-flight
    kernel never sees its weights overwritten.
  * :meth:`prefetch_slots` hands the FFN a list of per-slot views, which
    libmoe355 consumes as a pointer table: the reference's per-step
    ``torch.stack`` of the banks (``_pack``) disappears from the hot path.
    :meth:`prefetch` still returns stacked banks for callers that want them.

With ``device="cpu"`` (unit tests) the "HBM" is host memory and resident
entries are views of the host pool, as in the reference, where ``.to("cpu")``
of a CPU tensor is the tensor itself.
"""

from __future__ import annotations

import logging
import time
from collections import OrderedDict, deque
from dataclasses import dataclass
from typing import Deque, Dict, List, Optional, Sequence, Tuple

import torch

from reframework_amd import _capi, env

logger = logging.getLogger(__name__)


def _quantize_int8(w: torch.Tensor) -> Tuple[torch.Tensor, float, torch.Tensor]:
    """(codes shaped like ``w``, scale, int32 code sums of its last-dim rows)
    by libmoe355_host's symmetric per-tensor rule."""
    if w.numel() == 0:
        return (torch.zeros_like(w, dtype=torch.int8, device="cpu"), 1.0,
                torch.zeros(w.shape[:-1] if w.dim() else (), dtype=torch.int32).reshape(-1))
    h = w.detach().cpu().contiguous()
    rows = h.reshape(-1, h.shape[-1]) if h.dim() >= 2 else h.reshape(1, -1)
    q, scale, rs = _capi.host_quantize_int8(rows)
    return q.reshape(h.shape), scale, rs


def _sym_int8_quantize(w: torch.Tensor) -> Tuple[torch.Tensor, float]:
    """Symmetric per-tensor int8 codes and scale, ``w ~= q * scale``
    (reference: offload_cache.py:58-72): scale = max |w| / 127 in fp32, codes
    the fp32 quotient ``w / scale`` rounded half to even and clamped to +-127;
    an all-zero tensor gets scale 1.0. Computed by libmoe355_host."""
    q, scale, _ = _quantize_int8(w)
    return q, scale


@dataclass
class OffloadStats:
    """Counters for observability / benchmarking."""

    hits: int = 0
    misses: int = 0
    evictions: int = 0
    transfers_bytes: int = 0
    subs: int = 0
    predicts: int = 0
    inflight_bytes: int = 0
    # CPU/GPU split forward: experts computed on the host cores (not in the
    # reference's counters, so not in as_dict)
    host_experts: int = 0

    def reset(self) -> None:
        for name in ("hits", "misses", "evictions", "transfers_bytes", "subs", "predicts",
                     "inflight_bytes", "host_experts"):
            setattr(self, name, 0)

    def as_dict(self) -> dict:
        return {
            "hits": self.hits,
            "misses": self.misses,
            "evictions": self.evictions,
            "subs": self.subs,
            "predicts": self.predicts,
            "inflight_bytes": self.inflight_bytes,
            "transfer_mb": self.transfers_bytes / (1024 * 1024),
        }


class Prediction:
    """Rolling routed-set history of one layer that drives the lookahead.

    ``record_step`` on a decode step ages every seen expert, stores the routed
    set, ranks the next step's experts and hands them to
    :meth:`ExpertOffloadCache.reserve`; a prefill step clears the history
    instead (reference: offload_cache.py:108-223).
    """

    def __init__(self, cache: "ExpertOffloadCache", window: int = 32) -> None:
        self.cache = cache
        self.window = max(1, int(window))
        self._history: Deque[frozenset] = deque(maxlen=self.window)
        self._age: Dict[int, int] = {}  # decode steps since the expert last routed

    def reset(self) -> None:
        self._history.clear()
        self._age.clear()

    def record_step(self, routed: Sequence[int], *, is_prefill: bool, forward_ms: float,
                    inflight_bytes: float = 0.0) -> None:
        routed_set = frozenset(int(i) for i in routed)
        if is_prefill:
            self.reset()
            return
        for e in self._age:
            self._age[e] += 1
        for e in routed_set:
            self._age[e] = 0
        self._history.append(routed_set)
        predicted = self.predict_next()
        if predicted:
            self.cache.reserve(predicted, forward_ms=forward_ms, protect_current=routed,
                               inflight_bytes=inflight_bytes)

    def predict_next(self, limit: Optional[int] = None) -> List[int]:
        """Non-resident experts ranked by window frequency, then recency, then id.

        score = 1000 * (#steps routed in the window) + (window - age); an expert
        never aged counts as age = window.
        """
        freq: Dict[int, int] = {}
        for step in self._history:
            for e in step:
                freq[e] = freq.get(e, 0) + 1
        if not freq:
            return []
        ranked = sorted(
            freq, key=lambda e: (-(freq[e] * 1000 + self.window - self._age.get(e, self.window)), e)
        )
        out: List[int] = []
        for e in ranked:
            if e in self.cache._lru:
                continue
            out.append(e)
            if limit is not None and len(out) >= limit:
                break
        return out


# Host->device expert copies still running, per device (events of every
# cache's copies, pruned as they complete): the CPU/GPU split forward bounds
# its loads by this count so they never queue up behind each other.
_INFLIGHT: Dict[int, List[object]] = {}


def inflight_copies(device: torch.device) -> int:
    evs = _INFLIGHT.get(device.index if device.index is not None else 0)
    if not evs:
        return 0
    evs[:] = [e for e in evs if not e.query()]
    return len(evs)


def _note_inflight(device: torch.device, event) -> None:
    evs = _INFLIGHT.setdefault(device.index if device.index is not None else 0, [])
    evs[:] = [e for e in evs if not e.query()]
    evs.append(event)


# One host->device copy stream per device, shared by every cache on it. A
# process gets a few hardware queues (GPU_MAX_HW_QUEUES, 4 by default) and
# streams beyond them share queues: a copy stream on the compute stream's
# queue puts the marker that ends each of its copies in that queue, so the
# kernels queued after it wait for the copy (6 ms for a Mixtral expert). With
# a stream per layer cache (32 in the offload decode) some always shared it.
_COPY_STREAMS: Dict[int, "torch.cuda.Stream"] = {}


def _copy_stream_for(device: torch.device) -> "torch.cuda.Stream":
    idx = device.index if device.index is not None else torch.cuda.current_device()
    stream = _COPY_STREAMS.get(idx)
    if stream is None:
        stream = torch.cuda.Stream(device=device)  # default priority
        _COPY_STREAMS[idx] = stream
    return stream


class _HostPool:
    """Owner of one staged host buffer, shared by every cache that reads it
    (``share_host``).

    Copies out of the buffer are raw ``hipMemcpyAsync`` calls, which torch's
    pinned allocator does not track: once the last reference to a pinned
    block is gone it may hand the pages out again at once. Each cache
    therefore notes the last copy it queued on its copy stream here, and the
    buffer is released only after every noted copy has finished (when the
    holder itself is dropped, i.e. when the last cache reading it lets go or
    replaces it)."""

    __slots__ = ("buf", "_last", "touched", "int8")

    def __init__(self, buf: torch.Tensor) -> None:
        self.buf = buf
        self._last: Dict[int, object] = {}  # copy stream handle -> last copy event
        self.touched = False  # every page read once by the host (see touch_pages)
        # the int8 bank of the pool's experts, built once for every cache
        # reading the pool: ([(q1, q2, s1, s2)], [(row sums 1, row sums 2)])
        self.int8: Optional[Tuple[list, list]] = None

    def touch_pages(self) -> None:
        """Read one element of every 4 KiB page from the host. The driver
        maps pinned pages into the process on first access, so without this
        the first host computation of each expert pays a page fault per page
        (~20 ms for a Mixtral expert)."""
        if self.touched:
            return
        step = max(1, 4096 // self.buf.element_size())
        self.buf[::step].float().sum()
        self.touched = True

    def note_copy(self, stream_key: int, event) -> None:
        self._last[stream_key] = event  # stream order: it covers the earlier copies

    def drain(self) -> None:
        """Wait for every copy noted so far."""
        last, self._last = self._last, {}
        for ev in last.values():
            ev.synchronize()

    def __del__(self) -> None:
        try:
            self.drain()
        except Exception:  # interpreter shutdown: the runtime may already be gone
            pass


class _Slot:
    """One HBM buffer holding an expert's w1 then w2, plus its stream events."""

    __slots__ = ("buf", "w1", "w2", "ready", "last_copy", "free_after", "refs", "reads",
                 "handed")

    def __init__(self, buf: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor) -> None:
        self.buf = buf
        self.w1 = w1
        self.w2 = w2
        self.ready: Optional[torch.cuda.Event] = None  # copy into the slot finished
        # The last copy into the slot, kept after release: a slot evicted
        # before anything read it may still be filling on one layer's copy
        # stream when another layer's copy stream takes it.
        self.last_copy: Optional[torch.cuda.Event] = None
        # Events the next copy into the slot waits for: its readers finished.
        self.free_after: List[torch.cuda.Event] = []
        # Readers marked by mark_read (one event per compute stream), and
        # whether the slot was handed out since the last mark: an unmarked
        # hand-out makes the release wait for everything queued.
        self.reads: Dict[int, torch.cuda.Event] = {}
        self.handed = False
        self.refs = 0


class ExpertPool:
    """One HBM slot pool and one LRU shared by the offload caches of several
    layers (no counterpart in the reference, whose caches are per layer).

    Recency is global over (layer cache, expert), as in litemoe's global LRU
    (litemoe/src/litemoe/cache/lru.py:66-102): a hit moves the entry to the
    back, a miss is appended, and the oldest entries are evicted while the
    pool is over ``capacity``. Unlike that cache, the experts of the request
    being served are never evicted by it (their slots are about to be read),
    so a request larger than the pool overflows it, as the per-layer cache
    does. Freed slots go to a free list shared by all member caches (experts
    of one model have one size).
    """

    def __init__(self, capacity: int) -> None:
        self.capacity = int(capacity)
        self._order: "OrderedDict[Tuple[int, int], ExpertOffloadCache]" = OrderedDict()
        self._free: List[_Slot] = []
        self.n_slots = 0

    def __len__(self) -> int:
        return len(self._order)

    def touch(self, cache: "ExpertOffloadCache", idx: int) -> None:
        key = (id(cache), int(idx))
        self._order[key] = cache
        self._order.move_to_end(key)

    def forget(self, cache: "ExpertOffloadCache", idx: int) -> None:
        self._order.pop((id(cache), int(idx)), None)

    def evict(self, cache: "ExpertOffloadCache", hard: Sequence[int], incoming: int = 0) -> None:
        """Evict oldest-first down to capacity, sparing ``cache``'s ``hard``;
        with ``incoming`` > 0, make room for that many entries about to be
        admitted (the victims the same admission would evict afterwards)."""
        spare = {(id(cache), int(i)) for i in hard}
        while len(self._order) + incoming > self.capacity:
            victim = next((k for k in self._order if k not in spare), None)
            if victim is None:
                return
            owner = self._order.pop(victim)
            owner._drop(victim[1])

    def acquire(self, make) -> _Slot:
        if self._free:
            return self._free.pop()
        self.n_slots += 1
        return make()

    def release(self, slot: _Slot) -> None:
        self._free.append(slot)


class ExpertOffloadCache:
    """Pinned-host expert pool + an HBM LRU window of expert slots.

    Parameters
    ----------
    device: where resident experts live (``cuda:N``; ``cpu`` for policy tests).
    lru_capacity: resident expert slots kept (one slot = one expert's w1+w2).
    dtype: storage dtype of the experts.
    """

    def __init__(self, device, lru_capacity: int, dtype: torch.dtype = torch.float16,
                 pool: Optional[ExpertPool] = None) -> None:
        self.device = torch.device(device)
        self.lru_capacity = int(lru_capacity)
        # With a shared pool, residency and eviction are global across the
        # member caches and lru_capacity is not used.
        self._pool = pool
        self.dtype = dtype
        self._host: List[Tuple[torch.Tensor, torch.Tensor]] = []
        self._host_buf: Optional[torch.Tensor] = None
        self._host_pool: Optional[_HostPool] = None
        self._host_off: List[int] = []
        self._pinned = False
        self._lru: "OrderedDict[int, Tuple[torch.Tensor, torch.Tensor]]" = OrderedDict()
        self.stats = OffloadStats()
        self._next_reserve: frozenset = frozenset()
        self.sim_table: Optional[torch.Tensor] = None
        self._predictor: Optional[Prediction] = None
        self._bw_gb_s: Optional[float] = None
        self._bw_headroom: float = 0.9
        self._cpu_split = False
        self._int8_host: List[Tuple[torch.Tensor, torch.Tensor, float, float]] = []
        # int32 code sums of each int8 expert's rows (w1, w2), for the host kernels
        self._int8_rowsums: List[Tuple[torch.Tensor, torch.Tensor]] = []
        self._host_int8 = False  # the split's host half runs on the int8 bank
        # HBM slot pool (cuda devices only)
        self._slot_of: Dict[int, _Slot] = {}
        self._free_slots: List[_Slot] = []
        self._n_slots = 0
        self._copy_stream: Optional[torch.cuda.Stream] = None
        self._copy_log: Optional[List[Tuple[torch.cuda.Event, torch.cuda.Event, int]]] = None
        self._n1 = 0
        self._n2 = 0

    # ----------------------------------------------------------------- factory
    @classmethod
    def from_config(cls, cfg, *, device=None, lru_capacity: Optional[int] = None):
        return cls(
            device=torch.device(device or cfg.device),
            lru_capacity=lru_capacity if lru_capacity is not None else env.get_moe_cache_size(),
            dtype=cfg.dtype,
        )

    # ------------------------------------------------------------------- setup
    def load(self, experts: Sequence[Dict[str, torch.Tensor]]) -> None:
        """Stage per-expert ``{"w1": [2I,H], "w2": [H,I]}`` in one host pool.

        The pool is pinned (hipHostMalloc through torch) when a GPU is present,
        else pageable, as on a CPU-only box in the reference.
        """
        w1s = [e["w1"].detach().to(dtype=self.dtype).contiguous() for e in experts]
        w2s = [e["w2"].detach().to(dtype=self.dtype).contiguous() for e in experts]
        buf = self._alloc_pool([(tuple(a.shape), tuple(b.shape)) for a, b in zip(w1s, w2s)])
        for (v1, v2), w1, w2 in zip(self._host, w1s, w2s):
            v1.copy_(w1)
            v2.copy_(w2)
        del w1s, w2s, buf
        self._loaded()

    def load_from(self, num_experts: int, hidden: int, inter: int, fetch) -> None:
        """Stage experts one at a time from ``fetch(e) -> (gate [I,H], up
        [I,H], down [H,I])`` (host tensors of any float dtype, e.g. lazily read
        checkpoint slices) straight into the host pool, without first
        building per-expert tensors."""
        self._alloc_pool([((2 * inter, hidden), (hidden, inter))] * num_experts)
        for e, (v1, v2) in enumerate(self._host):
            g, u, d = fetch(e)
            if tuple(g.shape) != (inter, hidden) or tuple(u.shape) != (inter, hidden) or \
                    tuple(d.shape) != (hidden, inter):
                raise ValueError(f"expert {e}: shapes {tuple(g.shape)}, {tuple(u.shape)}, "
                                 f"{tuple(d.shape)} do not match hidden={hidden} inter={inter}")
            v1[:inter].copy_(g)
            v1[inter:].copy_(u)
            v2.copy_(d)
        self._loaded()

    def share_host(self, other: "ExpertOffloadCache") -> None:
        """Use ``other``'s staged host pool instead of staging a copy: layers
        whose experts hold the same weights keep one pinned pool between
        them (and a deep offload stack can be built on a host that cannot
        pin every layer's experts). HBM slots, LRU and statistics stay this
        cache's own; the pool stays alive while either cache holds it."""
        if not other._host:
            raise ValueError("the other cache has no staged experts")
        if other.dtype != self.dtype:
            raise ValueError(f"host pool dtype {other.dtype} != cache dtype {self.dtype}")
        self._host_pool = other._host_pool
        self._host_buf = other._host_buf
        self._host = list(other._host)
        self._host_off = list(other._host_off)
        self._pinned = other._pinned
        self._int8_host = []
        self._int8_rowsums = []
        self._host_int8 = False
        self._cpu_split = False
        self._loaded()

    def _alloc_pool(self, shapes) -> torch.Tensor:
        """One host buffer holding every expert's w1 then w2; pinned
        (hipHostMalloc through torch) when a GPU is present, else pageable."""
        total = 0
        for s1, s2 in shapes:
            total += s1[0] * s1[1] + s2[0] * s2[1]
        # The pool being replaced (if any) is released when its holder is
        # dropped, after the copies every sharing cache queued out of it.
        try:
            buf = torch.empty(total, dtype=self.dtype, pin_memory=True)
            self._pinned = True
        except (RuntimeError, AssertionError):
            buf = torch.empty(total, dtype=self.dtype)
            self._pinned = False
        self._host_pool = _HostPool(buf)
        self._host_buf = buf
        self._host, self._host_off = [], []
        off = 0
        for s1, s2 in shapes:
            self._host_off.append(off)
            n1, n2 = s1[0] * s1[1], s2[0] * s2[1]
            v1 = buf[off:off + n1].view(s1)
            v2 = buf[off + n1:off + n1 + n2].view(s2)
            off += n1 + n2
            self._host.append((v1, v2))
        return buf

    def _loaded(self) -> None:
        if self._host:
            self._n1 = self._host[0][0].numel()
            self._n2 = self._host[0][1].numel()
        self._release_all()
        self._lru = OrderedDict()
        self.stats.reset()
        # an int8 bank describes the previous pool's weights
        self._int8_host = []
        self._int8_rowsums = []
        if self._cpu_split:  # an armed split reads the new pool: rebuild what it needs
            self.enable_host_experts(int8=self._host_int8)
        logger.info("ExpertOffloadCache staged %d experts (%s) in %s host pool; LRU cap=%d",
                    len(self._host), self.dtype, "pinned" if self._pinned else "pageable",
                    self.lru_capacity)

    @property
    def num_experts(self) -> int:
        return len(self._host)

    @property
    def cpu_split(self) -> bool:
        return self._cpu_split

    def resident_set(self) -> frozenset:
        return frozenset(self._lru.keys())

    def set_sim_table(self, sim: torch.Tensor) -> None:
        E = len(self._host)
        sim = torch.as_tensor(sim, dtype=torch.float32).cpu()
        if tuple(sim.shape) != (E, E):
            raise ValueError(f"sim_table shape {tuple(sim.shape)} != [E,E]=[{E},{E}]")
        self.sim_table = sim

    def attach_predictor(self, window: int = 32) -> None:
        self._predictor = Prediction(self, window=window)
        self._bw_headroom = max(0.05, min(1.0, env.get_moe_predict_headroom()))
        self.measure_bandwidth()

    def quantize_int8_host(self) -> None:
        """Per-expert symmetric int8 host bank (reference: offload_cache.py:386-407).
        Caches reading one staged pool (``share_host``) build it once and
        share it."""
        if not self._host:
            return
        shared = self._host_pool is not None and self._host_pool.int8 is not None
        if shared:  # another cache on the same staged pool built it
            bank, sums = self._host_pool.int8
        else:
            bank, sums = [], []
            for w1, w2 in self._host:
                q1, s1, r1 = _quantize_int8(w1)
                q2, s2, r2 = _quantize_int8(w2)
                bank.append((q1, q2, s1, s2))
                sums.append((r1, r2))
            if self._host_pool is not None:
                self._host_pool.int8 = (bank, sums)
        self._int8_host = list(bank)
        self._int8_rowsums = list(sums)
        self._host_int8 = True  # as in the reference, the split's host half uses this bank
        self._cpu_split = True

    def cpu_banks(self, indices: Sequence[int]):
        """Stacked int8 banks + scales of ``indices`` (ascending, at most
        ``RE_MAX_PACK`` (default 4) of them) and their local index."""
        uniq = sorted(set(int(i) for i in indices))
        max_pack = env.get_max_pack(4)
        if len(uniq) > max_pack:
            uniq = uniq[:max_pack]
        local_index = {idx: k for k, idx in enumerate(uniq)}
        if not uniq:
            H = self._host[0][0].shape[1]
            I = self._host[0][1].shape[1]
            return (torch.empty((0, 2 * I, H), dtype=torch.int8),
                    torch.empty((0, H, I), dtype=torch.int8),
                    torch.empty((0,), dtype=torch.float32),
                    torch.empty((0,), dtype=torch.float32), local_index)
        q1 = torch.stack([self._int8_host[i][0] for i in uniq], dim=0)
        q2 = torch.stack([self._int8_host[i][1] for i in uniq], dim=0)
        s1 = torch.tensor([self._int8_host[i][2] for i in uniq], dtype=torch.float32)
        s2 = torch.tensor([self._int8_host[i][3] for i in uniq], dtype=torch.float32)
        return q1, q2, s1, s2, local_index

    def measure_bandwidth(self) -> Optional[float]:
        """Host->HBM GB/s over the same pinned hipMemcpyAsync path ``_fill`` uses,
        timed with HIP events; None without a GPU."""
        if not torch.cuda.is_available() or self.device.type != "cuda":
            return None
        try:
            n = 1 << 20
            src = torch.empty(n, dtype=self.dtype, pin_memory=self._pinned)
            dst = torch.empty(n, dtype=self.dtype, device=self.device)
            cs = self._side_stream()
            nbytes = n * src.element_size()
            _capi.h2d_async(dst.data_ptr(), src.data_ptr(), nbytes, cs.cuda_stream)  # warm-up
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 3
            start.record(cs)
            for _ in range(reps):
                _capi.h2d_async(dst.data_ptr(), src.data_ptr(), nbytes, cs.cuda_stream)
            stop.record(cs)
            stop.synchronize()
            ms = start.elapsed_time(stop)
            if ms > 0:
                self._bw_gb_s = nbytes * reps / (ms / 1000.0) / 1e9
            return self._bw_gb_s
        except Exception as exc:  # best effort, like the reference's probe
            logger.warning("host->HBM bandwidth measure failed: %s", exc)
            return None

    def use_pool(self, pool: Optional["ExpertPool"]) -> None:
        """Switch between a per-layer LRU window (None) and a shared pool;
        the resident set starts empty."""
        self.reset_lru()
        self._free_slots = []
        self._n_slots = 0
        self._pool = pool

    def log_copies(self, on: bool = True) -> None:
        """Time every miss copy with HIP events on the copy stream (off by
        default; costs two events per miss)."""
        self._copy_log = [] if on else None

    def copy_summary(self) -> Tuple[int, float]:
        """(bytes, milliseconds) summed over the logged miss copies; waits for
        them to finish."""
        if not self._copy_log:
            return 0, 0.0
        self._copy_log[-1][1].synchronize()
        return (sum(n for _, _, n in self._copy_log),
                sum(a.elapsed_time(b) for a, b, _ in self._copy_log))

    def reset_lru(self) -> None:
        if self._pool is not None:
            for idx in list(self._lru):
                self._pool.forget(self, idx)
        self._release_all()
        self._lru = OrderedDict()
        self._next_reserve = frozenset()
        if self._predictor is not None:
            self._predictor.reset()

    # ------------------------------------------------------------------ access
    def _admit(self, indices: Sequence[int]) -> List[int]:
        """Residency bookkeeping shared by prefetch and prefetch_slots
        (reference: offload_cache.py:478-506)."""
        uniq = sorted(set(int(i) for i in indices if int(i) >= 0))
        hits = sum(1 for i in uniq if i in self._lru)
        logger.debug("[offload] prefetch: requested=%d unique=%d hit=%d miss=%d lru_size=%d",
                     len(indices), len(uniq), hits, len(uniq) - hits, len(self._lru))
        if self.sim_table is None:
            # Evict first what admitting the misses will evict anyway, so
            # their copies reuse the freed slots and residency never exceeds
            # max(capacity, request). (With a similarity table a victim may
            # still serve a miss as its substitute: keep the reference order.)
            self._make_room(uniq, len(uniq) - hits)
        for idx in uniq:
            if idx in self._lru:
                self.stats.hits += 1
            elif self._substitute(idx) is None:
                self._fill(idx)
            self._lru.move_to_end(idx)
            if self._pool is not None:
                self._pool.touch(self, idx)
        if self._pool is not None:
            self._pool.evict(self, uniq)
        else:
            self._evict(uniq, self._next_reserve - set(uniq))
        return uniq

    def _make_room(self, hard: Sequence[int], incoming: int) -> None:
        """Evict, ahead of admitting ``incoming`` new entries, the entries
        the eviction after the admission would pick: the admitted entries are
        hard-protected, so they are never the victims, and the victims' order
        does not depend on them."""
        if incoming <= 0:
            return
        if self._pool is not None:
            self._pool.evict(self, hard, incoming=incoming)
        else:
            self._evict(hard, self._next_reserve - set(int(i) for i in hard), incoming=incoming)

    def prefetch(self, indices: Sequence[int]) -> Tuple[torch.Tensor, torch.Tensor, Dict[int, int]]:
        """Bring ``indices`` resident; return stacked banks ``[N,2I,H]``,
        ``[N,H,I]`` (ascending ids) and the global->row map."""
        return self._pack(self._admit(indices))

    def prefetch_slots(self, indices: Sequence[int]):
        """Like :meth:`prefetch` but without the stacking copy: returns the
        per-expert resident views (w1 list, w2 list) in ascending id order and
        the global->row map, after making the current stream wait for any copy
        still filling them."""
        uniq = self._admit(indices)
        self._wait_ready(uniq)
        self._hand_out(uniq)
        w1 = [self._lru[i][0] for i in uniq]
        w2 = [self._lru[i][1] for i in uniq]
        return w1, w2, {idx: k for k, idx in enumerate(uniq)}

    def _hand_out(self, ids: Sequence[int]) -> None:
        for i in ids:
            slot = self._slot_of.get(i)
            if slot is not None:
                slot.handed = True

    def mark_read(self, ids: Sequence[int]) -> None:
        """Record that every kernel reading the slots of ``ids`` (views
        handed out by prefetch_slots / split_slots) is queued on the current
        stream: a later copy into one of these slots then waits only for an
        event recorded here, not for everything queued at its eviction. A
        caller that never marks keeps that conservative wait."""
        if self.device.type != "cuda":
            return
        stream = torch.cuda.current_stream(self.device)
        ev = None
        for i in ids:
            slot = self._slot_of.get(int(i))
            if slot is None:
                continue
            if ev is None:
                ev = torch.cuda.Event()
                ev.record(stream)
            slot.reads[int(stream.cuda_stream)] = ev
            slot.handed = False

    def split_prefetch(self, indices: Sequence[int]):
        """Split the routed set by residency: stacked banks of the hits and the
        list of misses (reference: offload_cache.py:509-552)."""
        uniq = sorted(set(int(i) for i in indices))
        hits = [i for i in uniq if i in self._lru]
        misses = [i for i in uniq if i not in self._lru]
        for i in hits:
            self._lru.move_to_end(i)
            self.stats.hits += 1
        if hits:
            banks = self._pack(hits)
        else:
            w1r, w2r = self._host[0]
            H, I = w1r.shape[1], w2r.shape[1]
            banks = (torch.empty((0, 2 * I, H), dtype=self.dtype, device=self.device),
                     torch.empty((0, H, I), dtype=self.dtype, device=self.device), {})
        return banks, misses

    def enable_host_experts(self, int8: bool = False) -> None:
        """Arm the CPU/GPU split for this cache: experts that are not
        resident are computed on the host cores (libmoe355_host). By default
        straight from the staged 16-bit pool with the device kernels'
        numerics; with ``int8`` from the reference's per-tensor int8 bank
        (quantize_int8_host, offload_cache.py:386-407), built here, which
        reads half the bytes per expert."""
        if not self._host:
            return
        _capi.host_lib()  # a missing host library fails here, not mid-forward
        if int8:
            self.quantize_int8_host()
        elif self._host_pool is not None:
            self._host_pool.touch_pages()
        self._host_int8 = bool(int8)
        self._cpu_split = True

    @property
    def host_int8(self) -> bool:
        """Whether the split's host half runs on the int8 bank."""
        return self._host_int8

    def split_slots(self, indices: Sequence[int]):
        """Split ``indices`` for the CPU/GPU split forward (reference:
        split_prefetch, offload_cache.py:509-552): experts resident in device
        memory whose copy has landed go to the device half (hits: moved to the
        recent end), every other one to the host half. Nothing is copied here.
        Returns (w1 views, w2 views, {id: row}) of the device half, in
        ascending id, and the host half's ids."""
        uniq = sorted(set(int(i) for i in indices if int(i) >= 0))
        dev_ids, host_ids = [], []
        for i in uniq:
            slot = self._slot_of.get(i)
            landed = i in self._lru and (slot is None or slot.ready is None or slot.ready.query())
            if landed:
                self.stats.hits += 1
                self._lru.move_to_end(i)
                if self._pool is not None:
                    self._pool.touch(self, i)
                dev_ids.append(i)
            else:
                host_ids.append(i)
        self._wait_ready(dev_ids)
        self._hand_out(dev_ids)
        w1 = [self._lru[i][0] for i in dev_ids]
        w2 = [self._lru[i][1] for i in dev_ids]
        return w1, w2, {idx: k for k, idx in enumerate(dev_ids)}, host_ids

    def load_while_idle(self, indices: Sequence[int], max_inflight: int) -> List[int]:
        """The split forward's reactive load (reference: reactive_load after
        the merge, moe_layer.py:601): make the non-resident experts of
        ``indices`` resident, in ascending id, while fewer than
        ``max_inflight`` host->device copies run on this device. Evicts as
        reactive_load does (only the experts being loaded are protected).
        Returns the ids loaded."""
        loaded: List[int] = []
        if self.device.type != "cuda":
            return loaded
        for i in sorted(set(int(x) for x in indices)):
            if i in self._lru:
                continue
            if inflight_copies(self.device) >= max_inflight:
                break
            self._make_room(loaded + [i], 1)
            self._fill(i)
            loaded.append(i)
            if self._pool is not None:
                self._pool.touch(self, i)
        return loaded

    def reactive_load(self, indices: Sequence[int]) -> None:
        uniq = sorted(set(int(i) for i in indices))
        self._make_room(uniq, sum(1 for i in uniq if i not in self._lru))
        for i in uniq:
            if i not in self._lru:
                self._fill(i)
            if self._pool is not None:
                self._pool.touch(self, i)
        if self._pool is not None:
            self._pool.evict(self, uniq)
        else:
            self._evict(uniq, self._next_reserve - set(uniq))

    def reserve(
        self,
        predicted: Sequence[int],
        *,
        forward_ms: float = 0.0,
        bandwidth_gb_s: Optional[float] = None,
        protect_current: Sequence[int] = (),
        inflight_bytes: float = 0.0,
    ) -> int:
        """Load the predicted next-step experts, most likely first; return how
        many were loaded (reference: offload_cache.py:569-643).

        k is bounded by the byte budget ``bw * window * headroom - inflight``
        (stop at the first expert that does not fit, once one is loaded) and by
        evictable room: only experts outside ``protect_current`` and
        ``predicted`` are evicted, and loading stops once the LRU is over
        capacity with nothing stale left.
        """
        if not predicted or (self._pool is None and self.lru_capacity <= 0):
            return 0
        protect = {int(i) for i in protect_current} | {int(i) for i in predicted}
        bw = bandwidth_gb_s if bandwidth_gb_s is not None else self._bw_gb_s
        budget: Optional[float] = None
        if forward_ms > 0 and bw and bw > 0:
            budget = bw * 1e9 * (forward_ms / 1000.0) * self._bw_headroom
            if inflight_bytes and inflight_bytes > 0:
                budget = max(0.0, budget - inflight_bytes)
                self.stats.inflight_bytes += int(inflight_bytes)
        loaded: List[int] = []
        for idx in (int(i) for i in predicted):
            if idx in self._lru:
                continue
            w1, w2 = self._host[idx]
            nbytes = (w1.numel() + w2.numel()) * self.dtype.itemsize
            if budget is not None:
                if nbytes > budget and loaded:
                    break
                budget -= nbytes
            # only stale entries (outside protect) make room, before the copy
            if self._pool is not None:
                self._pool.evict(self, protect, incoming=1)
            else:
                self._evict(protect, incoming=1)
            self._fill(idx)
            self.stats.predicts += 1
            loaded.append(idx)
            if self._pool is not None:
                self._pool.touch(self, idx)
                self._pool.evict(self, protect)
                if len(self._pool) > self._pool.capacity:
                    break
                continue
            self._evict(protect)
            if len(self._lru) > self.lru_capacity:
                break
        self._next_reserve = frozenset(loaded)
        return len(loaded)

    # --------------------------------------------------------------- internals
    def _side_stream(self) -> torch.cuda.Stream:
        if self._copy_stream is None:
            self._copy_stream = _copy_stream_for(self.device)
        return self._copy_stream

    def _acquire_slot(self) -> _Slot:
        w1r, w2r = self._host[0]

        def make() -> _Slot:
            buf = torch.empty(self._n1 + self._n2, dtype=self.dtype, device=self.device)
            return _Slot(buf, buf[:self._n1].view(w1r.shape), buf[self._n1:].view(w2r.shape))

        if self._pool is not None:
            slot = self._pool.acquire(make)
            if slot.buf.numel() < self._n1 + self._n2:  # freed by a layer with smaller experts
                slot = make()
                self._pool.n_slots += 1
            # a slot from another layer's cache holds that layer's layout
            slot.w1 = slot.buf[:self._n1].view(w1r.shape)
            slot.w2 = slot.buf[self._n1:].view(w2r.shape)
            return slot
        if self._free_slots:
            return self._free_slots.pop()
        self._n_slots += 1
        return make()

    def _release(self, slot: _Slot) -> None:
        """Return a slot to the free list once its last holder lets go. Its
        next copy (``_fill``, possibly on another layer's copy stream) waits
        for ``free_after`` (the events of its marked readers; if the slot was
        handed out since the last ``mark_read``, every kernel queued so far on
        the compute stream) and for ``last_copy`` (the copy that filled it,
        which nothing may have waited for if the slot was evicted unread)."""
        slot.refs -= 1
        if slot.refs > 0:
            return
        if slot.handed:
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(self.device))
            slot.reads[int(torch.cuda.current_stream(self.device).cuda_stream)] = ev
        slot.free_after = list(slot.reads.values())
        slot.reads = {}
        slot.handed = False
        slot.ready = None
        if self._pool is not None:
            self._pool.release(slot)
        else:
            self._free_slots.append(slot)

    def _release_all(self) -> None:
        for slot in set(self._slot_of.values()):
            slot.refs = 1
            self._release(slot)
        self._slot_of = {}

    def _wait_ready(self, ids: Sequence[int]) -> None:
        if self.device.type != "cuda":
            return
        stream = torch.cuda.current_stream(self.device)
        for i in ids:
            slot = self._slot_of.get(i)
            if slot is not None and slot.ready is not None:
                stream.wait_event(slot.ready)

    def _fill(self, idx: int) -> None:
        """Make expert ``idx`` resident (a miss): one async H2D into a slot."""
        w1, w2 = self._host[idx]
        nbytes = (w1.numel() + w2.numel()) * self.dtype.itemsize
        if self.device.type == "cuda":
            slot = self._acquire_slot()
            cs = self._side_stream()
            for ev_ in slot.free_after:
                cs.wait_event(ev_)
            if slot.last_copy is not None:
                cs.wait_event(slot.last_copy)
            src = self._host_buf.data_ptr() + self._host_off[idx] * self._host_buf.element_size()
            t0 = None
            if self._copy_log is not None:
                t0 = torch.cuda.Event(enable_timing=True)
                t0.record(cs)
            _capi.h2d_async(slot.buf.data_ptr(), src, nbytes, cs.cuda_stream)
            # The copy is raw hipMemcpyAsync: tell torch's device allocator
            # that the copy stream uses the slot, so a dropped slot's memory
            # is not handed out again before the copy is done, and note the
            # copy on the host pool, which is not released before it is done.
            slot.buf.record_stream(cs)
            ev = torch.cuda.Event(enable_timing=t0 is not None)
            ev.record(cs)
            self._host_pool.note_copy(cs.cuda_stream, ev)
            _note_inflight(self.device, ev)
            if t0 is not None:
                self._copy_log.append((t0, ev, nbytes))
            slot.ready = ev
            slot.last_copy = ev
            slot.refs = 1
            self._slot_of[idx] = slot
            self._lru[idx] = (slot.w1, slot.w2)
        else:
            self._lru[idx] = (w1.to(device=self.device), w2.to(device=self.device))
        self.stats.transfers_bytes += nbytes
        self.stats.misses += 1

    def _drop(self, idx: int) -> None:
        """Evict ``idx`` on the shared pool's decision."""
        if self._lru.pop(idx, None) is None:
            return
        slot = self._slot_of.pop(idx, None)
        if slot is not None:
            self._release(slot)
        self.stats.evictions += 1

    def _evict(self, hard_protect: Sequence[int], soft_protect: Sequence[int] = (),
               incoming: int = 0) -> None:
        """Evict down to ``lru_capacity`` (less ``incoming`` entries about to
        be admitted): stale entries first, then soft ones, never hard ones.
        ``lru`` picks the oldest; ``least_stale`` picks the largest routing age
        (never seen = window), oldest on ties."""
        hard = {int(i) for i in hard_protect}
        soft = {int(i) for i in soft_protect} - hard
        predictor = self._predictor
        if env.get_moe_cache_policy() == "least_stale" and predictor is not None:
            age, window = predictor._age, predictor.window

            def victim_of(cands: List[int]) -> Optional[int]:
                best, best_age = None, -1
                for i in cands:  # LRU order, oldest first: strict '>' keeps the oldest on ties
                    a = age.get(i, window)
                    if a > best_age:
                        best, best_age = i, a
                return best
        else:
            def victim_of(cands: List[int]) -> Optional[int]:
                return cands[0] if cands else None

        while len(self._lru) + incoming > self.lru_capacity:
            victim = victim_of([i for i in self._lru if i not in hard and i not in soft])
            if victim is None:
                victim = victim_of([i for i in self._lru if i in soft])
            if victim is None:
                return
            self._lru.pop(victim)
            slot = self._slot_of.pop(victim, None)
            if slot is not None:
                self._release(slot)
            self.stats.evictions += 1

    def _substitute(self, idx: int) -> Optional[int]:
        """Serve a miss with the most similar resident expert (argmax of the
        similarity row over residents, first index on ties)."""
        if self.sim_table is None or idx in self._lru:
            return None
        residents = [i for i in self._lru if i != idx]
        if not residents:
            return None
        row = self.sim_table[idx]
        cand = torch.full((self.num_experts,), float("-inf"), dtype=row.dtype)
        cand[residents] = row[residents]
        best = int(cand.argmax().item())
        self.stats.subs += 1
        self._lru[idx] = self._lru[best]
        slot = self._slot_of.get(best)
        if slot is not None:
            slot.refs += 1
            self._slot_of[idx] = slot
        return best

    def _pack(self, uniq: Sequence[int]) -> Tuple[torch.Tensor, torch.Tensor, Dict[int, int]]:
        local_index = {idx: k for k, idx in enumerate(uniq)}
        self._wait_ready(uniq)
        w1 = torch.stack([self._lru[i][0] for i in uniq], dim=0)
        w2 = torch.stack([self._lru[i][1] for i in uniq], dim=0)
        self.mark_read(uniq)  # the stacking copies are the slots' readers
        return w1, w2, local_index

    # ------------------------------------------------------------------- stats
    def report(self) -> str:
        s = self.stats.as_dict()
        return (f"offload: hit={s['hits']} miss={s['misses']} sub={s['subs']} "
                f"pred={s['predicts']} evict={s['evictions']} transfer={s['transfer_mb']:.1f}MB")


__all__ = ["ExpertOffloadCache", "ExpertPool", "OffloadStats", "Prediction"]
