"""ctypes binding of libmoe355.so (declared in include/moe355.h).

The library is built in-tree (``make -C reframework_amd/csrc``) and loaded from
this package directory. Nothing here computes: every function forwards raw
device pointers and a HIP stream to the C ABI and turns a non-zero status into
:class:`MoeLibError`. There is deliberately no fallback: if the library is
missing, :func:`lib` raises, so a GPU run can never silently take another path.
"""

from __future__ import annotations

import ctypes
import os
import re
import threading
from collections import OrderedDict
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

LIB_NAME = "libmoe355.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                           "include", "moe355.h")

F32, BF16, F16 = 0, 1, 2
ACT_CODES = {"silu": 0, "gelu": 1, "gelu_tanh": 2}
PATH_MFMA_TILED, PATH_MFMA_SKINNY, PATH_SIMT, PATH_MFMA_TILED128 = 0, 1, 2, 4
MAX_EXPERTS = 256
STATIC_SCRATCH_BYTES = 64 << 20

_DTYPE_CODES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}


class MoeLibError(RuntimeError):
    """A libmoe355 entry point returned a non-zero status."""


class Plan(ctypes.Structure):
    """Mirror of ``moe355_plan``."""

    _fields_ = [
        ("path", ctypes.c_int),
        ("tile_rows", ctypes.c_int),
        ("max_tiles", ctypes.c_int),
        ("down_splits", ctypes.c_int),
        ("rows", ctypes.c_int),
        ("n_blocks", ctypes.c_int),
        ("T", ctypes.c_int),
        ("H", ctypes.c_int),
        ("I", ctypes.c_int),
        ("E", ctypes.c_int),
        ("K", ctypes.c_int),
        ("dtype", ctypes.c_int),
        ("workspace_bytes", ctypes.c_size_t),
        ("off_block_counts", ctypes.c_size_t),
        ("off_offsets", ctypes.c_size_t),
        ("off_slot_to_row", ctypes.c_size_t),
        ("off_row_src", ctypes.c_size_t),
        ("off_tile_map", ctypes.c_size_t),
        ("off_inter", ctypes.c_size_t),
        ("off_y", ctypes.c_size_t),
        ("off_part", ctypes.c_size_t),
    ]


_I, _Z, _P = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p
_PP = ctypes.POINTER(ctypes.c_void_p)
_PI32 = ctypes.POINTER(ctypes.c_int32)
_PPLAN = ctypes.POINTER(Plan)

# name -> (restype, argtypes)
_SIGNATURES: Dict[str, Tuple[object, List[object]]] = {
    "moe355_version": (_I, []),
    "moe355_last_error": (ctypes.c_char_p, []),
    "moe355_router_topk": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P]),
    "moe355_router_topk_ld": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _I,
                                   _P]),
    "moe355_topk_from_logits": (_I, [_P, _I, _I, _I, _I, _P, _P, _P]),
    "moe355_add_rmsnorm": (_I, [_P, _P, _P, _P, _P, _I, ctypes.c_float, _I, _I, _I, _P, _P]),
    "moe355_add_rmsnorm_router_topk": (_I, [_P, _P, _P, _P, _P, _I, ctypes.c_float, _P, _P, _I,
                                            _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P]),
    "moe355_make_plan": (_I, [_I, _I, _I, _I, _I, _I, _PPLAN]),
    "moe355_make_plan_path": (_I, [_I, _I, _I, _I, _I, _I, _I, _PPLAN]),
    "moe355_permute": (_I, [_PPLAN, _P, _I, _PI32, _I, _P, _P]),
    "moe355_gate_up": (_I, [_PPLAN, _P, _PP, _I, _P, _P]),
    "moe355_down": (_I, [_PPLAN, _PP, _P, _P]),
    "moe355_combine": (_I, [_PPLAN, _P, _P, _I, _P, _P]),
    "moe355_fused_experts": (_I, [_P, _PP, _PP, _P, _P, _I, _PI32, _I, _I, _I, _I, _I, _I, _I,
                                  _I, _P, _I, _P, _Z, _P]),
    "moe355_fused_experts_static": (_I, [_P, _PP, _PP, _P, _P, _I, _PI32, _I, _I, _I, _I, _I,
                                         _I, _I, _I, _P, _I, _P]),
    "moe355_cast_f32": (_I, [_P, _P, _Z, _I, _P]),
    "moe355_h2d_async": (_I, [_P, _P, _Z, _P]),
    "moe355_host_staging_alloc": (_I, [_Z, ctypes.POINTER(ctypes.c_void_p)]),
    "moe355_host_staging_free": (_I, [_P]),
    "moe355_copy_to_host": (_I, [_P, _P, _Z, _P]),
    "moe355_copy_to_host_multi": (_I, [_P, _I, _P, _P, _P, _P]),
    "moe355_merge_host_f32": (_I, [_P, _P, _Z, _I, _P, _P]),
}

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()

# libmoe355_host.so (include/moe355_host.h): the host half of the CPU/GPU
# split forward, plain C++ on the host cores.
HOST_LIB_NAME = "libmoe355_host.so"
HOST_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), HOST_LIB_NAME)
HOST_HEADER_PATH = os.path.join(os.path.dirname(HEADER_PATH), "moe355_host.h")
_HOST_SIGNATURES: Dict[str, Tuple[object, List[object]]] = {
    "moe355_host_version": (_I, []),
    "moe355_host_last_error": (ctypes.c_char_p, []),
    "moe355_host_experts": (_I, [_P, _I, _I, _I, _I, _I, _PP, _PP, _P, _P, _P, _I, _I, _P]),
    "moe355_host_quantize_int8": (_I, [_P, _I, _I, _I, _P, _P, _P, _I]),
    "moe355_host_int8_row_sums": (_I, [_P, _I, _I, _P, _I]),
    "moe355_host_experts_int8": (_I, [_P, _I, _I, _I, _I, _I, _PP, _PP, _P, _P, _PP, _PP, _P, _P,
                                      _P, _I, _I, _P]),
}
_host_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load libmoe355.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise MoeLibError(
                        f"{LIB_NAME} is not built at {LIB_PATH}; run "
                        "`make -C reframework_amd/csrc` (or __graft_entry__.build())"
                    )
                handle = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in _SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def host_lib() -> ctypes.CDLL:
    """Load libmoe355_host.so once; raise if it has not been built."""
    global _host_lib
    if _host_lib is None:
        with _lock:
            if _host_lib is None:
                if not os.path.exists(HOST_LIB_PATH):
                    raise MoeLibError(
                        f"{HOST_LIB_NAME} is not built at {HOST_LIB_PATH}; run "
                        "`make -C reframework_amd/csrc` (or __graft_entry__.build())"
                    )
                handle = ctypes.CDLL(HOST_LIB_PATH)
                for name, (res, args) in _HOST_SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _host_lib = handle
    return _host_lib


def header_symbols(path: str = HEADER_PATH) -> List[str]:
    """Entry points declared in include/moe355.h."""
    with open(path, "r", encoding="utf-8") as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(moe355_[a-z0-9_]+)\s*\(", text)))


def _check(name: str, rc: int) -> None:
    if rc != 0:
        msg = lib().moe355_last_error()
        raise MoeLibError(f"{name} failed (status {rc}): {msg.decode() if msg else ''}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"libmoe355 handles float32/bfloat16/float16, not {dtype}") from None


def act_code(activation: str) -> int:
    try:
        return ACT_CODES[activation]
    except KeyError:
        raise ValueError(
            f"unknown gated activation {activation!r}; known: {tuple(ACT_CODES)}"
        ) from None


def stream_handle(device: torch.device, stream: Optional[torch.cuda.Stream] = None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream(device)
    return int(s.cuda_stream)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else int(t.data_ptr())


# Host arrays of expert pointers, keyed by their contents: a decode step hands
# the same tables to every call, and building a ctypes array per call cost
# tens of microseconds of host time per 64-expert bank (more than the router
# kernels at decode sizes). A table holds only the pointer values, so a cached
# one is exactly the array the call would have built.
_TABLES: "OrderedDict[Tuple[int, ...], ctypes.Array]" = OrderedDict()
_TABLES_MAX = 256


def _ptr_table(ptrs: Sequence[int]):
    """(array to pass for a pointer-table argument, keep-alive) of ``ptrs``."""
    key = tuple(ptrs)
    arr = _TABLES.get(key)
    if arr is None:
        arr = (ctypes.c_void_p * len(key))(*key)
        with _lock:
            _TABLES[key] = arr
            if len(_TABLES) > _TABLES_MAX:
                _TABLES.popitem(last=False)
    return arr, arr


# ------------------------------------------------------------------ wrappers
def version() -> int:
    return int(lib().moe355_version())


_PLANS: "OrderedDict[Tuple[int, ...], Plan]" = OrderedDict()


def make_plan(T: int, H: int, I: int, E: int, K: int, dtype: int, path: int = -1) -> Plan:
    """Execution plan of a fused_experts call; ``path`` forces a kernel family
    (PATH_*), -1 lets the library choose. Plans depend on the shape (and the
    CU count, which one kind of device shares), so they are cached; the entry
    points only read them. Do not modify a returned plan."""
    key = (T, H, I, E, K, dtype, path)
    plan = _PLANS.get(key)
    if plan is not None:
        return plan
    plan = Plan()
    if path < 0:
        _check("moe355_make_plan", lib().moe355_make_plan(T, H, I, E, K, dtype, ctypes.byref(plan)))
    else:
        _check("moe355_make_plan_path",
               lib().moe355_make_plan_path(T, H, I, E, K, dtype, path, ctypes.byref(plan)))
    with _lock:
        _PLANS[key] = plan
        if len(_PLANS) > 1024:
            _PLANS.popitem(last=False)
    return plan


def router_topk(x: torch.Tensor, gate: torch.Tensor, bias: Optional[torch.Tensor], K: int,
                renormalize: bool, round_logits: bool, entropy_k_min: int,
                topk_w: torch.Tensor, topk_ids: torch.Tensor,
                logits_out: Optional[torch.Tensor] = None, stream: Optional[int] = None) -> None:
    """Routes x into topk_w / topk_ids of shape [T, ld] (ld >= K, row-major):
    the first K columns of each row; columns K.. are left as they are."""
    T, H = x.shape
    E = gate.shape[0]
    ld = topk_w.shape[1] if topk_w.dim() == 2 else K
    if topk_ids.dim() == 2 and topk_ids.shape[1] != ld:
        raise ValueError(f"topk_w and topk_ids rows differ: {ld} vs {topk_ids.shape[1]}")
    s = stream if stream is not None else stream_handle(x.device)
    _check("moe355_router_topk_ld", lib().moe355_router_topk_ld(
        _ptr(x), _ptr(gate), _ptr(bias), T, H, E, K, dtype_code(x.dtype), int(renormalize),
        int(round_logits), int(entropy_k_min), _ptr(logits_out), _ptr(topk_w), _ptr(topk_ids), ld,
        s))


def topk_from_logits(logits: torch.Tensor, K: int, renormalize: bool, topk_w: torch.Tensor,
                     topk_ids: torch.Tensor, stream: Optional[int] = None) -> None:
    T, E = logits.shape
    s = stream if stream is not None else stream_handle(logits.device)
    _check("moe355_topk_from_logits", lib().moe355_topk_from_logits(
        _ptr(logits), T, E, K, int(renormalize), _ptr(topk_w), _ptr(topk_ids), s))


def add_rmsnorm(x: torch.Tensor, residual: Optional[torch.Tensor],
                residual_out: Optional[torch.Tensor], weight: torch.Tensor,
                bias: Optional[torch.Tensor], eps: float, normed_out: torch.Tensor,
                stream: Optional[int] = None) -> None:
    T, H = x.shape
    s = stream if stream is not None else stream_handle(x.device)
    _check("moe355_add_rmsnorm", lib().moe355_add_rmsnorm(
        _ptr(x), _ptr(residual), _ptr(residual_out), _ptr(weight), _ptr(bias),
        dtype_code(weight.dtype), float(eps), T, H, dtype_code(x.dtype), _ptr(normed_out), s))


def add_rmsnorm_router_topk(x: torch.Tensor, residual: Optional[torch.Tensor],
                            residual_out: Optional[torch.Tensor], norm_weight: torch.Tensor,
                            norm_bias: Optional[torch.Tensor], eps: float, gate: torch.Tensor,
                            router_bias: Optional[torch.Tensor], K: int, renormalize: bool,
                            round_logits: bool, normed_out: torch.Tensor, topk_w: torch.Tensor,
                            topk_ids: torch.Tensor, stream: Optional[int] = None,
                            logits_out: Optional[torch.Tensor] = None) -> None:
    T, H = x.shape
    E = gate.shape[0]
    s = stream if stream is not None else stream_handle(x.device)
    _check("moe355_add_rmsnorm_router_topk", lib().moe355_add_rmsnorm_router_topk(
        _ptr(x), _ptr(residual), _ptr(residual_out), _ptr(norm_weight), _ptr(norm_bias),
        dtype_code(norm_weight.dtype), float(eps), _ptr(gate), _ptr(router_bias), T, H, E, K,
        dtype_code(x.dtype), int(renormalize), int(round_logits), _ptr(normed_out),
        _ptr(logits_out), _ptr(topk_w), _ptr(topk_ids), s))


def permute(plan: Plan, topk_ids: torch.Tensor, workspace: torch.Tensor,
            expert_map: Optional[Sequence[int]] = None, stream: Optional[int] = None) -> None:
    s = stream if stream is not None else stream_handle(topk_ids.device)
    if expert_map:
        m = (ctypes.c_int32 * len(expert_map))(*expert_map)
        mp, mlen = ctypes.cast(m, _PI32), len(expert_map)
    else:
        mp, mlen = None, 0
    _check("moe355_permute", lib().moe355_permute(
        ctypes.byref(plan), _ptr(topk_ids), int(topk_ids.dtype == torch.int64), mp, mlen,
        _ptr(workspace), s))


def gate_up(plan: Plan, x: torch.Tensor, w1_ptrs: Sequence[int], act: int,
            workspace: torch.Tensor, stream: Optional[int] = None) -> None:
    s = stream if stream is not None else stream_handle(x.device)
    tab, _keep = _ptr_table(w1_ptrs)
    _check("moe355_gate_up", lib().moe355_gate_up(ctypes.byref(plan), _ptr(x), tab, act,
                                                  _ptr(workspace), s))


def down(plan: Plan, w2_ptrs: Sequence[int], workspace: torch.Tensor,
         stream: Optional[int] = None) -> None:
    s = stream if stream is not None else stream_handle(workspace.device)
    tab, _keep = _ptr_table(w2_ptrs)
    _check("moe355_down", lib().moe355_down(ctypes.byref(plan), tab, _ptr(workspace), s))


def combine(plan: Plan, topk_w: torch.Tensor, out: torch.Tensor, accumulate_f32: bool,
            workspace: torch.Tensor, stream: Optional[int] = None) -> None:
    s = stream if stream is not None else stream_handle(out.device)
    _check("moe355_combine", lib().moe355_combine(ctypes.byref(plan), _ptr(topk_w), _ptr(out),
                                                  int(accumulate_f32), _ptr(workspace), s))


def fused_experts(x: torch.Tensor, w1_ptrs: Sequence[int], w2_ptrs: Sequence[int], I: int,
                  topk_w: torch.Tensor, topk_ids: torch.Tensor, act: int, out: torch.Tensor,
                  workspace: torch.Tensor, expert_map: Optional[Sequence[int]] = None,
                  accumulate_f32: bool = False, stream: Optional[int] = None,
                  plan: Optional[Plan] = None) -> None:
    """The whole routed-expert computation. With a ``plan`` whose kernel family
    was forced (make_plan(..., path)), the four stages run one by one on that
    plan; otherwise one moe355_fused_experts call plans for itself."""
    T, H = x.shape
    K = topk_ids.shape[1]
    E = len(w1_ptrs)
    s = stream if stream is not None else stream_handle(x.device)
    if plan is not None and plan.path != make_plan(T, H, I, E, K, dtype_code(x.dtype)).path:
        permute(plan, topk_ids, workspace, expert_map=expert_map, stream=s)
        gate_up(plan, x, w1_ptrs, act, workspace, stream=s)
        down(plan, w2_ptrs, workspace, stream=s)
        combine(plan, topk_w, out, accumulate_f32, workspace, stream=s)
        return
    t1, _k1 = _ptr_table(w1_ptrs)
    t2, _k2 = _ptr_table(w2_ptrs)
    if expert_map:
        m = (ctypes.c_int32 * len(expert_map))(*expert_map)
        mp, mlen = ctypes.cast(m, _PI32), len(expert_map)
    else:
        mp, mlen = None, 0
    _check("moe355_fused_experts", lib().moe355_fused_experts(
        _ptr(x), t1, t2, _ptr(topk_w), _ptr(topk_ids), int(topk_ids.dtype == torch.int64), mp,
        mlen, T, H, I, E, K, dtype_code(x.dtype), act, _ptr(out), int(accumulate_f32),
        _ptr(workspace), workspace.numel() * workspace.element_size(), s))


def fused_experts_static(x: torch.Tensor, w1_ptrs: Sequence[int], w2_ptrs: Sequence[int], I: int,
                         topk_w: torch.Tensor, topk_ids: torch.Tensor, act: int,
                         out: torch.Tensor, expert_map: Optional[Sequence[int]] = None,
                         accumulate_f32: bool = False, stream: Optional[int] = None) -> None:
    """moe355_fused_experts_static: the routed-expert computation on the
    library's static scratch (no workspace; see include/moe355.h for its
    size limit and the rule that calls on one device must not overlap)."""
    T, H = x.shape
    K = topk_ids.shape[1]
    E = len(w1_ptrs)
    s = stream if stream is not None else stream_handle(x.device)
    t1, _k1 = _ptr_table(w1_ptrs)
    t2, _k2 = _ptr_table(w2_ptrs)
    if expert_map:
        m = (ctypes.c_int32 * len(expert_map))(*expert_map)
        mp, mlen = ctypes.cast(m, _PI32), len(expert_map)
    else:
        mp, mlen = None, 0
    _check("moe355_fused_experts_static", lib().moe355_fused_experts_static(
        _ptr(x), t1, t2, _ptr(topk_w), _ptr(topk_ids), int(topk_ids.dtype == torch.int64), mp,
        mlen, T, H, I, E, K, dtype_code(x.dtype), act, _ptr(out), int(accumulate_f32), s))


def cast_f32(src: torch.Tensor, dst: torch.Tensor, stream: Optional[int] = None) -> None:
    s = stream if stream is not None else stream_handle(src.device)
    _check("moe355_cast_f32", lib().moe355_cast_f32(_ptr(src), _ptr(dst), src.numel(),
                                                    dtype_code(dst.dtype), s))


def h2d_async(dst_ptr: int, src_ptr: int, nbytes: int, stream: int) -> None:
    _check("moe355_h2d_async", lib().moe355_h2d_async(dst_ptr, src_ptr, nbytes, stream))


def copy_to_host(host_dst: int, src: torch.Tensor, nbytes: int,
                 stream: Optional[int] = None) -> None:
    """moe355_copy_to_host: ``nbytes`` of ``src`` into mapped pinned host
    memory at address ``host_dst`` by a kernel on the stream."""
    s = stream if stream is not None else stream_handle(src.device)
    _check("moe355_copy_to_host", lib().moe355_copy_to_host(host_dst, _ptr(src), nbytes, s))


def copy_to_host_multi(host_dst: int, regions, stream: Optional[int] = None) -> None:
    """moe355_copy_to_host_multi: ``regions`` = [(src tensor, byte offset in
    the host buffer, bytes)] (at most 4), copied by one kernel on the stream."""
    n = len(regions)
    if n == 0:
        return
    s = stream if stream is not None else stream_handle(regions[0][0].device)
    srcs = (ctypes.c_void_p * n)(*[int(t.data_ptr()) for t, _, _ in regions])
    offs = (ctypes.c_size_t * n)(*[int(o) for _, o, _ in regions])
    sizes = (ctypes.c_size_t * n)(*[int(b) for _, _, b in regions])
    _check("moe355_copy_to_host_multi",
           lib().moe355_copy_to_host_multi(host_dst, n, srcs, offs, sizes, s))


def merge_host_f32(acc: torch.Tensor, host_src: int, out: torch.Tensor,
                   stream: Optional[int] = None) -> None:
    """moe355_merge_host_f32: out = (out dtype) (acc + the fp32 host array at
    address ``host_src``), the host array read by the kernel."""
    s = stream if stream is not None else stream_handle(acc.device)
    _check("moe355_merge_host_f32", lib().moe355_merge_host_f32(
        _ptr(acc), host_src, acc.numel(), dtype_code(out.dtype), _ptr(out), s))


class HostStaging:
    """One mapped, coherent pinned host buffer (moe355_host_staging_alloc)
    that kernels on one stream read and write directly: the CPU/GPU split
    forward's routing, hidden states and host-half result travel through it.
    Calls on one stream are ordered, so a step may reuse it once the previous
    step's kernels that touch it are queued before its own. Kept for the life
    of the process (a queued kernel may still read it when a caller drops
    it)."""

    CAPACITY = 8 << 20

    def __init__(self, nbytes: int = CAPACITY) -> None:
        p = ctypes.c_void_p()
        _check("moe355_host_staging_alloc", lib().moe355_host_staging_alloc(nbytes,
                                                                            ctypes.byref(p)))
        self.ptr = int(p.value)
        self.nbytes = nbytes
        self._bytes = (ctypes.c_uint8 * nbytes).from_address(self.ptr)

    def array(self, offset: int, dtype, count: int):
        """numpy view of ``count`` elements of ``dtype`` at byte ``offset``."""
        import numpy as np

        return np.frombuffer(self._bytes, dtype=dtype, count=count, offset=offset)


_STAGING: Dict[Tuple[int, int], HostStaging] = {}


def staging(device: torch.device, stream: int) -> HostStaging:
    """The staging buffer of (device, stream), created on first use."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    buf = _STAGING.get(key)
    if buf is None:
        with torch.cuda.device(key[0]):
            buf = HostStaging()
        _STAGING[key] = buf
    return buf


def host_experts(x: torch.Tensor, w1: Sequence[torch.Tensor], w2: Sequence[torch.Tensor],
                 slot_offsets, slot_tokens, slot_weights, act: int, out: torch.Tensor,
                 n_threads: int = 0) -> None:
    """moe355_host_experts: ``out`` (host fp32 [T,H]) += the experts given
    (host tensors [2I,H] / [H,I] in x's dtype) over their slots. The slot
    arrays are contiguous int32 / int32 / float32 numpy arrays."""
    if x.device.type != "cpu" or out.device.type != "cpu" or out.dtype != torch.float32:
        raise ValueError("host_experts takes host tensors and an fp32 host output")
    T, H = x.shape
    I = w2[0].shape[1] if len(w2) else 1
    for a, b in zip(w1, w2):
        if a.device.type != "cpu" or b.device.type != "cpu" or a.dtype != x.dtype or \
                b.dtype != x.dtype or tuple(a.shape) != (2 * I, H) or tuple(b.shape) != (H, I) or \
                not a.is_contiguous() or not b.is_contiguous():
            raise ValueError("host expert weights must be contiguous host [2I,H] / [H,I] "
                             "tensors of x's dtype")
    t1, _k1 = _ptr_table([int(a.data_ptr()) for a in w1])
    t2, _k2 = _ptr_table([int(b.data_ptr()) for b in w2])
    rc = host_lib().moe355_host_experts(
        _ptr(x), T, H, I, dtype_code(x.dtype), len(w1), t1, t2, slot_offsets.ctypes.data,
        slot_tokens.ctypes.data, slot_weights.ctypes.data, int(act), int(n_threads), _ptr(out))
    if rc != 0:
        msg = host_lib().moe355_host_last_error()
        raise MoeLibError(f"moe355_host_experts failed (status {rc}): "
                          f"{msg.decode() if msg else ''}")


def _host_check(name: str, rc: int) -> None:
    if rc != 0:
        msg = host_lib().moe355_host_last_error()
        raise MoeLibError(f"{name} failed (status {rc}): {msg.decode() if msg else ''}")


def host_quantize_int8(w: torch.Tensor, n_threads: int = 0):
    """moe355_host_quantize_int8 on a contiguous host [rows, cols] weight:
    (int8 codes [rows, cols], scale (float), int32 row code sums [rows])."""
    if w.device.type != "cpu" or w.dim() != 2 or not w.is_contiguous():
        raise ValueError("host_quantize_int8 takes a contiguous host [rows, cols] tensor")
    rows, cols = w.shape
    q = torch.empty((rows, cols), dtype=torch.int8)
    rs = torch.empty((rows,), dtype=torch.int32)
    scale = ctypes.c_float(0.0)
    _host_check("moe355_host_quantize_int8", host_lib().moe355_host_quantize_int8(
        _ptr(w), rows, cols, dtype_code(w.dtype), _ptr(q), ctypes.addressof(scale), _ptr(rs),
        int(n_threads)))
    return q, float(scale.value), rs


def host_int8_row_sums(q: torch.Tensor, n_threads: int = 0) -> torch.Tensor:
    """moe355_host_int8_row_sums: int32 sums of the rows of a contiguous host
    int8 [rows, cols] matrix of codes."""
    if q.device.type != "cpu" or q.dtype != torch.int8 or q.dim() != 2 or not q.is_contiguous():
        raise ValueError("host_int8_row_sums takes a contiguous host int8 [rows, cols] tensor")
    rs = torch.empty((q.shape[0],), dtype=torch.int32)
    _host_check("moe355_host_int8_row_sums", host_lib().moe355_host_int8_row_sums(
        _ptr(q), q.shape[0], q.shape[1], _ptr(rs), int(n_threads)))
    return rs


def host_experts_int8(x: torch.Tensor, w1q: Sequence[torch.Tensor], w2q: Sequence[torch.Tensor],
                      s1: Sequence[float], s2: Sequence[float], rs1: Sequence[torch.Tensor],
                      rs2: Sequence[torch.Tensor], slot_offsets, slot_tokens, slot_weights,
                      act: int, out: torch.Tensor, n_threads: int = 0) -> None:
    """moe355_host_experts_int8: ``out`` (host fp32 [T,H]) += the int8
    experts given (codes [2I,H] / [H,I], their scales and row code sums from
    host_quantize_int8) over their slots, with the reference's int8 numerics."""
    if x.device.type != "cpu" or out.device.type != "cpu" or out.dtype != torch.float32:
        raise ValueError("host_experts_int8 takes host tensors and an fp32 host output")
    T, H = x.shape
    n = len(w1q)
    if not (len(w2q) == len(s1) == len(s2) == len(rs1) == len(rs2) == n):
        raise ValueError("host_experts_int8: per-expert lists differ in length")
    I = w2q[0].shape[1] if n else 1
    for a, b, r1, r2 in zip(w1q, w2q, rs1, rs2):
        if a.dtype != torch.int8 or b.dtype != torch.int8 or tuple(a.shape) != (2 * I, H) or \
                tuple(b.shape) != (H, I) or not a.is_contiguous() or not b.is_contiguous() or \
                r1.dtype != torch.int32 or r2.dtype != torch.int32 or \
                tuple(r1.shape) != (2 * I,) or tuple(r2.shape) != (H,) or \
                a.device.type != "cpu" or b.device.type != "cpu":
            raise ValueError("int8 host experts must be contiguous host int8 [2I,H] / [H,I] codes "
                             "with int32 row sums [2I] / [H]")
    t1, _k1 = _ptr_table([int(a.data_ptr()) for a in w1q])
    t2, _k2 = _ptr_table([int(b.data_ptr()) for b in w2q])
    r1t, _k3 = _ptr_table([int(r.data_ptr()) for r in rs1])
    r2t, _k4 = _ptr_table([int(r.data_ptr()) for r in rs2])
    sc1 = np.ascontiguousarray(np.asarray(s1, dtype=np.float32).reshape(-1)) if n else \
        np.zeros(1, np.float32)
    sc2 = np.ascontiguousarray(np.asarray(s2, dtype=np.float32).reshape(-1)) if n else \
        np.zeros(1, np.float32)
    _host_check("moe355_host_experts_int8", host_lib().moe355_host_experts_int8(
        _ptr(x), T, H, I, dtype_code(x.dtype), n, t1, t2, sc1.ctypes.data, sc2.ctypes.data,
        r1t, r2t, slot_offsets.ctypes.data, slot_tokens.ctypes.data, slot_weights.ctypes.data,
        int(act), int(n_threads), _ptr(out)))


# ------------------------------------------------------------------ workspace
class WorkspacePool:
    """One growable device byte buffer per (device, stream).

    libmoe355 allocates nothing; the host hands it this buffer. Calls on one
    stream are ordered, so reusing the buffer across calls is safe; calls on
    different streams get different buffers.
    """

    def __init__(self) -> None:
        self._bufs: Dict[Tuple[int, int], torch.Tensor] = {}

    def get(self, device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
        key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            self._bufs.pop(key, None)
            buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf


workspaces = WorkspacePool()
