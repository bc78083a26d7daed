"""RE_* environment flags read by the MoE layer and the expert cache.

Same names, defaults and parsing as the reference's getters
(reframework/env.py:14-43, :68-153), restricted to the flags the MoE path
reads. The reference's MoE code also reads four variables straight from
``os.environ`` (reframework/moe/moe_layer.py:214-218, 362, 430, 465, 471;
reframework/moe/offload_cache.py:420); they have getters here with the
defaults the reference uses at each site.
"""

from __future__ import annotations

import logging
import os


def _get(name: str, default: str) -> str:
    return os.environ.get(name, default).strip()


def _get_bool(name: str, default: bool = False) -> bool:
    raw = os.environ.get(name)
    if raw is None:
        return default
    return raw.strip().lower() in {"1", "true", "yes", "on", "y"}


def _get_int(name: str, default: int) -> int:
    raw = os.environ.get(name)
    if raw is None:
        return default
    try:
        return int(raw)
    except ValueError:
        return default


def _get_float(name: str, default: float) -> float:
    raw = os.environ.get(name)
    if raw is None:
        return default
    try:
        return float(raw)
    except ValueError:
        return default


def get_log_level() -> int:
    return getattr(logging, _get("RE_LOG_LEVEL", "INFO").upper(), logging.INFO)


# --- MoE host offload ---------------------------------------------------------
def get_moe_offload_enabled() -> bool:
    return _get_bool("RE_MOE_OFFLOAD", True)


def get_moe_cache_size() -> int:
    """Resident expert slots per layer; 0 = sized by the engine from free HBM."""
    return _get_int("RE_MOE_CACHE_SIZE", 0)


def get_moe_cache_ratio() -> float:
    return _get_float("RE_MOE_CACHE_RATIO", 0.5)


def get_moe_substitute() -> bool:
    return _get_bool("RE_MOE_SUBSTITUTE", True)


def get_moe_predict() -> bool:
    return _get_bool("RE_MOE_PREDICT", True)


def get_moe_predict_window() -> int:
    return _get_int("RE_MOE_PREDICT_WINDOW", 32)


def get_moe_predict_headroom() -> float:
    return _get_float("RE_MOE_PREDICT_HEADROOM", 0.9)


def get_moe_prefill_overlap() -> bool:
    return _get_bool("RE_MOE_PREFILL_OVERLAP", True)


def get_moe_cache_policy() -> str:
    """``lru`` (default) or ``least_stale``; any other value means ``lru``."""
    p = _get("RE_CACHE_POLICY", "lru").lower()
    return p if p in ("lru", "least_stale") else "lru"


def get_moe_cpu_split() -> bool:
    return _get_bool("RE_MOE_CPU_SPLIT", False)


def get_moe_split_copy_depth() -> int:
    """RE_MOE_SPLIT_COPY_DEPTH (not in the reference): host->device expert
    copies the CPU/GPU split forward keeps in flight per device when it makes
    the experts it computed on the host resident for later steps (the
    reference loads every one, moe_layer.py:601). 0 loads none."""
    return max(0, _get_int("RE_MOE_SPLIT_COPY_DEPTH", 2))


def get_moe_split_int8() -> bool:
    """RE_MOE_SPLIT_INT8 (not in the reference): 1 runs the CPU/GPU split's
    host half on the per-tensor int8 bank with the reference's int8 numerics
    (fused_experts_cpu_int8, fused.py:140-197), half the host bytes per
    expert; 0 (default) multiplies the staged 16-bit weights with the device
    kernels' numerics."""
    return _get_bool("RE_MOE_SPLIT_INT8", False)


def get_moe_shuttle_steps() -> int:
    return _get_int("RE_MOE_SHUTTLE_STEPS", 0)


# --- knobs the reference reads directly from os.environ -----------------------
def get_chunk_size(default: int = 0) -> int:
    """RE_CHUNK_SIZE: experts per chunk of the exact streaming offload path.
    FusedMoE.forward treats unset as 0 (path off); _forward_streaming itself
    defaults to 8 (moe_layer.py:362, 465)."""
    return int(os.environ.get("RE_CHUNK_SIZE", str(default)))


def get_max_pack(default: int) -> int:
    """RE_MAX_PACK: experts kept per offload step (2 in FusedMoE._banks,
    4 in ExpertOffloadCache.cpu_banks)."""
    return int(os.environ.get("RE_MAX_PACK", str(default)))


def get_entropy_k() -> bool:
    return os.environ.get("RE_ENTROPY_K", "").lower() in {"1", "true", "yes", "on"}


def get_entropy_k_min(default: int) -> int:
    return int(os.environ.get("RE_ENTROPY_K_MIN") or default)


__all__ = [
    "get_log_level",
    "get_moe_offload_enabled",
    "get_moe_cache_size",
    "get_moe_cache_ratio",
    "get_moe_substitute",
    "get_moe_predict",
    "get_moe_predict_window",
    "get_moe_predict_headroom",
    "get_moe_prefill_overlap",
    "get_moe_cache_policy",
    "get_moe_cpu_split",
    "get_moe_split_copy_depth",
    "get_moe_shuttle_steps",
    "get_chunk_size",
    "get_max_pack",
    "get_entropy_k",
    "get_entropy_k_min",
]
