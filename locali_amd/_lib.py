"""ctypes binding of liblocali_amd.so (include/locali_core.h, include/locali_planner.h,
include/locali_moe.h).

The library is built in-tree by ``python -m locali_amd.build``. There is no
CPU or eager fallback: if the library is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("LOCALI_AMD_LIB", Path(__file__).resolve().parent / "liblocali_amd.so"))

DT_F32, DT_F16, DT_BF16 = 0, 1, 2
SCORE_SQRTSOFTPLUS, SCORE_SIGMOID, SCORE_SOFTMAX = 0, 1, 2
COMBINE_ROUNDED, COMBINE_FP32 = 0, 1


class LocaliError(RuntimeError):
    pass


class CacheResult(ctypes.Structure):
    _fields_ = [
        ("key", ctypes.c_int32),
        ("slot", ctypes.c_int32),
        ("evicted_key", ctypes.c_int32),
        ("hit", ctypes.c_uint8),
        ("placed", ctypes.c_uint8),
    ]


class DPlanStats(ctypes.Structure):
    _fields_ = [
        ("hits", ctypes.c_uint64),
        ("misses", ctypes.c_uint64),
        ("evictions", ctypes.c_uint64),
        ("calls", ctypes.c_uint64),
        ("error", ctypes.c_int32),
        ("probation", ctypes.c_int32),
        ("protected_", ctypes.c_int32),
        ("free_slots", ctypes.c_int32),
        ("last_keys", ctypes.c_int32),
        ("last_misses", ctypes.c_int32),
        ("prefetched", ctypes.c_uint64),
        ("prefetch_used", ctypes.c_uint64),
        ("prefetch_wasted", ctypes.c_uint64),
    ]


class QProj(ctypes.Structure):
    _fields_ = [
        ("weight", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("biases", ctypes.c_void_p),
        ("bits", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("rows", ctypes.c_int32),
        ("cols", ctypes.c_int32),
        ("meta_dtype", ctypes.c_int32),
        ("n_slots", ctypes.c_int32),
    ]


class FillPiece(ctypes.Structure):
    _fields_ = [("dst", ctypes.c_void_p), ("src_host", ctypes.c_void_p), ("bytes", ctypes.c_size_t)]


class ExpertArena(ctypes.Structure):
    _fields_ = [("gate", QProj), ("up", QProj), ("down", QProj)]


class Router(ctypes.Structure):
    _fields_ = [
        ("weight", ctypes.c_void_p),
        ("weight_dtype", ctypes.c_int32),
        ("n_experts", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("score_func", ctypes.c_int32),
        ("norm_topk", ctypes.c_int32),
        ("routed_scale", ctypes.c_float),
        ("score_bias", ctypes.c_void_p),
        ("tid2eid", ctypes.c_void_p),
        ("vocab", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int32
_SZ = ctypes.c_size_t
_F = ctypes.c_float

_SIGNATURES = {
    # scheduler (locali_core.h)
    "locali_cache_create": ([_I, _I, _I], ctypes.c_void_p),
    "locali_cache_create_policy": ([_I, _I, _I, _I], ctypes.c_void_p),
    "locali_cache_destroy": ([_P], None),
    "locali_cache_note_token": ([_P], None),
    "locali_cache_plan": ([_P, ctypes.POINTER(ctypes.c_int32), _SZ, ctypes.POINTER(ctypes.c_int32),
                           _SZ, ctypes.c_int, ctypes.POINTER(CacheResult)], ctypes.c_int),
    "locali_cache_plan_each": ([_P, ctypes.POINTER(ctypes.c_int32), _SZ, ctypes.POINTER(ctypes.c_int32),
                                _SZ, ctypes.c_int, ctypes.POINTER(CacheResult)], ctypes.c_int),
    "locali_cache_peek": ([_P, _I], _I),
    "locali_cache_probation_size": ([_P], _I),
    "locali_cache_protected_size": ([_P], _I),
    "locali_dplan_state_bytes": ([_I, _I, _I], _SZ),
    "locali_dplan_lds_bytes": ([_I, _I, _I], _SZ),
    "locali_dplan_init": ([_P, _SZ, _I, _I, _I, _I, _I, _P], ctypes.c_int),
    "locali_dplan_plan": ([_P, _I, _I, _I, _I, _P, _I, _I, _I, _I, _I, _P, _P], ctypes.c_int),
    "locali_dplan_fill": ([_P, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t), _I, _P, _I, _I,
                           _I, _P], ctypes.c_int),
    "locali_dplan_plan_fill": ([_P, _I, _I, _I, _I, _P, _I, _I, _I, _I, _I, _P, ctypes.POINTER(ctypes.c_void_p),
                                ctypes.POINTER(ctypes.c_size_t), _I, _P, _P], ctypes.c_int),
    "locali_moe_stream_read": ([_P, _SZ, _P, _I, _P], ctypes.c_int),
    "locali_dplan_prefetch": ([_P, _I, _I, _I, _I, _P, _P, _I, _I, _I, _I, _I, ctypes.POINTER(ctypes.c_void_p),
                               ctypes.POINTER(ctypes.c_size_t), _I, _P, _P], ctypes.c_int),
    "locali_dplan_host_view": ([ctypes.POINTER(ctypes.c_void_p), _I, ctypes.POINTER(ctypes.c_uint64)],
                               ctypes.c_int),
    "locali_dplan_read": ([_P, ctypes.POINTER(DPlanStats), ctypes.POINTER(CacheResult), _I, _P], ctypes.c_int),
    "locali_dplan_peek": ([_P, _I, _P], _I),
    # GPU (locali_moe.h)
    "locali_moe_workspace_bytes": ([_I, _I, _I, _I, _I, _I], _SZ),
    "locali_moe_router": ([ctypes.POINTER(Router), _P, _I, _I, _I, _P, _P, _P, _I, _P, _P, _P,
                           _P, _SZ, _P], ctypes.c_int),
    "locali_moe_dispatch": ([_P, _I, _I, _I, _P, _P, _P], ctypes.c_int),
    "locali_moe_expert_decode": ([ctypes.POINTER(ExpertArena), ctypes.POINTER(ExpertArena), _P, _I,
                                  _I, _I, _P, _P, _F, _I, _I, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "locali_moe_decode_gateup": ([ctypes.POINTER(ExpertArena), ctypes.POINTER(ExpertArena), _P, _I,
                                  _I, _I, _P, _F, _I, _P, _P, _SZ, _P], ctypes.c_int),
    "locali_moe_decode_down_combine": ([ctypes.POINTER(ExpertArena), ctypes.POINTER(ExpertArena), _I,
                                        _I, _I, _P, _P, _I, _P, _P, _SZ, _P], ctypes.c_int),
    "locali_moe_expert_grouped": ([ctypes.POINTER(ExpertArena), ctypes.POINTER(ExpertArena), _P, _I,
                                   _I, _I, _I, _P, _P, _P, _F, _I, _I, _P, _P, _SZ, _P], ctypes.c_int),
    "locali_moe_expert_prefill": ([ctypes.POINTER(ExpertArena), ctypes.POINTER(ExpertArena), _P, _I,
                                   _I, _I, _I, _P, _P, _P, _F, _I, _I, _P, _P, _SZ, _P], ctypes.c_int),
    "locali_moe_expert_grouped_stages": ([ctypes.POINTER(ExpertArena), ctypes.POINTER(ExpertArena), _P, _I,
                                          _I, _I, _I, _P, _P, _P, _F, _I, _I, _P, _P, _P, _P, _P, _SZ, _P],
                                         ctypes.c_int),
    "locali_moe_router_logits": ([ctypes.POINTER(Router), _P, _I, _I, _I, _P, _P], ctypes.c_int),
    "locali_moe_decode_gateup_select": ([ctypes.POINTER(Router), ctypes.POINTER(ExpertArena),
                                         ctypes.POINTER(ExpertArena), _P, _P, _I, _I, _P, _P, _F, _I, _P, _P,
                                         _P, _P, _P, _SZ, _P], ctypes.c_int),
    "locali_moe_combine": ([_P, _P, _P, _I, _I, _I, _I, _I, _P, _P], ctypes.c_int),
    "locali_moe_combine_routes": ([_P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P], ctypes.c_int),
    "locali_moe_arena_fill": ([_P, _P, _SZ, _P], ctypes.c_int),
    "locali_moe_arena_fill_batch": ([ctypes.POINTER(FillPiece), ctypes.c_int32, _P], ctypes.c_int),
    "locali_moe_arena_fill_slots": ([ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t), _I, _I,
                                     ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_void_p), _I, _P],
                                    ctypes.c_int),
    "locali_moe_forward": ([ctypes.POINTER(Router), ctypes.POINTER(ExpertArena),
                            ctypes.POINTER(ExpertArena), _P, _P, _I, _I, _P, _F, _I, _P, _P, _P, _P,
                            _SZ, _P], ctypes.c_int),
    "locali_moe_forward_noalloc": ([ctypes.POINTER(Router), ctypes.POINTER(ExpertArena),
                                    ctypes.POINTER(ExpertArena), _P, _P, _I, _I, _P, _F, _I, _P, _P, _P,
                                    _P], ctypes.c_int),
    "locali_moe_last_error": ([], ctypes.c_char_p),
}

EXPORTS = tuple(_SIGNATURES)

_lib = None


def lib() -> ctypes.CDLL:
    """Load (once) and return the library, raising loudly when it is absent."""
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            raise LocaliError(
                f"{LIB_PATH} is missing: build it with `python -m locali_amd.build` "
                "(there is no CPU fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (argtypes, restype) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().locali_moe_last_error()
        raise LocaliError(f"{what} failed ({rc}): {msg.decode() if msg else ''}")
