"""ctypes binding of libethos_hip.so (the C-ABI in include/ethos_hip.h).

torch is imported first so that its HIP runtime is the one the library binds to
(both carry the soname libamdhip64.so.7).  There is no fallback: if the library is
missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime the library must share)

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libethos_hip.so")

ETHOS_F32 = 0
ETHOS_BF16 = 1

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/ethos_hip.h
SIGNATURES = {
    "ethos_last_error": (ctypes.c_char_p, []),
    "ethos_abi_version": (ctypes.c_int, []),
    "ethos_stage_events": (ctypes.c_int, [_vp, _i32]),
    "ethos_query_proj_workspace_bytes": (_sz, [_i64, _i32, _i32, _i32, _i32]),
    "ethos_query_proj": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _vp, _sz, _vp, _vp]),
    "ethos_query_proj_weights_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "ethos_query_proj_prepare": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32, _vp, _sz, _vp]),
    "ethos_query_proj_prepared": (ctypes.c_int, [_vp, _vp, _vp, _sz, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _vp,
                                                 _sz, _vp, _vp]),
    "ethos_route_topk": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "ethos_route_keys_bytes": (_sz, [_i32, _i32, _i32]),
    "ethos_route_prepare_keys": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, _vp, _sz, _vp]),
    "ethos_route_topk_prepared": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _sz, _i64, _i32, _i32, _i32, _i32, _i32,
                                                 _vp, _vp, _vp]),
    "ethos_sort_workspace_bytes": (_sz, [_i64, _i64]),
    "ethos_sort_segment": (ctypes.c_int, [_vp, _i64, _i64, _vp, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ethos_sort_segment_noalloc": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ethos_sort_segment_token_proj": (ctypes.c_int, [_vp, _i64, _i64, _vp, _sz, _vp, _vp, _vp, _vp, _vp, _vp,
                                                     _vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp, _vp]),
    "ethos_generate": (ctypes.c_int, [_vp, _i64, _vp, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "ethos_apply_workspace_bytes": (_sz, [_i64, _i32, _i32, _i32, _i32]),
    "ethos_apply_scatter": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32,
                                           _vp, _sz, _vp, _vp]),
    "ethos_expert_backward_workspace_bytes": (_sz, [_i64, _i32, _i32, _i32]),
    "ethos_expert_backward": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _vp,
                                             _sz, _vp, _vp, _vp, _vp, _vp]),
    "ethos_expert_forward_workspace_bytes": (_sz, [_i64, _i32, _i32, _i64, _i32, _i32, _i32, _i32]),
    "ethos_expert_forward": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp,
                                            _vp, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _sz, _vp, _vp,
                                            _vp]),
    "ethos_token_proj": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp, _vp]),
    "ethos_apply_hidden_workspace_bytes": (_sz, [_i64, _i32, _i32, _i32, _i32, _i32]),
    "ethos_apply_hidden": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32,
                                          _vp, _sz, _vp, _vp]),
}

# ethos_sort_segment_noalloc's limit (ETHOS_NOALLOC_MAX_PAIRS in the header)
NOALLOC_MAX_PAIRS = 1 << 20

_lib = None


class EthosError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise EthosError(f"{LIB_PATH} is not built; run `python -m ethos_amd.build` (needs ROCm hipcc)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int, name: str) -> None:
    if rc != 0:
        msg = load().ethos_last_error().decode(errors="replace")
        raise EthosError(f"{name} failed with code {rc}: {msg}")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return ETHOS_BF16
    if dt == torch.float32:
        return ETHOS_F32
    raise TypeError(f"ETHOS HIP kernels support float32 and bfloat16, got {dt}")
