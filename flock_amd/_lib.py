"""ctypes binding of libflock_attn.so (declared in include/flock_attn.h, flock_q8.h).

This is the Python counterpart of the Deno.dlopen binding a TypeScript host
would declare. The library is loaded from this package's directory only; if it
is missing this module raises -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libflock_attn.so")

FLK_OK = 0
FLK_ERR_ARG = -1
FLK_ERR_CACHE_FULL = -2
FLK_ERR_UNSUPPORTED = -3
FLK_ERR_WORKSPACE = -4
FLK_ERR_HIP = -5

ROPE_NEOX = 0
ROPE_NORM = 1

_p = ctypes.c_void_p
_u32 = ctypes.c_uint32
_i32 = ctypes.c_int32
_u64 = ctypes.c_uint64
_f32 = ctypes.c_float

# name -> (restype, argtypes); the exact set of entry points in include/*.h.
SIGNATURES: dict[str, tuple] = {
    "flk_last_error": (ctypes.c_char_p, []),
    "flk_version": (ctypes.c_char_p, []),
    "flk_device_count": (_i32, [ctypes.POINTER(_i32)]),
    "flk_set_stream": (_i32, [_p]),
    "flk_alloc": (_i32, [ctypes.POINTER(_p), _u64]),
    "flk_free": (_i32, [_p]),
    "flk_h2d": (_i32, [_p, _p, _u64, _u64]),
    "flk_d2h": (_i32, [_p, _p, _u64, _u64]),
    "flk_memset": (_i32, [_p, _i32, _u64]),
    "flk_sync": (_i32, []),
    "flk_workspace_bytes": (_u64, [_u32, _u32, _u32, _u32, _u32, _u32]),
    "flk_call_workspace_bytes": (_u64, [_i32, _u32, _u32, _u32, _u32, _u32, _u32]),
    "flk_rmsnorm": (_i32, [_p, _p, _p, _u32, _u32, _f32]),
    "flk_rope": (_i32, [_p, _p, _u32, _u32, _u32, _u32, _i32]),
    "flk_kv_append": (_i32, [_p, _p, _p, _p, _u32, _u32, _u32, _u32, _u32]),
    "flk_qk_prologue": (
        _i32,
        [_p, _p, _p, _p, _p, _p, _f32, _i32, _p, _p, _p, _u32, _u32, _u32, _u32, _u32, _u32],
    ),
    "flk_qk_prologue_strided": (
        _i32,
        [_p, _p, _p, _u32, _p, _p, _p, _f32, _i32, _p, _p, _p, _u32, _u32, _u32, _u32, _u32,
         _u32],
    ),
    "flk_attn_decode": (_i32, [_p, _p, _p, _p, _u32, _u32, _u32, _u32, _p, _u64]),
    "flk_attn_prefill": (_i32, [_p, _p, _p, _p, _u32, _u32, _u32, _u32, _u32, _p, _u64]),
    "flk_decode_layer": (
        _i32,
        [_p, _p, _p, _p, _p, _p, _f32, _i32, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _u32,
         _p, _u64],
    ),
    "flk_decode_layer_noalloc": (
        _i32,
        [_p, _p, _p, _p, _p, _p, _f32, _i32, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _u32],
    ),
    "flk_attn_decode_ragged": (
        _i32, [_p, _p, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _u32, _p, _u64]),
    "flk_decode_layer_ragged": (
        _i32,
        [_p, _p, _p, _p, _p, _p, _f32, _i32, _p, _p, _p, _p, _p, _p, _u32, _u32, _u32, _u32,
         _u32, _p, _u64]),
    # include/flock_q8.h
    "flk_q8_matvec": (_i32, [_p, _p, _p, _p, _u32, _u32, _u32]),
    "flk_q8_split": (_i32, [_p, _u32, _u32, _p, _p]),
    "flk_q8_matvec_ex": (_i32, [_p, _p, _p, _p, _u32, _u32, _u32, _p, _f32, _p, _p]),
    "flk_q8_gate_up_swiglu": (_i32, [_p, _p, _p, _p, _u32, _u32, _u32, _p, _f32]),
    "flk_swiglu": (_i32, [_p, _p, _p, _u32]),
    "flk_add": (_i32, [_p, _p, _p, _u32]),
    # include/flock_graph.h
    "flk_decode_layer_dev": (
        _i32,
        [_p, _p, _p, _p, _p, _p, _f32, _i32, _p, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _p, _u64]),
    "flk_embed": (_i32, [_p, _p, _p, _u32, _u32, _u32, _p]),
    "flk_advance": (_i32, [_p, _u32, _p, _p, _u32]),
    "flk_stream_create": (_i32, [ctypes.POINTER(_p)]),
    "flk_stream_destroy": (_i32, [_p]),
    "flk_capture_begin": (_i32, []),
    "flk_capture_end": (_i32, [ctypes.POINTER(_p)]),
    "flk_graph_launch": (_i32, [_p]),
    "flk_graph_destroy": (_i32, [_p]),
    # include/flock_wire.h
    "flk_f32_to_f16": (_i32, [_p, _p, _u64]),
    "flk_f16_to_f32": (_i32, [_p, _p, _u64]),
    "flk_wire_header_pack": (_i32, [_u32, _u32, _u32, _u32, _p]),
    "flk_wire_header_unpack": (_i32, [_p, _u64, _p, _p, _p, _p, _p]),
    "flk_argmax_ws_bytes": (_u64, [_u32]),
    "flk_argmax": (_i32, [_p, _u32, _p, _p, _p, _u64]),
    "flk_lm_head_ws_bytes": (_u64, [_u32, _u32]),
    "flk_lm_head": (_i32, [_p, _p, _f32, _p, _p, _u32, _u32, _p, _p, _p, _p, _p, _u64]),
}


class FlockError(RuntimeError):
    """A non-zero status from libflock_attn (the reference throws an Error)."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class CacheFullError(FlockError):
    pass


class WorkspaceError(FlockError):
    pass


class UnsupportedError(FlockError):
    pass


_ERRORS = {
    FLK_ERR_CACHE_FULL: CacheFullError,
    FLK_ERR_WORKSPACE: WorkspaceError,
    FLK_ERR_UNSUPPORTED: UnsupportedError,
}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load libflock_attn.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m flock_amd.build` "
                "(there is no CPU fallback for this path)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    """Raise the FlockError for a non-zero status."""
    if rc == FLK_OK:
        return
    msg = lib().flk_last_error().decode(errors="replace")
    cls = _ERRORS.get(rc, FlockError)
    raise cls(rc, f"{what}: {msg}" if what else msg)
