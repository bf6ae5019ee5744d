"""ctypes binding of the HIP kernel library (the C ABI of include/probjax_hip.h).

The library is loaded from ``probjax_amd/_lib/libprobjax_hip.so`` (built by
``probjax_amd.build``).  There is no fallback: a missing or stale library is
an error, so that nothing silently runs on another implementation.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libprobjax_hip.so"

PJX_DTYPE_F32 = 0
PJX_DTYPE_BF16 = 1
PJX_DTYPE_F16 = 2
PJX_OK = 0
PJX_DECODE_STATIC_SCRATCH_BYTES = 32 << 20  # include/probjax_hip.h



class ScoreMods(ctypes.Structure):
    """``pjx_score_mods`` of include/probjax_hip.h (extended masks and score
    modifiers; device pointers as integers, None for absent)."""

    _fields_ = [
        ("causal_shift", ctypes.c_int32),
        ("window_left", ctypes.c_int32),
        ("window_right", ctypes.c_int32),
        ("prefix_lengths", ctypes.c_void_p),
        ("seq_lengths", ctypes.c_void_p),
        ("segment_q", ctypes.c_void_p),
        ("segment_k", ctypes.c_void_p),
        ("alibi_slopes", ctypes.c_void_p),
        ("alibi_symmetric", ctypes.c_int32),
        ("softcap", ctypes.c_float),
        ("head_scales", ctypes.c_void_p),
        ("constant", ctypes.c_float),
        ("row_kv_lengths", ctypes.c_void_p),
    ]


# (name, restype, argtypes) of every exported entry point.
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_MODS = ctypes.POINTER(ScoreMods)
_SIGNATURES = {
    "pjx_version": (ctypes.c_int, []),
    "pjx_last_error": (ctypes.c_char_p, []),
    "pjx_last_launches": (ctypes.c_char_p, []),
    "pjx_flash_fwd": (
        ctypes.c_int,
        [ctypes.c_int, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
         _I64, _I64, _I64, _I64, ctypes.c_int, ctypes.c_float, _MODS, _P],
    ),
    "pjx_flash_bwd_workspace_size": (ctypes.c_size_t, [_I64, _I64, _I64]),
    "pjx_flash_bwd_ds_workspace_size": (ctypes.c_size_t, [ctypes.c_int, _I64, _I64, _I64, _I64, _I64]),
    "pjx_flash_bwd": (
        ctypes.c_int,
        [ctypes.c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P, _P, _I64,
         _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_int, ctypes.c_float, _MODS, _P],
    ),
    "pjx_decode_workspace_size": (ctypes.c_size_t, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "pjx_splitkv_decode": (
        ctypes.c_int,
        [ctypes.c_int, _P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _I64, _I64, _I64, _I64,
         _I64, _I64, _I64, ctypes.c_float, _I64, _P],
    ),
    "pjx_splitkv_decode_static": (
        ctypes.c_int,
        [ctypes.c_int, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         ctypes.c_float, _I64, _P],
    ),
    "pjx_mla_decode": (
        ctypes.c_int,
        [ctypes.c_int, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _I64, _I64, _I64, _I64,
         _I64, _I64, ctypes.c_float, _I64, _P],
    ),
    "pjx_mla_fwd": (
        ctypes.c_int,
        [ctypes.c_int, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I64, _I64, ctypes.c_int, ctypes.c_float, _MODS, _P],
    ),
    "pjx_mla_bwd_workspace_size": (ctypes.c_size_t, [_I64, _I64, _I64, _I64, _I64]),
    "pjx_mla_bwd": (
        ctypes.c_int,
        [ctypes.c_int, _P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P, _P, _I64, _I64, _I64,
         _I64, _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_int, ctypes.c_float, _MODS, _P],
    ),
    "pjx_mla_project": (
        ctypes.c_int,
        [ctypes.c_int, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    ),
}
EXPORTED = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib = None


class NativeLibraryError(RuntimeError):
    """The HIP kernel library is missing, stale, or reported an error."""


def load() -> ctypes.CDLL:
    """Load (once) and return the kernel library; raise if it is unavailable."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise NativeLibraryError(
                f"HIP kernel library not found at {LIB_PATH}; build it with "
                "`python -m probjax_amd.build`"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                raise NativeLibraryError(f"{LIB_PATH} does not export {name}: rebuild it")
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def check(rc: int) -> None:
    """Raise with the library's message when an entry point failed."""
    if rc != PJX_OK:
        msg = load().pjx_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(msg)
        raise NativeLibraryError(f"error {rc}: {msg}")


def last_launches() -> list:
    """Kernel instances (``"name<template args>"``) that the calling thread's
    last entry-point call launched, in order (``pjx_last_launches``)."""
    s = load().pjx_last_launches().decode(errors="replace")
    return s.split(";") if s else []
