"""ctypes loader for libpal_hip.so and status -> exception mapping.

Stands in for the reference's nanobind module ``pal_core``
(src/pal_core/bindings.cpp:41-226).  The shared library exports the plain C
ABI declared in include/pal_hip.h.  There is no fallback: if the library is
missing or fails to load, every operator raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_NAME = "libpal_hip.so"
LIB_PATH = Path(os.environ.get("PAL_HIP_LIB", Path(__file__).resolve().parent / LIB_NAME))

PAL_OK = 0
PAL_ERR_INVALID_ARGUMENT = -1
PAL_ERR_RUNTIME = -2
PAL_ERR_HIP = -3

DTYPE_FLOAT16 = 0
DTYPE_BFLOAT16 = 1
DTYPE_FP8_E4M3 = 2
DTYPE_FLOAT32 = 3

ROPE_NONE = 0
ROPE_NEOX = 1
ROPE_GPTJ = 2

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_void_p = ctypes.c_void_p
_c_size_t = ctypes.c_size_t

# name -> (restype, argtypes); must match include/pal_hip.h
_SIGNATURES = {
    "pal_last_error": (ctypes.c_char_p, []),
    "pal_version": (ctypes.c_char_p, []),
    "pal_get_k_cache_stripe_size": (_c_int, [_c_int]),
    "pal_get_optimal_page_size": (_c_int, []),
    "pal_get_k_cache_shape": (_c_int, [_c_i64, _c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_c_i64)]),
    "pal_get_v_cache_shape": (_c_int, [_c_i64, _c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_c_i64)]),
    "pal_fill_kv_pages": (
        _c_int,
        [_c_void_p] * 7 + [_c_int, _c_i64, _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_void_p],
    ),
    "pal_fill_kv_pages_fp8": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int] + [_c_void_p] * 7
        + [_c_i64, _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_void_p],
    ),
    "pal_rope_fill_kv_pages": (
        _c_int,
        [_c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p, _c_int] + [_c_void_p] * 5
        + [_c_i64, _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_i64]
        + [_c_void_p, _c_i64, _c_int, _c_int, _c_void_p, _c_void_p, _c_int, _c_int, _c_void_p],
    ),
    "pal_paged_attention_decode_workspace_size": (
        _c_size_t,
        [_c_int, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_int],
    ),
    "pal_paged_attention_decode": (
        _c_int,
        [_c_void_p] * 6
        + [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_int]
        + [_c_void_p, _c_size_t, _c_void_p],
    ),
    "pal_paged_attention_decode_fp8_workspace_size": (
        _c_size_t,
        [_c_int, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_int],
    ),
    "pal_paged_attention_decode_fp8": (
        _c_int,
        [_c_void_p] * 8
        + [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_int]
        + [_c_void_p, _c_size_t, _c_void_p],
    ),
    "pal_paged_attention_decode_noalloc": (
        _c_int,
        [_c_void_p] * 6
        + [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_int]
        + [_c_void_p],
    ),
    "pal_paged_attention_prefill": (
        _c_int,
        [_c_void_p] * 8 + [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_void_p],
    ),
    "pal_paged_attention_prefill_fp8": (
        _c_int,
        [_c_void_p] * 10 + [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_void_p],
    ),
    "pal_paged_attention_fp8_workspace_size": (
        _c_size_t,
        [_c_int, _c_i64, _c_int, _c_int, _c_int, _c_int],
    ),
    "pal_paged_attention_fp8": (
        _c_int,
        [_c_void_p] * 10
        + [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64]
        + [_c_void_p, _c_size_t, _c_void_p],
    ),
    "pal_paged_attention_workspace_size": (
        _c_size_t,
        [_c_int, _c_i64, _c_int, _c_int, _c_int, _c_int],
    ),
    "pal_paged_attention": (
        _c_int,
        [_c_void_p] * 8
        + [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64]
        + [_c_void_p, _c_size_t, _c_void_p],
    ),
    "pal_page_pool_create": (_c_int, [_c_i64, ctypes.POINTER(_c_void_p)]),
    "pal_page_pool_destroy": (_c_int, [_c_void_p]),
    "pal_page_pool_alloc": (_c_int, [_c_void_p, _c_i64, _c_void_p]),
    "pal_page_pool_free": (_c_int, [_c_void_p, _c_void_p, _c_i64]),
    "pal_page_pool_num_free": (_c_i64, [_c_void_p]),
    "pal_page_pool_compaction_plan": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_i64, ctypes.POINTER(_c_i64)]),
    "pal_copy_pages": (
        _c_int,
        [_c_void_p] * 4 + [_c_i64, _c_int, _c_i64, _c_void_p, _c_void_p, _c_i64, _c_void_p],
    ),
    "pal_remap_pages": (_c_int, [_c_void_p, _c_i64, _c_void_p, _c_i64, _c_void_p]),
    "pal_debug_flags": (_c_int, [_c_int, ctypes.POINTER(ctypes.c_uint32)]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class LibraryNotBuiltError(RuntimeError):
    """Raised when libpal_hip.so is missing or cannot be loaded."""


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library with typed entry points."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise LibraryNotBuiltError(
                f"{LIB_PATH} not found: build it with `python proxy-attention-lab_amd/build_lib.py` "
                "(the paged-attention operators have no CPU fallback)"
            )
        try:
            handle = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:  # pragma: no cover - depends on the environment
            raise LibraryNotBuiltError(f"failed to load {LIB_PATH}: {exc}") from exc
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
        return _lib


def exported_symbols() -> list[str]:
    """Names of the C entry points the Python layer binds."""
    return list(_SIGNATURES)


def last_error() -> str:
    msg = lib().pal_last_error()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    """Translate a C-ABI status into the reference's exception classes.

    PAL_ERR_INVALID_ARGUMENT -> ValueError (std::invalid_argument under
    nanobind), PAL_ERR_RUNTIME / PAL_ERR_HIP -> RuntimeError.
    """
    if status == PAL_OK:
        return
    msg = last_error() or f"status {status}"
    if status == PAL_ERR_INVALID_ARGUMENT:
        raise ValueError(msg)
    raise RuntimeError(msg)
