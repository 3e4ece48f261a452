"""ctypes binding of ``libakv_amd.so`` (the C ABI declared in include/akv_amd.h).

The library is built in-tree by ``akv_amd.build``.  Loading never builds and
never falls back to another implementation: a missing or stale library is an
error.
"""

import ctypes
import threading
from ctypes import c_char_p, c_int32, c_int64, c_void_p
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "libakv_amd.so"

AKV_OK = 0
AKV_EINVAL = -22
AKV_EHIP = -5
AKV_ERUNTIME = -71
AKV_F32, AKV_F16, AKV_BF16 = 0, 1, 2
AKV_I32, AKV_I64 = 0, 1
# status word of akv_compact_rows
AKV_STATUS_SIZES, AKV_STATUS_INCOMPLETE, AKV_STATUS_REBUILT = 1, 2, 4
AKV_STATUS_UNUSABLE = AKV_STATUS_SIZES | AKV_STATUS_INCOMPLETE

_P = c_void_p
_SIGNATURES = {
    "akv_last_error": (c_char_p, []),
    "akv_version": (c_char_p, []),
    "akv_reposition_kv_layers": (
        c_int32,
        [_P, _P, c_int32, c_int32, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64,
         c_int64, _P, _P, _P, c_int64, c_int64, _P, c_int32, c_int64, c_int32, c_int32, _P],
    ),
    "akv_reposition_kv_layers_gated": (
        c_int32,
        [_P, _P, c_int32, c_int32, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64,
         c_int64, _P, _P, _P, c_int64, c_int64, _P, c_int32, c_int64, c_int32, c_int32, _P, _P],
    ),
    "akv_compact_workspace_bytes": (c_int64, [c_int32, c_int64]),
    "akv_compact_launches": (c_int32, [c_int32, c_int64, c_int64, _P]),
    "akv_compact_rows": (
        c_int32,
        [c_int32, _P, c_int64, _P, c_int64, _P, _P, _P, _P, _P, _P, _P, c_int64, _P, c_int64,
         _P, _P, _P, _P, _P, c_int64, _P, _P, c_int64, _P, _P, c_int32, _P, _P, c_int64, _P, _P],
    ),
    "akv_compact_pages": (
        c_int32,
        [c_int32, _P, c_int64, c_int32, _P, c_int64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
         _P, _P, _P, _P, _P, _P],
    ),
    "akv_decode_indices": (
        c_int32,
        [_P, _P, c_int64, _P, c_int32, _P, c_int32, _P, c_int32, _P, c_int32, _P, c_int32,
         _P, c_int32, c_int64, c_int32, _P, _P],
    ),
    "akv_window_lengths": (
        c_int32,
        [_P, _P, c_int32, _P, c_int32, _P, c_int32, _P, c_int64, c_int32, _P],
    ),
    "akv_build_indptr": (
        c_int32,
        [_P, c_int32, c_int32, _P, c_int32, _P, c_int32, c_int64, _P],
    ),
    "akv_write_row_slots": (
        c_int32,
        [_P, _P, c_int32, _P, c_int32, _P, c_int32, c_int64, _P],
    ),
    "akv_write_extend_rows": (
        c_int32,
        [_P, c_int64, _P, _P, c_int32, _P, c_int32, _P, _P, _P, c_int32, _P, c_int32, c_int32, _P],
    ),
    "akv_decode_attention_workspace_bytes": (c_int64, [c_int32, c_int32, c_int32, c_int64]),
    "akv_decode_attention": (
        c_int32,
        [_P, c_int64, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int32, c_int32,
         c_int32, c_int32, _P, _P, _P, ctypes.c_float, _P, c_int32, c_int64, c_int64, c_int64,
         _P, c_int64, _P, _P],
    ),
    "akv_decode_attention_noalloc_max_bytes": (c_int64, []),
    "akv_decode_attention_noalloc": (
        c_int32,
        [_P, c_int64, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int32, c_int32,
         c_int32, c_int32, _P, _P, _P, ctypes.c_float, _P, c_int32, c_int64, c_int64, c_int64, _P, _P],
    ),
    "akv_context_attention": (
        c_int32,
        [_P, c_int64, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int64, _P, _P, c_int64, c_int64,
         c_int64, c_int64, c_int32, c_int32, c_int32, c_int32, _P, _P, c_int32, _P, c_int32, _P, _P,
         c_int32, c_int32, _P, ctypes.c_float, ctypes.c_float, _P, c_int32, c_int64, c_int64, c_int64, _P],
    ),
    "akv_bind_workspace_bytes": (c_int64, [c_int32, c_int64]),
    "akv_bind_occurrences": (
        c_int32,
        [c_int32, _P, c_int64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, _P, _P, _P,
         c_int64, _P],
    ),
    "akv_copy_kv_rows": (
        c_int32,
        [_P, _P, _P, _P, c_int32, c_int64, c_int64, c_int64, c_int64, c_int64, _P, _P, c_int64, _P, _P],
    ),
    "akv_plan_ownership": (
        c_int32,
        [c_int64, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, c_int64, _P, _P, _P, _P, _P, _P, _P, _P, _P,
         _P, _P, _P, _P, _P],
    ),
    "akv_advance_ownership": (
        c_int32,
        [c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, _P, c_int32, _P, c_int64, _P, _P, _P,
         _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    ),
    "akv_gather_slots": (
        c_int32,
        [c_int32, _P, c_int64, c_int64, _P, _P, _P, c_int64, c_int64, _P, _P, _P],
    ),
    "akv_window_count": (
        c_int32,
        [c_int64, _P, _P, _P, c_int64, _P, _P, _P, _P, _P, c_int64, c_int64, _P],
    ),
    "akv_window_compile": (
        c_int32,
        [c_int64, _P, _P, _P, c_int64, _P, _P, _P, _P, _P, c_int64, c_int64, _P, _P, _P, _P, _P, _P,
         _P, _P],
    ),
    "akv_window_compile_bounded": (
        c_int32,
        [c_int64, _P, _P, _P, c_int64, _P, _P, _P, _P, _P, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P,
         _P, _P],
    ),
    "akv_plan_count": (
        c_int32,
        [c_int64, _P, c_int64, _P, _P, c_int64, _P, _P, c_int64, _P, _P],
    ),
    "akv_plan_compile": (
        c_int32,
        [_P, c_int32, c_int64, _P, c_int64, _P, _P, c_int64, _P, _P, c_int64, _P, _P, _P,
         c_int64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, _P, _P, _P, _P, _P],
    ),
}

EXPORTED = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib = None


class AkvError(RuntimeError):
    """A HIP launch failure reported by the library."""


def load():
    """Return the loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIBRARY_PATH.exists():
                raise RuntimeError(
                    f"akv_amd HIP library not built ({LIBRARY_PATH}); run "
                    "`python -m akv_amd.build` (there is no CPU fallback)"
                )
            lib = ctypes.CDLL(str(LIBRARY_PATH))
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def last_error():
    return load().akv_last_error().decode()


def check(rc, what):
    """Turn a C status into a Python exception (ValueError for bad arguments)."""
    if rc == AKV_OK:
        return
    message = last_error() or f"{what} failed with status {rc}"
    if rc == AKV_EINVAL:
        raise ValueError(message)
    raise AkvError(message)


def ptr(t):
    """Device/host address of a tensor or numpy array, or None."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data
