"""ctypes binding of ``libmi_amd.so`` (the gfx950 C-ABI library).

The library is built in-tree by ``build.py``.  Loading never falls back to
anything else: a missing or unloadable library raises ``RuntimeError`` so that
no caller can silently run a CPU path.  Every status code is converted by
:func:`check` into ``ValueError`` (bad or unsupported arguments) or
``RuntimeError`` (workspace too small, launch failure), carrying the
library's message.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmi_amd.so"

MI_OK = 0
MI_ERR_INVALID = -1
MI_ERR_UNSUPPORTED = -2
MI_ERR_WORKSPACE = -3
MI_ERR_LAUNCH = -4

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_u64 = ctypes.c_uint64
_c_f32 = ctypes.c_float
_c_sz = ctypes.c_size_t
_vp = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/mi_amd.h exactly.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "mi_last_error": (ctypes.c_char_p, []),
    "mi_version": (ctypes.c_int, []),
    "mi_paged_kv_append": (
        ctypes.c_int,
        [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp, _c_i64, _vp, _c_i64, _vp, _vp, _vp,
         _c_i32, _c_i32, _c_i32, _c_i32, _vp],
    ),
    "mi_rope_append": (
        ctypes.c_int,
        [_vp, _c_i64, _vp, _vp, _vp, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp, _c_i64, _vp, _c_i64, _vp, _vp,
         _vp, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _vp],
    ),
    "mi_decode_workspace_size": (_c_sz, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "mi_decode_plan": (
        ctypes.c_int,
        [_vp, _c_sz, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _vp],
    ),
    "mi_decode_run": (
        ctypes.c_int,
        [_vp, _c_sz, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i32, _c_i32,
         _c_i32, _c_i32, _c_i32, _c_f32, _c_i32, _vp],
    ),
    "mi_decode_rope_append_run": (
        ctypes.c_int,
        [_vp, _c_sz, _vp, _c_i64, _vp, _vp, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i32,
         _c_i32, _c_i32, _c_i32, _c_i32, _c_f32, _c_i32, _vp],
    ),
    "mi_decode_static_capacity": (_c_sz, []),
    "mi_decode_static": (
        ctypes.c_int,
        [_vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32,
         _c_i32, _c_i32, _c_f32, _vp],
    ),
    "mi_prefill_workspace_size": (_c_sz, [_c_i32, _c_i64]),
    "mi_prefill_plan": (
        ctypes.c_int,
        [_vp, _c_sz, _vp, _vp, _vp, _c_i32, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _vp],
    ),
    "mi_prefill_run": (
        ctypes.c_int,
        [_vp, _c_sz, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i32, _c_i64,
         _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_f32, _vp],
    ),
    "mi_sample_workspace_size": (_c_sz, [_c_i32, _c_i32]),
    "mi_sample": (
        ctypes.c_int,
        [_vp, _c_i64, _c_i32, _c_i32, _vp, _vp, _c_u64, _vp, _vp, _vp, _c_sz, _vp],
    ),
    "mi_add_rms_norm": (
        _c_i32,
        [_vp, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _vp, _c_i64, _c_i64, _c_i32, _c_f32, _vp],
    ),
    "mi_silu_mul": (_c_i32, [_vp, _c_i64, _vp, _c_i64, _c_i64, _c_i32, _vp]),
    "mi_page_table_state_size": (_c_sz, [_c_i32, _c_i32, _c_i32]),
    "mi_page_table_init": (ctypes.c_int, [_vp, _c_i32, _c_i32, _c_i32, _vp]),
    "mi_page_table_step": (
        ctypes.c_int,
        [_vp, _c_i32, _c_i32, _c_i32, _vp, _c_i32, _c_i32, _vp, _vp, _c_i64, _vp, _vp, _vp, _vp,
         _vp],
    ),
    "mi_page_table_step_decode_plan": (
        ctypes.c_int,
        [_vp, _c_i32, _c_i32, _c_i32, _vp, _c_i32, _c_i32, _vp, _vp, _c_i64, _vp, _vp, _vp, _vp,
         _c_i32, _vp, _c_sz, _c_i32, _c_i32, _c_i32, _vp],
    ),
    "mi_page_table_error_offset": (_c_sz, [_c_i32, _c_i32, _c_i32]),
    "mi_pages_zero": (ctypes.c_int, [_vp, _c_i64, _c_i32, _c_i64, _c_i64, _vp, _c_i32, _vp]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load ``libmi_amd.so`` once and attach the prototypes."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python minimal-inference_amd/build.py` "
                "(there is no fallback path)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        missing = [n for n in SIGNATURES if not hasattr(lib, n)]
        if missing:
            raise RuntimeError(f"{LIB_PATH} lacks entry points {missing}; rebuild it")
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    msg = load().mi_last_error()
    return msg.decode() if msg else ""


def check(status: int, what: str) -> None:
    """Raise the Python exception matching a library status code."""
    if status == MI_OK:
        return
    msg = f"{what}: {last_error()} (status {status})"
    if status in (MI_ERR_INVALID, MI_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise on failure."""
    check(getattr(load(), name)(*args), name)
