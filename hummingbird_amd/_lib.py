"""ctypes binding of `libhummingbird_amd.so` (the C ABI declared in include/hummingbird_amd.h).

The library is loaded lazily on first use. There is no fallback: if the shared library is missing, every
operator raises `RuntimeError` telling the user to build it (`python -m hummingbird_amd._build`).
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_char_p, c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

# HUMMINGBIRD_AMD_LIB names another build of the same library (the host-sanitizer build of `_build.py`).
LIB_PATH = Path(os.environ.get("HUMMINGBIRD_AMD_LIB") or Path(__file__).resolve().parent / "libhummingbird_amd.so")

HB_OK = 0
HB_BF16 = 0
HB_F32 = 1
HB_F16 = 2

# status code -> Python exception type. Shape/argument errors mirror the reference's trace-time ValueErrors
# (sa3jax/dense_attention.py:119-120, sa3jax/band_attention.py:138-140); launch failures are RuntimeErrors.
_ERRORS = {1: ValueError, 2: ValueError, 3: TypeError, 4: ValueError, 5: ValueError, 6: ValueError,
           7: ValueError, 8: ValueError, 9: RuntimeError, 10: ValueError}

# name -> (restype, argtypes), exactly the declarations of include/hummingbird_amd.h
SIGNATURES = {
    "hb_last_error": (c_char_p, []),
    "hb_status_name": (c_char_p, [c_int]),
    "hb_version": (c_char_p, []),
    "hb_rope_tables": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "hb_dense_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "hb_dense_validate": (c_int, [c_int, c_int64, c_int, c_int, c_int, c_int, c_int, c_float]),
    "hb_dense_diffattn": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                  c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float, c_void_p,
                                  c_size_t]),
    "hb_dense_noalloc_max_bytes": (c_size_t, []),
    "hb_dense_diffattn_noalloc": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
                                          c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float]),
    "hb_dense_prep": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                              c_void_p, c_int, c_int, c_int, c_int, c_float, c_void_p, c_size_t]),
    "hb_dense_attend": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float, c_void_p, c_size_t]),
    "hb_dit_qkv_proj": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int64, c_int, c_void_p, c_void_p,
                                c_void_p, c_int, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float, c_void_p,
                                c_size_t]),
    "hb_dense_attend_qq": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                   c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float, c_void_p, c_size_t]),
    "hb_proj": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int,
                        c_int]),
    "hb_proj_glu": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int64, c_void_p, c_int, c_void_p,
                            c_int64, c_int64, c_int, c_int]),
    "hb_proj_residual": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64,
                                 c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int, c_int]),
    "hb_band_validate": (c_int, [c_int, c_int64, c_int, c_int, c_int, c_int, c_int, c_int]),
    "hb_band_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "hb_band_diffattn": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                 c_int, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_size_t]),
    "hb_cross_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "hb_cross_validate": (c_int, [c_int, c_int64, c_int64, c_int, c_int, c_int, c_int, c_int, c_float]),
    "hb_cross_prep": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int, c_int, c_int, c_int, c_float,
                              c_void_p, c_size_t]),
    "hb_cross_attend": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                c_int, c_int, c_int, c_int, c_float, c_void_p, c_size_t]),
    "hb_dyt": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_int]),
    "hb_glu": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int, c_void_p, c_int64, c_int64, c_int]),
    "hb_residual_dyt": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_int64, c_int64, c_int]),
    "hb_rms_modulate": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_float, c_void_p, c_void_p, c_int64,
                                c_int, c_void_p, c_int64, c_int64, c_int]),
    "hb_gated_residual": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64,
                                  c_void_p, c_int, c_int, c_void_p, c_int64, c_int64, c_int]),
    "hb_residual_rms": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64,
                                c_void_p, c_int, c_void_p, c_float, c_void_p, c_void_p, c_int64, c_int, c_void_p,
                                c_void_p, c_int64, c_int64, c_int]),
}

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the shared library once and attach the C prototypes."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH.name} is not built; run `python -m hummingbird_amd._build` "
                               "(hummingbird_amd has no non-HIP fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    """Raise the exception matching a non-zero status, with the library's message."""
    if status == HB_OK:
        return
    lib = load()
    msg = lib.hb_last_error().decode()
    name = lib.hb_status_name(status).decode()
    raise _ERRORS.get(status, RuntimeError)(f"{what}: {name}: {msg}")
