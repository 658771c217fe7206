"""ctypes binding of the C-ABI library (include/specfit_amd.h).

Loading fails loudly: there is no CPU or PyTorch fallback for any kernel.
"""
from __future__ import annotations

import ctypes
import os
import threading

from .build import LIB_PATH

SF_ABI_VERSION = 13
SF_ERR_HIP_BASE = 1000

_lock = threading.Lock()
_lib = None

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t

# name -> (argtypes, restype); mirrors include/specfit_amd.h.
SIGNATURES = {
    "sf_abi_version": ([], _i),
    "sf_error_string": ([_i], ctypes.c_char_p),
    "sf_router_topk": ([_p, _p, _i, _i, _i, _i, _i, _p, _p, _p, _p], _i),
    "sf_dispatch": ([_p, _i, _i, _i, _p, _p, _p, _p, _p, _p], _i),
    "sf_grouped_swiglu": ([_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p],
                          _i),
    "sf_grouped_swiglu_table": ([_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _p, _i64, _p, _p, _p], _i),
    "sf_grouped_swiglu_table_noalloc": ([_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _p, _i64, _p,
                                         _p], _i),
    "sf_expert_swiglu": ([_p, _i, _i64, _i, _i, _p, _p, _p, _p], _i),
    "sf_combine": ([_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _p], _i),
    "sf_copy_h2d": ([_p, _p, _sz, _p], _i),
    "sf_expert_record_bytes": ([_i64, _i64, _i64, _i64], _i64),
    "sf_expert_decode": ([_p, _sz, _i64, _p, _i, _i, _i, _p, _p], _i),
    "sf_tree_attention": ([_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64,
                           _i, _i, _i, _i, _i, ctypes.c_float, _p, _p], _i),
    "sf_rms_norm": ([_p, _i64, _i, _i, _p, ctypes.c_float, _p, _i64, _p], _i),
    "sf_qk_norm_rope": ([_p, _i64, _p, _i64, _i, _i, _i, _i, _p, _p, ctypes.c_float, _p, _p, _p,
                         _p, _p], _i),
}


class NativeLibraryError(RuntimeError):
    """The HIP library is missing, stale or failed a call."""


def library_path() -> str:
    return os.environ.get("SPECFIT_AMD_LIB", LIB_PATH)


def lib():
    """The loaded library; raises NativeLibraryError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise NativeLibraryError(
                f"specfit_amd HIP library not found at {path}; build it with "
                "`python -m specfit_amd.build` (there is no fallback path)")
        try:
            handle = ctypes.CDLL(path)
        except OSError as exc:
            raise NativeLibraryError(f"cannot load {path}: {exc}") from exc
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = restype
        version = handle.sf_abi_version()
        if version != SF_ABI_VERSION:
            raise NativeLibraryError(
                f"{path} has ABI version {version}, expected {SF_ABI_VERSION}")
        _lib = handle
        return handle


def error_string(code: int) -> str:
    raw = lib().sf_error_string(int(code))
    return raw.decode() if raw else f"error {code}"


def check(code: int, what: str) -> None:
    """Raise RuntimeError (with the HIP error text) for a non-zero status."""
    if code != 0:
        raise RuntimeError(f"{what} failed: {error_string(code)} (code {code})")
