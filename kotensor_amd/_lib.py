"""ctypes binding of libkotensor_hip.so (the C ABI in include/kotensor_hip.h).

This is the Python counterpart of the JDK Foreign Function & Memory downcalls a
Kotlin host makes: every entry point takes plain pointers and sizes and returns an
int32 status. A negative status raises :class:`IllegalArgumentException`, a
positive (HIP runtime) status or KT_ERR_STATE :class:`IllegalStateException`, mirroring the
reference's ``require`` / ``check`` failures.

The library is loaded from the package directory and never replaced by anything
else: if it is missing, every call raises.
"""
from __future__ import annotations

import ctypes
import importlib.util
import os
import sys
import threading
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "libkotensor_hip.so"


class IllegalArgumentException(ValueError):
    """An argument error (the reference's ``require`` failures)."""

    def __init__(self, message: str, status: int = -1):
        super().__init__(message)
        self.status = status


class IllegalStateException(RuntimeError):
    """A runtime failure of the device (HIP error code in ``status``)."""

    def __init__(self, message: str, status: int = 1):
        super().__init__(message)
        self.status = status


class LibraryMissingError(RuntimeError):
    """libkotensor_hip.so has not been built; there is no fallback path."""


# status codes, include/kotensor_hip.h
KT_OK = 0
KT_ERR_ARGUMENT = -1
KT_ERR_SHAPE = -2
KT_ERR_NAN = -3
KT_ERR_ZEROS = -4
KT_ERR_RANGE = -5
KT_ERR_STATE = -6


class _QWeight(ctypes.Structure):
    _fields_ = [
        ("qdata", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("zeros", ctypes.c_void_p),
        ("rows", ctypes.c_int32),
        ("columns", ctypes.c_int32),
        ("bits", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("packed", ctypes.c_void_p),
    ]


QWeight = _QWeight


class QMatmulStep(ctypes.Structure):
    """kt_qmatmul_step: one step of kt_qmatmul_chain."""
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("norm_weight", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("normed", ctypes.c_void_p),
        ("weights", ctypes.POINTER(_QWeight)),
        ("count", ctypes.c_int32),
        ("outputs", ctypes.POINTER(ctypes.c_void_p)),
        ("biases", ctypes.POINTER(ctypes.c_void_p)),
        ("accumulate", ctypes.c_int32),
        ("alpha", ctypes.c_float),
        ("swiglu_gate", ctypes.c_int32),
    ]


class _StEntry(ctypes.Structure):
    """kt_st_entry: one tensor of a safetensors header."""
    _fields_ = [
        ("dtype", ctypes.c_char * 8),
        ("rank", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 8),
        ("offset", ctypes.c_int64),
        ("nbytes", ctypes.c_int64),
    ]


StEntry = _StEntry

_P = ctypes.c_void_p
_I = ctypes.c_int32
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> argument types (all return int32)
SIGNATURES = {
    "kt_abi_version": [],
    "kt_last_error": [ctypes.c_char_p, _SZ],
    "kt_device_count": [ctypes.POINTER(_I)],
    "kt_set_device": [_I],
    "kt_set_kernel_config": [_I, _I, _I, _I, _I],
    "kt_dev_alloc": [_SZ, ctypes.POINTER(_P)],
    "kt_dev_free": [_P],
    "kt_memcpy_h2d": [_P, _P, _SZ, _P],
    "kt_memcpy_d2h": [_P, _P, _SZ, _P],
    "kt_memcpy_d2d": [_P, _P, _SZ, _P],
    "kt_memset": [_P, _I, _SZ, _P],
    "kt_stream_create": [ctypes.POINTER(_P)],
    "kt_stream_destroy": [_P],
    "kt_stream_sync": [_P],
    "kt_debug_wait_limits": [ctypes.c_uint32, _I],
    "kt_qweight_layout": [_I, _I, _I, _I, _I, ctypes.POINTER(ctypes.c_int64)],
    "kt_qweight_check": [ctypes.POINTER(_QWeight)],
    "kt_qweight_packed_bytes": [_I, _I, _I, _I, ctypes.POINTER(ctypes.c_int64)],
    "kt_qweight_pack": [ctypes.POINTER(_QWeight), _P, _P],
    "kt_quantize": [_P, _I, _I, _I, _I, _P, _P, _P, _P],
    "kt_qmatmul": [_P, _I, ctypes.POINTER(_QWeight), _P, _I, _F, _P],
    "kt_qmatmul_noalloc": [_P, _I, ctypes.POINTER(_QWeight), _P, _I, _F, _P],
    "kt_qlinear_forward": [_P, _I, ctypes.POINTER(_QWeight), _P, _P, _P],
    "kt_qmatmul_group": [_P, _I, ctypes.POINTER(_QWeight), _I, ctypes.POINTER(_P), ctypes.POINTER(_P), _I, _F, _P],
    "kt_qmatmul_transposed": [_P, _I, ctypes.POINTER(_QWeight), _P, _I, _P],
    "kt_fused_cross_entropy": [_P, _I, ctypes.POINTER(_QWeight), _P, _P, _I, _P, _P, _P, _I, _P],
    "kt_dequantize_rows": [ctypes.POINTER(_QWeight), _P, _I, _P, _P],
    "kt_dequantize_columns": [ctypes.POINTER(_QWeight), _P, _I, _P, _P],
    "kt_rope_inv_freq": [_I, _F, _F, _F, _F, _I, _P],
    "kt_rmsnorm": [_P, _I, _I, _P, _F, _P, _P],
    "kt_rope_kv": [_P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _P],
    "kt_attention": [_P, _I, _P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P],
    "kt_silu_mul": [_P, _P, ctypes.c_int64, _P],
    "kt_swiglu_qmatmul": [_P, _P, _I, ctypes.POINTER(_QWeight), _P, _I, _F, _P, _P],
    "kt_rope_attention": [_P, _P, _P, _P, _I, _P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P],
    "kt_rmsnorm_qmatmul_group": [_P, _P, _F, _P, _I, ctypes.POINTER(_QWeight), _I, ctypes.POINTER(_P), ctypes.POINTER(_P), _I, _F, _P],
    "kt_rmsnorm_swiglu_gate": [_P, _P, _F, _P, _I, ctypes.POINTER(_QWeight), ctypes.POINTER(_QWeight), _P, _P, _P, _P, _P],
    "kt_qmatmul_chain": [ctypes.POINTER(QMatmulStep), _I, _P],
    "kt_argmax": [_P, _I, _P, _P],
    "kt_argmax_advance": [_P, _I, _P, _P, _P, _I, _P],
    "kt_position_add": [_P, _I, _P],
    "kt_record_token": [_P, _P, _P, _I, _P],
    "kt_graph_begin": [_P],
    "kt_graph_end": [_P, _P],
    "kt_graph_launch": [_P, _P],
    "kt_graph_destroy": [_P],
    "kt_add_inplace": [_P, _P, ctypes.c_int64, _P],
    "kt_fill_normal": [_P, ctypes.c_int64, ctypes.c_uint64, _F, _F, _P],
    "kt_st_open": [ctypes.c_char_p, ctypes.POINTER(_P)],
    "kt_st_close": [_P],
    "kt_st_count": [_P, ctypes.POINTER(_I)],
    "kt_st_name": [_P, _I, ctypes.c_char_p, _SZ],
    "kt_st_find": [_P, ctypes.c_char_p, ctypes.POINTER(_StEntry)],
    "kt_st_metadata": [_P, ctypes.c_char_p, ctypes.c_char_p, _SZ],
    "kt_st_metadata_key": [_P, _I, ctypes.c_char_p, _SZ],
    "kt_st_data": [_P, ctypes.c_char_p, ctypes.POINTER(_P), ctypes.POINTER(ctypes.c_int64)],
    "kt_st_load_qweight": [_P, ctypes.c_char_p, ctypes.POINTER(_QWeight), _P],
    "kt_st_writer_create": [ctypes.POINTER(_P)],
    "kt_st_writer_destroy": [_P],
    "kt_st_writer_metadata": [_P, ctypes.c_char_p, ctypes.c_char_p],
    "kt_st_writer_add": [_P, ctypes.c_char_p, ctypes.c_char_p, _I, ctypes.POINTER(ctypes.c_int64), _P, ctypes.c_int64, _I],
    "kt_st_writer_add_qweight": [_P, ctypes.c_char_p, ctypes.POINTER(_QWeight)],
    "kt_st_writer_save": [_P, ctypes.c_char_p, _P],
}

_lock = threading.Lock()
_lib = None


def _load():
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY_PATH.exists():
            raise LibraryMissingError(
                f"{LIBRARY_PATH} is not built; run `python -m kotensor_amd.build` "
                "(there is no CPU fallback for the HIP path)"
            )
        # torch bundles its own HIP runtime under the same soname; loading it first
        # makes this library bind to that copy, so a process never holds two runtimes.
        if "torch" not in sys.modules and importlib.util.find_spec("torch") is not None \
                and os.environ.get("KOTENSOR_NO_TORCH_PRELOAD") != "1":
            import torch  # noqa: F401
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _I
        _lib = lib
        return lib


def lib():
    """The loaded library (loads it on first use)."""
    return _load()


def last_error() -> str:
    buf = ctypes.create_string_buffer(512)
    lib().kt_last_error(buf, 512)
    return buf.value.decode("utf-8", "replace")


def check(status: int, what: str = "") -> None:
    if status == KT_OK:
        return
    message = last_error() or what
    if status < 0 and status != KT_ERR_STATE:
        raise IllegalArgumentException(message, status)
    raise IllegalStateException(message, status)


def call(name: str, *args) -> None:
    """Calls an entry point and raises on a non-zero status."""
    check(getattr(lib(), name)(*args), name)
