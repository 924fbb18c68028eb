"""ctypes binding of libtkmi.so (the C ABI declared in include/tkmi.h).

The library is loaded once, from this package directory.  There is no
fallback: if the library is missing or does not export the ABI this module
expects, every entry point raises.
"""

from __future__ import annotations

import ctypes
import pathlib
import threading
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_void_p

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libtkmi.so"
ABI_VERSION = 3

TK_OK, TK_ERR_ARG, TK_ERR_UNSUPPORTED, TK_ERR_HIP = 0, -1, -2, -3
TK_F32, TK_F16 = 0, 1
TK_EPI_BIAS, TK_EPI_BIAS_GELU, TK_EPI_BIAS_RESID = 0, 1, 2
TK_ROWS_KEEP_RESID, TK_ROWS_ZERO, TK_ROWS_ZERO_ALL = 1, 2, 3

_I64_3 = c_int64 * 3

# name -> (restype, argtypes); mirrors include/tkmi.h one to one.
SIGNATURES = {
    "tk_version": (c_int, []),
    "tk_last_error_string": (ctypes.c_char_p, []),
    "tk_ln_cast": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_float, c_void_p, c_void_p]
    ),
    "tk_add_ln_cast": (
        c_int,
        [c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_float,
         c_void_p],
    ),
    "tk_gemm": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_int64,
         c_int64, c_int64, c_int64, c_int, c_void_p, c_int, c_void_p],
    ),
    "tk_gemm_bias_add_ln": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_int, c_int64, c_int64, c_int64, c_float, c_void_p, c_int, c_void_p],
    ),
    "tk_gemm_ln_supported": (c_int, [c_int64]),
    "tk_flash_attn_fwd": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
         POINTER(c_int64), POINTER(c_int64), POINTER(c_int64), POINTER(c_int64), c_float, c_int,
         c_void_p, c_int64, c_void_p],
    ),
    "tk_attention_supported": (c_int, [c_int64]),
    "tk_qkv_attention": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64,
         c_float, c_int, c_void_p],
    ),
    "tk_qkv_attention_supported": (c_int, [c_int64, c_int64, c_int64, c_int64]),
    "tk_masked_softmax": (
        c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int, c_void_p, c_int64, c_void_p]
    ),
    "tk_small_forward": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int]
        + [c_void_p] * 14 + [c_float, c_float, c_float, c_float, c_void_p],
    ),
    "tk_small_forward_noalloc": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int]
        + [c_void_p] * 14 + [c_float, c_float, c_float, c_float, c_void_p],
    ),
    "tk_small_forward_supported": (c_int, [c_int64, c_int64, c_int64, c_int64, c_int64]),
}

_lock = threading.Lock()
_lib = None


class TkError(RuntimeError):
    """A libtkmi entry point returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed (status {status}): {message}")
        self.fn = fn
        self.status = status


def load() -> ctypes.CDLL:
    """Load libtkmi.so (once).  Raises if it is missing or has another ABI."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m tkmi.build` in "
                "transformer-kernel_amd/ (or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)  # AttributeError if the export is missing
            fn.restype = res
            fn.argtypes = args
        got = lib.tk_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {got}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


def is_available() -> bool:
    try:
        load()
        return True
    except Exception:
        return False


def call(name: str, *args) -> None:
    """Invoke an entry point and raise TkError on a non-zero status."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != TK_OK:
        msg = lib.tk_last_error_string()
        raise TkError(name, status, msg.decode() if msg else "")


def strides3(values) -> "ctypes.Array":
    return _I64_3(*[int(v) for v in values])
