"""ctypes binding of libttt_amd.so (declared in include/ttt_amd.h).

The library is loaded from this directory.  There is no fallback: if the
library is missing or fails to load, every entry point raises."""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libttt_amd.so")
ABI_VERSION = 7

DTYPE_F32 = 0
DTYPE_BF16 = 1

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_S = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/ttt_amd.h
SIGNATURES = {
    "ttt_abi_version": (_I, []),
    "ttt_error_string": (ctypes.c_char_p, [_I]),
    "ttt_linear_fwd": (_I, [_P] * 8 + [_I] * 7 + [_F] + [_P] * 5 + [_P, _S, _P]),
    "ttt_linear_saved_bytes": (_S, [_I] * 5),
    "ttt_linear_bwd": (_I, [_P] * 9 + [_I] * 7 + [_F] + [_P] * 8 + [_P, _S, _P]),
    "ttt_mlp_fwd": (_I, [_P] * 10 + [_I] * 9 + [_F] + [_P] * 13 + [_P, _S, _P]),
    "ttt_mlp_saved_bytes": (_S, [_I] * 7),
    "ttt_mlp_bwd_workspace_bytes": (_S, [_I] * 7),
    "ttt_mlp_bwd": (_I, [_P] * 15 + [_I] * 8 + [_F] + [_P] * 10 + [_P, _S, _P, _S, _P]),
    "ttt_mlp_cached_readout": (_I, [_P] * 7 + [_I] * 8 + [_F] + [_P, _P]),
    "ttt_mlp_memo_gates_bytes": (_S, [_I] * 6),
    "ttt_mlp_memo_combine": (_I, [_P] * 10 + [_I] * 8 + [_F] + [_P, _P, _S, _P]),
    "ttt_mlp_memo_combine_bwd": (_I, [_P] * 10 + [_I] * 8 + [_F] + [_P, _S, _P, _P, _P, _P]),
}

_lock = threading.Lock()
_lib = None


class TTTError(RuntimeError):
    pass


def load(path: str = LIB_PATH):
    """Load (once) and return the ctypes library handle."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise TTTError(f"{path} not found: build it with `python ttt-triton_amd/build_lib.py`")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        v = lib.ttt_abi_version()
        if v != ABI_VERSION:
            raise TTTError(f"libttt_amd ABI version {v}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().ttt_error_string(status).decode()
        if status == -5:
            raise TTTError(f"{what}: {msg}")
        raise ValueError(f"{what}: {msg} (status {status})")
