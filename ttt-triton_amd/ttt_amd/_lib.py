"""ctypes binding of libttt_amd.so (declared in include/ttt_amd.h).

The library is loaded from this directory.  There is no fallback: if the
library is missing or fails to load, every entry point raises."""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
# TTT_AMD_LIB names another build of the same library (e.g. the host-ASan
# checking build of build_lib.py --asan)
LIB_PATH = os.environ.get("TTT_AMD_LIB") or os.path.join(_HERE, "libttt_amd.so")
ABI_VERSION = 11

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

# eta forms (enum ttt_eta_rule): the dense [B,H,NC,K,K] tensor, or the per-token
# learning rate lr [B,H,NC,K] fp32 expanded on chip by a rule
ETA_DENSE = 0
ETA_LAYER = 1
ETA_CAUSAL = 2
ETA_DENSE_F32 = 3  # dense eta kept in fp32 under 16-bit activations (chosen from eta's dtype)
ETA_RULES = {"dense": ETA_DENSE, "layer": ETA_LAYER, "causal": ETA_CAUSAL}

# process-wide options (enum ttt_option)
OPT_MLP_BWD_POLL_LIMIT = 1
OPT_MLP_BWD_FUSED = 2
OPT_SMALL_KERNELS = 3

STATUS_TIMEOUT = -8
STATUS_SCRATCH = -9
MLP_BWD_NOALLOC_SCRATCH_BYTES = 64 << 20

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_S = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/ttt_amd.h
SIGNATURES = {
    "ttt_abi_version": (_I, []),
    "ttt_error_string": (ctypes.c_char_p, [_I]),
    "ttt_linear_fwd": (_I, [_P] * 8 + [_I] * 8 + [_F] + [_P] * 5 + [_P, _S, _P]),
    "ttt_linear_saved_bytes": (_S, [_I] * 5),
    "ttt_linear_bwd": (_I, [_P] * 9 + [_I] * 8 + [_F] + [_P] * 8 + [_P, _S, _P]),
    "ttt_mlp_fwd": (_I, [_P] * 10 + [_I] * 10 + [_F] + [_P] * 13 + [_P, _S, _P]),
    "ttt_mlp_saved_bytes": (_S, [_I] * 7),
    "ttt_mlp_bwd_workspace_bytes": (_S, [_I] * 7),
    "ttt_mlp_bwd": (_I, [_P] * 15 + [_I] * 9 + [_F] + [_P] * 10 + [_P, _S, _P, _S, _P]),
    "ttt_mlp_bwd_noalloc": (_I, [_P] * 15 + [_I] * 9 + [_F] + [_P] * 10 + [_P, _S, _P]),
    "ttt_set_option": (_I, [_I, ctypes.c_longlong]),
    "ttt_get_option": (ctypes.c_longlong, [_I]),
    "ttt_mlp_bwd_check": (_I, [_P, _S] + [_I] * 7 + [_P]),
    "ttt_layer_io_partial_bytes": (_S, [_I] * 4),
    "ttt_qkvu_producer_fwd": (_I, [_P, _I] + [_P] * 3 + [_I] * 5 + [_F, _F, _I] + [_P] * 5 + [_P]),
    "ttt_qkvu_producer_bwd": (_I, [_P, _I] + [_P] * 3 + [_P] * 5 + [_I] * 5 + [_F, _F, _I] + [_P, _P, _S, _P]),
    "ttt_post_norm_fwd": (_I, [_P] * 3 + [_I] * 5 + [_F, _I] + [_P, _P, _P]),
    "ttt_post_norm_bwd": (_I, [_P] * 4 + [_I] * 6 + [_P, _P, _S, _P]),
    "ttt_mlp_cached_readout": (_I, [_P] * 7 + [_I] * 8 + [_F] + [_P, _P]),
    "ttt_mlp_memo_gates_bytes": (_S, [_I] * 6),
    "ttt_mlp_memo_workspace_bytes": (_S, [_I] * 8),
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
        if status in (-5, STATUS_TIMEOUT):
            raise TTTError(f"{what}: {msg}")
        raise ValueError(f"{what}: {msg} (status {status})")


def fast_linear_shape(K: int, F: int) -> bool:
    """Shapes of the specialised TTT-Linear kernels (16-token mini-batches in
    registers); every other valid shape takes the general-shape kernels, whose
    forward needs the saved buffer as scratch even without a backward."""
    return K == 16 and F in (32, 64)


def fast_mlp_shape(K: int, F: int, FF: int) -> bool:
    return fast_linear_shape(K, F) and FF in (64, 128, 256)


def eta_rule_code(rule) -> int:
    """ttt_eta_rule code of `rule` ("dense", "layer", "causal" or the code)."""
    if isinstance(rule, str):
        if rule not in ETA_RULES:
            raise ValueError(f"unknown eta rule {rule!r} (dense, layer or causal)")
        return ETA_RULES[rule]
    if int(rule) not in ETA_RULES.values():
        raise ValueError(f"unknown eta rule {rule}")
    return int(rule)


def set_option(option: int, value: int) -> None:
    check(load().ttt_set_option(int(option), int(value)), "ttt_set_option")


def get_option(option: int) -> int:
    return int(load().ttt_get_option(int(option)))
