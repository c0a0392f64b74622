"""ctypes binding of ``libkda_hip.so`` (the C ABI in ``include/kda_hip.h``).

The library is built in-tree by ``python -m mlx_vit_amd.build``.  There is no
fallback: if it is missing, every op raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libkda_hip.so")

ABI_VERSION = 4   # kda_abi_version() of the header this binding follows

KDA_OK = 0
KDA_E_INVALID = -1
KDA_E_UNSUPPORTED = -2
KDA_E_WORKSPACE = -3
KDA_E_HIP = -4

KDA_G_HEAD_F32 = 2   # g_dtype: fp32 g [B, T, H], one decay per head (dg likewise)

KDA_PASS_FWD = 0
KDA_PASS_BWD = 1
KDA_PASS_TRAIN = 2

NOALLOC_MAX_WORKSPACE = 128 << 20   # KDA_NOALLOC_MAX_WORKSPACE

KDA_LAYER_PRODUCER = 0
KDA_LAYER_RMSNORM = 1

WS_REGIONS = ("W", "U", "Qp", "QpT", "Kb", "KbT", "WT", "Aqk", "AqkT", "Akk", "Tii", "eG",
              "h", "dh", "Vp", "dVp", "SegX", "SegM", "SegS", "Pad", "PadB")

# every function the header declares, with its ctypes signature
_P, _I, _Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
_L, _F = ctypes.c_int64, ctypes.c_float
SIGNATURES = {
    "kda_abi_version": ([], _I),
    "kda_last_error": ([], ctypes.c_char_p),
    "kda_workspace_size": ([_I] * 7, _Z),
    "kda_workspace_offsets": ([_I] * 7 + [ctypes.POINTER(ctypes.c_int64)], _I),
    "kda_fwd": ([_P] * 8 + [_I] * 7 + [_P, _Z, _P], _I),
    "kda_bwd": ([_P] * 14 + [_I] * 7 + [_P, _Z, _P], _I),
    "kda_fwd_train": ([_P] * 8 + [_I] * 7 + [_P, _Z, _P], _I),
    "kda_fwd_noalloc": ([_P] * 8 + [_I] * 7 + [_P], _I),
    "kda_bwd_train": ([_P] * 14 + [_I] * 7 + [_P, _Z, _P], _I),
    "kda_train_kept_size": ([_I] * 6, _Z),
    "kda_bwd_train_split": ([_P] * 14 + [_I] * 7 + [_P, _Z, _P, _Z, _P], _I),
    "kda_fwd_gated": ([_I] + [_P] * 7 + [_L, _P, _F, _P, _P, _L, _P] + [_I] * 7 + [_P, _Z, _P], _I),
    "kda_solve_unit_triangular": ([_P] * 3 + [_I] * 4 + [_P], _I),
    "kda_layer_producer_fwd": ([_P] * 5 + [_L] * 3 + [_P] * 9 + [_I] * 4 + [_F] * 2 + [_I] * 2 + [_P], _I),
    "kda_layer_producer_bwd": ([_P] * 5 + [_L] * 3 + [_P] * 14 + [_L] * 3 + [_P] * 4 + [_I] * 4 + [_F] * 2
                               + [_I] * 2 + [_P, _Z, _P], _I),
    "kda_layer_gated_rmsnorm_fwd": ([_P, _P, _L, _P, _P, _L] + [_I] * 3 + [_F, _I, _P], _I),
    "kda_layer_gated_rmsnorm_bwd": ([_P, _P, _L, _P, _P, _L, _P, _P, _L, _P] + [_I] * 3 + [_F, _I, _P, _Z, _P], _I),
    "kda_layer_workspace_size": ([_I] * 5, _Z),
    "kda_profile_enable": ([_I], _I),
    "kda_profile_name": ([_I], ctypes.c_char_p),
    "kda_profile_read": ([_I, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int)], _I),
}
PROF_NKERNELS = 15

_lib = None
_lock = threading.Lock()


class KDAError(RuntimeError):
    """A HIP launch or runtime failure reported by the library."""


def load():
    """Load (once) and return the ctypes library handle."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m mlx_vit_amd.build` "
                    "(the KDA op has no CPU fallback)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (args, res) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = res
            if lib.kda_abi_version() != ABI_VERSION:
                raise RuntimeError("libkda_hip.so ABI version mismatch; rebuild it")
            _lib = lib
    return _lib


def last_error() -> str:
    return load().kda_last_error().decode("utf-8", "replace")


def check(rc: int, what: str) -> None:
    """Map a library return code to the reference's exception types: argument,
    shape and budget problems raise ``ValueError`` (as the reference's path
    validation does), device failures raise ``KDAError``."""
    if rc == KDA_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc in (KDA_E_INVALID, KDA_E_UNSUPPORTED, KDA_E_WORKSPACE):
        raise ValueError(msg)
    raise KDAError(msg)
