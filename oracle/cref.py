"""ctypes binding for ``liboracle_kda.so`` -- TEST INFRASTRUCTURE ONLY.

Wraps ``kda_oracle_fwd`` / ``kda_oracle_bwd`` (oracle/kda_oracle.c), the fp64
restatement of the reference step recurrence (nope_gdn_mlx.py:616-638) and of
its reverse-time backward (nope_gdn_mlx.py:3185-3295).  Accepts torch tensors
of any float dtype in the layer layout and returns float64 tensors.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Dict, Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_kda.so")
_lib = None


def build() -> str:
    """Compile the C oracle in place (``make -C oracle``)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is not built; run `make -C oracle`")
        lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int
        lib.kda_oracle_fwd.argtypes = [P] * 8 + [I] * 5
        lib.kda_oracle_fwd.restype = I
        lib.kda_oracle_bwd.argtypes = [P] * 14 + [I] * 5
        lib.kda_oracle_bwd.restype = I
        _lib = lib
    return _lib


def _threads(n: Optional[int]) -> int:
    if n:
        return n
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:  # pragma: no cover
        return 4


def _d(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    if t is None:
        return None
    return t.detach().to("cpu", torch.float64).contiguous()


def _p(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def forward(q, k, v, g, beta, s0=None, nthreads: Optional[int] = None) -> Dict[str, torch.Tensor]:
    """o (B,T,H,D) and s_final (B,H,D,D), float64."""
    lib = _load()
    q, k, v, g, beta, s0 = (_d(t) for t in (q, k, v, g, beta, s0))
    B, T, H, D = q.shape
    o = torch.zeros((B, T, H, D), dtype=torch.float64)
    sf = torch.zeros((B, H, D, D), dtype=torch.float64)
    rc = lib.kda_oracle_fwd(_p(q), _p(k), _p(v), _p(g), _p(beta), _p(s0), _p(o), _p(sf),
                            B, T, H, D, _threads(nthreads))
    if rc:
        raise RuntimeError(f"kda_oracle_fwd failed with code {rc}")
    return {"o": o, "s_final": sf}


def backward(q, k, v, g, beta, s0, do, ds_final=None,
             nthreads: Optional[int] = None) -> Dict[str, torch.Tensor]:
    """dq, dk, dv, dg (B,T,H,D), dbeta (B,T,H), ds0 (B,H,D,D), float64."""
    lib = _load()
    q, k, v, g, beta, s0, do, dsf = (_d(t) for t in (q, k, v, g, beta, s0, do, ds_final))
    B, T, H, D = q.shape
    z = lambda *s: torch.zeros(s, dtype=torch.float64)
    dq, dk, dv, dg = z(B, T, H, D), z(B, T, H, D), z(B, T, H, D), z(B, T, H, D)
    db, ds0 = z(B, T, H), z(B, H, D, D)
    rc = lib.kda_oracle_bwd(_p(q), _p(k), _p(v), _p(g), _p(beta), _p(s0), _p(do), _p(dsf),
                            _p(dq), _p(dk), _p(dv), _p(dg), _p(db), _p(ds0),
                            B, T, H, D, _threads(nthreads))
    if rc:
        raise RuntimeError(f"kda_oracle_bwd failed with code {rc}")
    return {"dq": dq, "dk": dk, "dv": dv, "dg": dg, "dbeta": db, "ds0": ds0}
