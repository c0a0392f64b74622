"""kda_fwd_noalloc: the forward on the library's static device scratch, called
through the C ABI, against kda_fwd with a caller workspace on the same inputs.
Two calls in a row (the second smaller, so it runs over what the first left
in the array), fp32 and bf16, with and without an initial state: o and the
final state must be bit-identical to kda_fwd's.  A shape whose workspace
exceeds the scratch, and a buffer that is not device memory of the stream's
GPU, are rejected before any device work."""
import ctypes

import pytest
import torch

from mlx_vit_amd import _lib
from oracle import kda_reference as R

pytestmark = pytest.mark.gpu

DEV = "cuda"
_CODE = {torch.float32: 0, torch.bfloat16: 1}


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _call(fn, x, ws=None):
    lib = _lib.load()
    q, k, v, g, beta, s0 = x
    B, T, H, D = q.shape
    o = torch.full_like(q, float("nan"))
    sf = torch.full((B, H, D, D), float("nan"), dtype=torch.float32, device=DEV)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [_p(q), _p(k), _p(v), _p(g), _p(beta), _p(s0), _p(o), _p(sf), B, T, H, D, 64,
            _CODE[q.dtype], _CODE[g.dtype]]
    if fn == "kda_fwd":
        rc = lib.kda_fwd(*args, _p(ws), ws.numel(), st)
    else:
        rc = lib.kda_fwd_noalloc(*args, st)
    _lib.check(rc, fn)
    return o, sf


def _inputs(B, T, H, D, dtype, seed, with_state):
    x = R.make_inputs(B, T, H, D, dtype=dtype, seed=seed, with_state=with_state, g_scale=0.5)
    s0 = x["s0"].to(DEV) if x["s0"] is not None else None
    return [x[n].to(DEV).contiguous() for n in ("q", "k", "v", "g", "beta")] + [s0]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_matches_kda_fwd_twice(dtype):
    shapes = [((3, 300, 4, 64), True, 1), ((1, 70, 2, 64), False, 2)]   # second call smaller
    for (B, T, H, D), with_state, seed in shapes:
        print("noalloc case", dtype, (B, T, H, D), "state" if with_state else "no state", flush=True)
        x = _inputs(B, T, H, D, dtype, seed, with_state)
        nbytes = _lib.load().kda_workspace_size(0, B, T, H, D, 64, _CODE[dtype])
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        o_ref, sf_ref = _call("kda_fwd", x, ws)
        o, sf = _call("kda_fwd_noalloc", x)
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref), (dtype, B, T, H, D)
        assert torch.equal(sf, sf_ref), (dtype, B, T, H, D)


def test_noalloc_config1_shape_fits():
    """The headline forward shape (B8 H12 T1568 D64 bf16) runs on the scratch."""
    x = _inputs(8, 1568, 12, 64, torch.bfloat16, 3, False)
    nbytes = _lib.load().kda_workspace_size(0, 8, 1568, 12, 64, 64, 1)
    assert nbytes <= _lib.NOALLOC_MAX_WORKSPACE
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    o_ref, sf_ref = _call("kda_fwd", x, ws)
    o, sf = _call("kda_fwd_noalloc", x)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(sf, sf_ref)


def test_noalloc_rejects_oversize():
    lib = _lib.load()
    B, T, H, D = 8, 8192, 16, 64      # ~540 MB of workspace
    assert lib.kda_workspace_size(0, B, T, H, D, 64, 1) > _lib.NOALLOC_MAX_WORKSPACE
    q = torch.empty((1,), device=DEV)  # never touched: the size check comes first
    p = _p(q)
    rc = lib.kda_fwd_noalloc(p, p, p, p, p, None, p, None, B, T, H, D, 64, 1, 1, None)
    assert rc == _lib.KDA_E_WORKSPACE
    assert "static scratch" in _lib.last_error()


def test_noalloc_rejects_host_pointer():
    """A host buffer as q is refused with KDA_E_INVALID before any launch: the
    kernels would run on the scratch of the stream's GPU, so every buffer must
    live there.  o stays untouched (NaN)."""
    import numpy as np
    lib = _lib.load()
    B, T, H, D = 1, 70, 2, 64
    x = _inputs(B, T, H, D, torch.bfloat16, 4, False)
    host_q = np.zeros(B * T * H * D, dtype=np.uint16)
    q_host = ctypes.c_void_p(host_q.ctypes.data)
    o = torch.full_like(x[0], float("nan"))
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.kda_fwd_noalloc(q_host, _p(x[1]), _p(x[2]), _p(x[3]), _p(x[4]), None, _p(o), None,
                             B, T, H, D, 64, 1, 1, st)
    assert rc == _lib.KDA_E_INVALID
    assert "not device memory" in _lib.last_error()
    torch.cuda.synchronize()
    assert torch.isnan(o.float()).all()
    # the refused call leaves no error behind: the next valid call succeeds
    o2, sf2 = _call("kda_fwd_noalloc", x)
    torch.cuda.synchronize()
    assert torch.isfinite(o2.float()).all()
