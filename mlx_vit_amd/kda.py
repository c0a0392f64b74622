"""The KDA chunkwise recurrence on MI355X: torch tensors in, HIP kernels out.

``chunk_kda(q, k, v, g, beta, initial_state)`` has the contract of the
reference's per-path KDA methods (nope_gdn_mlx.py:3056-3068, 2829-2865):

* ``q, k, v``: (B, T, H, D); ``g``: (B, T, H, D) per-channel log-decay (<= 0);
  ``beta``: (B, T, H); ``initial_state``: (B, H, D, D) or None (zeros), in the
  reference orientation ``S[i_v, j_k]`` so that ``o_t = S_t q_t``.
* returns ``(o, final_state)``: ``o`` in ``q.dtype``, the state in fp32.
* ``q`` is not scaled inside the op (the layer scales it beforehand,
  nope_gdn_mlx.py:796-799).

Differentiable in every input, including the initial state.  Arithmetic is fp32
with an fp32 state; bf16 inputs feed bf16 MFMA operands.  There is no CPU path:
tensors must live on a ROCm device and the HIP library must be built.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib

CHUNK = 64
# The chunk sizes the reference's layer is used with (nope_gdn_mlx.py:676, 4839-4856,
# 5035).  The chunked recurrence's result does not depend on the chunk size (the
# reference's own equivalence criterion, nope_gdn_mlx.py:4836-4914), so the
# kernels block at CHUNK whatever the caller's value.
CHUNK_SIZES = (8, 16, 32, 64)
# 96 (the reference's SSv2 model) runs the D = 128 kernels with channels
# 96..127 zero inside the library
FWD_HEAD_DIMS = (32, 64, 96, 128)
BWD_HEAD_DIMS = (32, 64, 96, 128)

_DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1}


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def head_decay_supported(D: int, dtype: torch.dtype) -> bool:
    """Whether the kernels take one decay per (b, t, h) -- g of shape (B, T, H),
    the scalar-alpha GDN's -- for this head size and operand dtype (otherwise
    broadcast g over the channels)."""
    return dtype == torch.bfloat16 and D in (32, 64)


def _g_code(g: torch.Tensor) -> int:
    """g_dtype code of a prepared g: per channel by dtype, or one fp32 decay per head."""
    return _lib.KDA_G_HEAD_F32 if g.dim() == 3 else _DTYPE_CODE[g.dtype]


def _prepare(q, k, v, g, beta, initial_state):
    """Validate and normalise inputs (contiguous, consistent dtypes).  g is
    (B, T, H, D), or (B, T, H) -- one decay per head, shared by its channels --
    where ``head_decay_supported``."""
    for name, t in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
    if q.dim() != 4:
        raise ValueError(f"q must be (B, T, H, D); got shape {tuple(q.shape)}")
    B, T, H, D = q.shape
    for name, t in (("k", k), ("v", v)):
        if tuple(t.shape) != (B, T, H, D):
            raise ValueError(f"{name} shape {tuple(t.shape)} != q shape {(B, T, H, D)}")
    if tuple(g.shape) == (B, T, H):
        if not head_decay_supported(D, q.dtype):
            raise ValueError(f"g of shape (B, T, H) (one decay per head) needs bf16 operands and head_dim in "
                             f"(32, 64); got {q.dtype}, head_dim={D}: broadcast g to (B, T, H, D)")
    elif tuple(g.shape) != (B, T, H, D):
        raise ValueError(f"g shape {tuple(g.shape)} != q shape {(B, T, H, D)} (or {(B, T, H)}, one per head)")
    if tuple(beta.shape) != (B, T, H):
        raise ValueError(f"beta shape {tuple(beta.shape)} != {(B, T, H)}")
    if initial_state is not None and tuple(initial_state.shape) != (B, H, D, D):
        raise ValueError(f"initial_state shape {tuple(initial_state.shape)} != {(B, H, D, D)}")
    if q.dtype not in _DTYPE_CODE:
        raise ValueError(f"q dtype {q.dtype} unsupported: use float32 or bfloat16")
    dev = q.device
    if dev.type != "cuda":
        raise ValueError("chunk_kda runs on a ROCm device; got tensors on " + str(dev))
    for name, t in (("k", k), ("v", v), ("g", g), ("beta", beta)):
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, q on {dev}")
    dt = q.dtype
    k, v, beta = (t if t.dtype == dt else t.to(dt) for t in (k, v, beta))
    if g.dtype not in _DTYPE_CODE or (g.dim() == 3 and g.dtype != torch.float32):
        g = g.to(torch.float32)
    q, k, v, g, beta = (t.contiguous() for t in (q, k, v, g, beta))
    if initial_state is not None:
        if initial_state.device != dev:
            raise ValueError(f"initial_state is on {initial_state.device}, q on {dev}")
        initial_state = initial_state.to(torch.float32).contiguous()
    return q, k, v, g, beta, initial_state


def _check_chunk(chunk_size: int) -> None:
    if chunk_size not in CHUNK_SIZES:
        raise ValueError(f"chunk_size={chunk_size}: expected one of {CHUNK_SIZES}")


def workspace_bytes(pass_: int, B: int, T: int, H: int, D: int, dtype: torch.dtype = torch.bfloat16) -> int:
    lib = _lib.load()
    n = lib.kda_workspace_size(pass_, B, T, H, D, CHUNK, _DTYPE_CODE.get(dtype, 0))
    if n == 0 and B * T * H > 0:
        raise ValueError(_lib.last_error())
    return int(n)


def workspace_offsets(pass_: int, B: int, T: int, H: int, D: int, dtype: torch.dtype = torch.float32) -> dict:
    lib = _lib.load()
    arr = (ctypes.c_int64 * len(_lib.WS_REGIONS))()
    _lib.check(lib.kda_workspace_offsets(pass_, B, T, H, D, CHUNK, _DTYPE_CODE.get(dtype, 0), arr),
               "kda_workspace_offsets")
    return {name: int(arr[i]) for i, name in enumerate(_lib.WS_REGIONS)}


def train_kept_bytes(B: int, T: int, H: int, D: int, dtype: torch.dtype = torch.bfloat16) -> int:
    """Bytes of the training pair's workspace that ``kda_forward_train`` writes
    and ``kda_backward_train`` reads (the rest is the backward's scratch)."""
    lib = _lib.load()
    n = lib.kda_train_kept_size(B, T, H, D, CHUNK, _DTYPE_CODE.get(dtype, 0))
    if n == 0 and B * T * H > 0:
        raise ValueError(_lib.last_error())
    return int(n)


def _workspace(pass_: int, B: int, T: int, H: int, D: int, dev: torch.device, dtype,
               given: Optional[torch.Tensor] = None, nbytes: Optional[int] = None) -> torch.Tensor:
    """The caller's workspace (checked: a contiguous uint8 tensor on the
    inputs' device; its size is checked by the library) or a new one of
    ``nbytes`` (default: the pass's whole workspace)."""
    if given is not None:
        if not isinstance(given, torch.Tensor) or given.dtype != torch.uint8 or not given.is_contiguous():
            raise ValueError("workspace must be a contiguous torch.uint8 tensor")
        if given.device != dev:
            raise ValueError(f"workspace is on {given.device}, q on {dev}")
        return given
    n = workspace_bytes(pass_, B, T, H, D, dtype) if nbytes is None else nbytes
    return torch.empty(max(n, 256), dtype=torch.uint8, device=dev)


def kda_forward(q, k, v, g, beta, initial_state=None, chunk_size: int = CHUNK,
                workspace: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Forward only (no autograd graph).  Returns (o, final_state)."""
    _check_chunk(chunk_size)
    q, k, v, g, beta, s0 = _prepare(q, k, v, g, beta, initial_state)
    B, T, H, D = q.shape
    if D not in FWD_HEAD_DIMS:
        raise ValueError(f"head_dim={D}: the forward supports {FWD_HEAD_DIMS}")
    lib = _lib.load()
    dev = q.device
    o = torch.empty_like(q)
    s_final = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
    ws = _workspace(_lib.KDA_PASS_FWD, B, T, H, D, dev, q.dtype, workspace)
    rc = lib.kda_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(s0), _ptr(o), _ptr(s_final),
                     B, T, H, D, chunk_size, _DTYPE_CODE[q.dtype], _g_code(g),
                     _ptr(ws), ws.numel(), _stream(dev))
    _lib.check(rc, "kda_fwd")
    return o, s_final


def kda_forward_train(q, k, v, g, beta, initial_state=None, chunk_size: int = CHUNK,
                      workspace: Optional[torch.Tensor] = None
                      ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Forward that also keeps the per-chunk factors the backward needs.
    Returns (o, final_state, workspace); pass the workspace, unmodified, to
    ``kda_backward_train`` with the same inputs.  A new workspace holds only
    the kept part (``train_kept_bytes``); a given one may also be the pair's
    whole workspace (``workspace_bytes(2, ...)``)."""
    _check_chunk(chunk_size)
    q, k, v, g, beta, s0 = _prepare(q, k, v, g, beta, initial_state)
    B, T, H, D = q.shape
    if D not in BWD_HEAD_DIMS:
        raise ValueError(f"head_dim={D}: training supports {BWD_HEAD_DIMS}")
    lib = _lib.load()
    dev = q.device
    o = torch.empty_like(q)
    s_final = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
    ws = _workspace(_lib.KDA_PASS_TRAIN, B, T, H, D, dev, q.dtype, workspace,
                    nbytes=train_kept_bytes(B, T, H, D, q.dtype))
    rc = lib.kda_fwd_train(_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(s0), _ptr(o), _ptr(s_final),
                           B, T, H, D, chunk_size, _DTYPE_CODE[q.dtype], _g_code(g),
                           _ptr(ws), ws.numel(), _stream(dev))
    _lib.check(rc, "kda_fwd_train")
    return o, s_final, ws


def kda_backward_train(q, k, v, g, beta, initial_state, do, ds_final, workspace: torch.Tensor,
                       chunk_size: int = CHUNK):
    """VJP from the workspace of ``kda_forward_train`` (same inputs): returns
    (dq, dk, dv, dg, dbeta, d_initial_state).  A workspace of the pair's whole
    size also serves as the backward's scratch; a kept-part one gets a scratch
    buffer allocated for the call."""
    return kda_backward(q, k, v, g, beta, initial_state, do, ds_final, chunk_size, workspace, _train=True)


def kda_backward(q, k, v, g, beta, initial_state, do, ds_final=None, chunk_size: int = CHUNK,
                 workspace: Optional[torch.Tensor] = None, _train: bool = False):
    """VJP of ``kda_forward``: returns (dq, dk, dv, dg, dbeta, d_initial_state)."""
    _check_chunk(chunk_size)
    q, k, v, g, beta, s0 = _prepare(q, k, v, g, beta, initial_state)
    B, T, H, D = q.shape
    if D not in BWD_HEAD_DIMS:
        raise ValueError(f"head_dim={D}: the backward supports {BWD_HEAD_DIMS}")
    if tuple(do.shape) != (B, T, H, D):
        raise ValueError(f"do shape {tuple(do.shape)} != {(B, T, H, D)}")
    if do.device != q.device:
        raise ValueError(f"do is on {do.device}, q on {q.device}")
    do = do.to(q.dtype).contiguous()
    if ds_final is not None:
        if tuple(ds_final.shape) != (B, H, D, D):
            raise ValueError(f"ds_final shape {tuple(ds_final.shape)} != {(B, H, D, D)}")
        if ds_final.device != q.device:
            raise ValueError(f"ds_final is on {ds_final.device}, q on {q.device}")
        ds_final = ds_final.to(torch.float32).contiguous()
    lib = _lib.load()
    dev = q.device
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dg, dbeta = torch.empty_like(g), torch.empty_like(beta)
    ds0 = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
    if _train and workspace is None:
        raise ValueError("kda_backward_train needs the workspace returned by kda_forward_train")
    ws = _workspace(_lib.KDA_PASS_BWD, B, T, H, D, dev, q.dtype, workspace)
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(s0), _ptr(do), _ptr(ds_final),
            _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dg), _ptr(dbeta), _ptr(ds0),
            B, T, H, D, chunk_size, _DTYPE_CODE[q.dtype], _g_code(g))
    if not _train:
        _lib.check(lib.kda_bwd(*args, _ptr(ws), ws.numel(), _stream(dev)), "kda_bwd")
        return dq, dk, dv, dg, dbeta, ds0
    total = workspace_bytes(_lib.KDA_PASS_TRAIN, B, T, H, D, q.dtype)
    if ws.numel() >= total:
        _lib.check(lib.kda_bwd_train(*args, _ptr(ws), ws.numel(), _stream(dev)), "kda_bwd_train")
    else:
        n = total - train_kept_bytes(B, T, H, D, q.dtype)
        scratch = torch.empty(max(n, 256), dtype=torch.uint8, device=dev)
        _lib.check(lib.kda_bwd_train_split(*args, _ptr(ws), ws.numel(), _ptr(scratch), scratch.numel(),
                                           _stream(dev)), "kda_bwd_train_split")
    return dq, dk, dv, dg, dbeta, ds0


def gated_supported(D: int, dtype: torch.dtype) -> bool:
    """Whether ``kda_forward_gated`` has a fused kernel for this head size and dtype."""
    return (dtype == torch.bfloat16 and D == 64) or (dtype == torch.float32 and D in (32, 64))


def kda_forward_gated(q, k, v, g, beta, initial_state, gate: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                      train: bool = False, workspace: Optional[torch.Tensor] = None):
    """The forward with the layer's output norm fused into the store of o
    (``kda_fwd_gated``): ``y = rms_norm(o) * norm_weight * sigmoid(gate)`` per
    head, the RMSNormGated the reference layer applies to the path's output
    (nope_gdn_mlx.py:340-366, 880-885).  gate (B, T, H*D) in q's dtype.
    Returns (y (B, T, H*D), o, final_state, workspace); with ``train`` the
    workspace is the training pair's (pass it to ``kda_backward_train``)."""
    _check_chunk(CHUNK)
    q, k, v, g, beta, s0 = _prepare(q, k, v, g, beta, initial_state)
    B, T, H, D = q.shape
    if not gated_supported(D, q.dtype):
        raise ValueError(f"kda_forward_gated: no fused kernel for head_dim={D} with {q.dtype}")
    if tuple(gate.shape) != (B, T, H * D):
        raise ValueError(f"gate shape {tuple(gate.shape)} != {(B, T, H * D)}")
    if gate.dtype != q.dtype:
        raise ValueError(f"gate has dtype {gate.dtype}; expected {q.dtype}")
    if gate.device != q.device:
        raise ValueError(f"gate is on {gate.device}, q on {q.device}")
    epv = 16 // q.element_size()
    if gate.stride(2) != 1 or gate.stride(1) % epv or gate.storage_offset() % epv or \
            (B > 1 and gate.stride(0) != T * gate.stride(1)):
        gate = gate.contiguous()
    ld_z = gate.stride(1) if T > 0 else H * D
    w = norm_weight.detach().to(device=q.device, dtype=torch.float32).contiguous()
    if tuple(w.shape) != (D,):
        raise ValueError(f"norm_weight shape {tuple(w.shape)} != {(D,)}")
    lib = _lib.load()
    dev = q.device
    o = torch.empty_like(q)
    y = torch.empty((B, T, H * D), dtype=q.dtype, device=dev)
    s_final = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
    pass_ = _lib.KDA_PASS_TRAIN if train else _lib.KDA_PASS_FWD
    ws = _workspace(pass_, B, T, H, D, dev, q.dtype, workspace,
                    nbytes=train_kept_bytes(B, T, H, D, q.dtype) if train else None)
    rc = lib.kda_fwd_gated(pass_, _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(s0), _ptr(gate), ld_z,
                           _ptr(w), float(eps), _ptr(o), _ptr(y), H * D, _ptr(s_final),
                           B, T, H, D, CHUNK, _DTYPE_CODE[q.dtype], _g_code(g),
                           _ptr(ws), ws.numel(), _stream(dev))
    _lib.check(rc, "kda_fwd_gated")
    return y, o, s_final, ws


class ChunkKDAFunction(torch.autograd.Function):
    """Autograd wrapper (the role of mx.custom_function in
    nope_gdn_mlx.py:2725-2808).  When a gradient is needed the forward keeps its
    inputs and the per-chunk factors of kda_forward_train -- not the U / S
    trajectories the reference keeps; the backward recomputes the
    chunk-boundary states from those factors."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, initial_state, chunk_size=CHUNK):
        if any(ctx.needs_input_grad):
            o, s_final, ws = kda_forward_train(q, k, v, g, beta, initial_state, chunk_size)
        else:
            (o, s_final), ws = kda_forward(q, k, v, g, beta, initial_state, chunk_size), None
        ctx.save_for_backward(q, k, v, g, beta, initial_state)
        ctx.ws = ws
        ctx.chunk_size = chunk_size
        ctx.has_state = initial_state is not None
        return o, s_final

    @staticmethod
    def backward(ctx, do, ds_final):
        q, k, v, g, beta, s0 = ctx.saved_tensors
        if do is None:
            do = torch.zeros_like(q)
        if ctx.ws is not None:
            dq, dk, dv, dg, dbeta, ds0 = kda_backward_train(q, k, v, g, beta, s0, do, ds_final, ctx.ws,
                                                            ctx.chunk_size)
            ctx.ws = None
        else:
            dq, dk, dv, dg, dbeta, ds0 = kda_backward(q, k, v, g, beta, s0, do, ds_final, ctx.chunk_size)
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype), dbeta.to(beta.dtype),
                ds0 if ctx.has_state else None, None)


def chunk_kda(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
              initial_state: Optional[torch.Tensor] = None, chunk_size: int = CHUNK
              ) -> Tuple[torch.Tensor, torch.Tensor]:
    """KDA chunkwise recurrence, differentiable.  Returns (o, final_state).
    chunk_size is the reference's blocking parameter (8, 16, 32 or 64); the
    result does not depend on it."""
    _check_chunk(chunk_size)
    return ChunkKDAFunction.apply(q, k, v, g, beta, initial_state, chunk_size)


GDN_LOG_ALPHA_MIN = -80.0


def chunk_gdn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, alpha: torch.Tensor, beta: torch.Tensor,
              initial_state: Optional[torch.Tensor] = None, chunk_size: int = CHUNK
              ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Scalar-alpha gated delta rule (the reference's original GDN,
    ``_gdn_step_fused`` nope_gdn_mlx.py:641-650, chunkwise form
    ``_chunkwise_scalar_wy`` nope_gdn_mlx.py:949-1064), differentiable.

    q, k, v (B, T, H, D); alpha, beta (B, T, H) with alpha in (0, 1].  The step
    ``S (alpha (I - beta k k^T)) + beta v k^T`` is the KDA step with every
    channel's decay e^{g} equal to alpha, so this runs the KDA kernels on
    g = log(alpha) (clamped at -80: e^-80 is below fp32's resolution of any
    state term).  With bf16 operands at head_dim 32 or 64 the kernels take g as
    one fp32 decay per (b, t, h) and return its gradient summed over the
    channels (``head_decay_supported``); otherwise g is broadcast over D.
    Autograd through the log (and the broadcast) gives d alpha = sum_d dg / alpha."""
    if alpha.dim() != 3 or tuple(alpha.shape) != tuple(q.shape[:3]):
        raise ValueError(f"alpha must be (B, T, H) = {tuple(q.shape[:3])}; got {tuple(alpha.shape)}")
    g = torch.clamp(torch.log(alpha.float()), min=GDN_LOG_ALPHA_MIN)
    if not (q.dim() == 4 and head_decay_supported(q.shape[-1], q.dtype)):
        g = g.unsqueeze(-1).expand(q.shape).contiguous()
    return chunk_kda(q, k, v, g, beta, initial_state, chunk_size)


def solve_unit_triangular(M: torch.Tensor, b: torch.Tensor, upper: bool = False) -> torch.Tensor:
    """y = M^-1 b for unit-triangular M (BH, C, C), b (BH, C, N); fp32, C <= 64.
    The HIP counterpart of GatedDeltaLayer._metal_solve_triangular(_upper)
    (nope_gdn_mlx.py:1160-1196, 1261-1286)."""
    if M.dim() != 3 or b.dim() != 3 or M.shape[0] != b.shape[0] or M.shape[1] != M.shape[2] \
            or b.shape[1] != M.shape[1]:
        raise ValueError(f"shape mismatch: M {tuple(M.shape)}, b {tuple(b.shape)}")
    if M.device.type != "cuda" or b.device != M.device:
        raise ValueError("solve_unit_triangular runs on a ROCm device")
    M = M.to(torch.float32).contiguous()
    b = b.to(torch.float32).contiguous()
    y = torch.empty_like(b)
    BH, Cm, N = b.shape
    rc = _lib.load().kda_solve_unit_triangular(_ptr(M), _ptr(b), _ptr(y), BH, Cm, N, int(bool(upper)),
                                               _stream(M.device))
    _lib.check(rc, "kda_solve_unit_triangular")
    return y
