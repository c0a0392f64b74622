"""GatedDeltaLayer on MI355X: the reference's KDA layer around the HIP recurrence.

The reference layer (``GatedDeltaLayer``, nope_gdn_mlx.py:653-885) turns its
input ``x (B, L, hidden)`` into the recurrence's operands, runs the recurrence,
and maps the result back to ``hidden``:

* projections ``q_proj/k_proj/v_proj``, the low-rank decay ``f_proj_2(f_proj_1(x))``,
  the write gate ``b_proj`` and the low-rank output gate ``g_proj_2(g_proj_1(x))``
  stay GEMMs (hipBLASLt through torch); q, k and v share one GEMM;
* the element-wise producer -- short causal conv + SiLU + L2 norm + scale,
  ``g = -exp(A_log) softplus(f + dt_bias)``, ``beta = sigmoid(b)``
  (nope_gdn_mlx.py:796-821) -- is one HIP kernel, ``kda_layer_producer_fwd``,
  that writes q, k, v, g, beta straight into the recurrence's (B, T, H, D)
  layout (no head-folding transposes, nope_gdn_mlx.py:845-849);
* the recurrence is ``compute_path='hip_chunkwise_kda'`` (``KDARecurrence``);
* the epilogue ``rms_norm(o) * sigmoid(gate)`` (RMSNormGated,
  nope_gdn_mlx.py:340-366, 880-885) is applied by the recurrence kernel as it
  stores o (``kda_fwd_gated``: bf16 at head_dim 64, fp32 at 32 and 64; the
  standalone kernel ``kda_layer_gated_rmsnorm_fwd`` otherwise), followed by
  the ``o_proj`` GEMM.

Parameter names and shapes follow the reference (``q_conv1d.weight`` is
``(H*D, 4, 1)`` like MLX's depthwise Conv1d weight, ``A_log (H,)``,
``dt_bias (H*D,)``, ``o_norm.weight (D,)``).  Every element-wise op has a HIP
adjoint; there is no CPU path.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .kda import (BWD_HEAD_DIMS, CHUNK, FWD_HEAD_DIMS, _DTYPE_CODE, _ptr, _stream, gated_supported,
                  kda_backward, kda_backward_train, kda_forward_gated)
from .recurrence import GDN_HIP_PATH, HIP_PATH, KDARecurrence

CONV_TAPS = 4


def _rows(t: torch.Tensor, name: str) -> int:
    """Row stride (elements) of a (B, T, N) tensor whose rows (b, t) sit at
    (b * T + t) * stride; the last dim must be unit-stride."""
    if t.dim() != 3:
        raise ValueError(f"{name} must be (B, T, N); got shape {tuple(t.shape)}")
    B, T, _ = t.shape
    if t.stride(2) != 1 or (B > 1 and T > 0 and t.stride(0) != T * t.stride(1)):
        raise ValueError(f"{name} rows are not evenly strided (strides {t.stride()})")
    return t.stride(1)


def _vec_ok(t: torch.Tensor) -> torch.Tensor:
    """Rows are read four channels at a time: make the row stride and the base
    offset multiples of 4 elements, copying when they are not."""
    if t.stride(-1) != 1 or t.stride(1) % 4 != 0 or t.storage_offset() % 4 != 0 or \
            (t.shape[0] > 1 and t.stride(0) != t.shape[1] * t.stride(1)):
        return t.contiguous()
    return t


def _check_dtype(name: str, t: torch.Tensor, dtype: torch.dtype) -> None:
    if t.dtype != dtype:
        raise ValueError(f"{name} has dtype {t.dtype}; expected {dtype}")


def producer_forward(qkv: torch.Tensor, xf: torch.Tensor, xb: torch.Tensor, conv_w: torch.Tensor,
                     conv_b: Optional[torch.Tensor], dt_bias: torch.Tensor, A_log: torch.Tensor,
                     num_heads: int, head_dim: int, scale: float, beta_mult: float = 1.0,
                     g_dtype: torch.dtype = torch.float32):
    """(q, k, v, g, beta) from the projection outputs.

    qkv (B, T, 3*H*D) = [q_proj | k_proj | v_proj](x); xf (B, T, H*D) =
    f_proj_2(f_proj_1(x)); xb (B, T, H) = b_proj(x); conv_w (3, H*D, 4) and
    conv_b (3, H*D) fp32 (q, k, v convs; tap 3 multiplies the current token);
    dt_bias (H*D,), A_log (H,) fp32.  Returns q, k, v, g (B, T, H, D) and beta
    (B, T, H); g in ``g_dtype``, the rest in qkv's dtype."""
    H, D = num_heads, head_dim
    HD = H * D
    dt = qkv.dtype
    if dt not in _DTYPE_CODE or g_dtype not in _DTYPE_CODE:
        raise ValueError(f"dtype {dt} / g dtype {g_dtype}: use float32 or bfloat16")
    gate = xf is not None
    qkv = _vec_ok(qkv)
    B, T, N = qkv.shape
    if N != 3 * HD:
        raise ValueError(f"qkv has {N} columns; expected 3*H*D = {3 * HD}")
    if tuple(xb.shape) != (B, T, H) or (gate and tuple(xf.shape) != (B, T, HD)):
        raise ValueError(f"xf {None if xf is None else tuple(xf.shape)} / xb {tuple(xb.shape)} do not match "
                         f"(B, T) = {(B, T)}")
    _check_dtype("xb", xb, dt)
    if xb.stride(-1) != 1 or (B > 1 and xb.stride(0) != T * xb.stride(1)):
        xb = xb.contiguous()
    ld_x, ld_b = _rows(qkv, "qkv"), _rows(xb, "xb")
    ld_f = 0
    if gate:
        _check_dtype("xf", xf, dt)
        xf = _vec_ok(xf)
        ld_f = _rows(xf, "xf")
        dt_bias = dt_bias.to(torch.float32).contiguous()
        A_log = A_log.to(torch.float32).contiguous()
    else:
        dt_bias = A_log = None
    conv_w = conv_w.to(torch.float32).contiguous()
    conv_b = None if conv_b is None else conv_b.to(torch.float32).contiguous()
    dev = qkv.device
    q = torch.empty((B, T, H, D), dtype=dt, device=dev)
    k, v = torch.empty_like(q), torch.empty_like(q)
    g = torch.empty((B, T, H, D), dtype=g_dtype, device=dev) if gate else None
    beta = torch.empty((B, T, H), dtype=dt, device=dev)
    es = qkv.element_size()
    base = qkv.data_ptr()
    lib = _lib.load()
    rc = lib.kda_layer_producer_fwd(
        base, base + HD * es, base + 2 * HD * es, _ptr(xf), _ptr(xb), ld_x, ld_f, ld_b,
        _ptr(conv_w), _ptr(conv_b), _ptr(dt_bias), _ptr(A_log),
        _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta),
        B, T, H, D, float(scale), float(beta_mult), _DTYPE_CODE[dt], _DTYPE_CODE[g_dtype], _stream(dev))
    _lib.check(rc, "kda_layer_producer_fwd")
    return q, k, v, g, beta


def producer_backward(qkv, xf, xb, conv_w, conv_b, dt_bias, A_log, dq, dk, dv, dg, dbeta,
                      num_heads: int, head_dim: int, scale: float, beta_mult: float = 1.0):
    """VJP of ``producer_forward``: returns (dqkv, dxf, dxb, dconv_w, dconv_b,
    ddt_bias, dA_log); the parameter gradients are fp32."""
    H, D = num_heads, head_dim
    HD = H * D
    dt = qkv.dtype
    gate = xf is not None
    qkv = _vec_ok(qkv)
    B, T, _ = qkv.shape
    if xb.stride(-1) != 1 or (B > 1 and xb.stride(0) != T * xb.stride(1)):
        xb = xb.contiguous()
    ld_x, ld_b = _rows(qkv, "qkv"), _rows(xb, "xb")
    dq, dk, dv = (t.to(dt).contiguous() for t in (dq, dk, dv))
    dbeta = dbeta.to(dt).contiguous()
    conv_w = conv_w.to(torch.float32).contiguous()
    conv_b = None if conv_b is None else conv_b.to(torch.float32).contiguous()
    dev = qkv.device
    f32 = dict(dtype=torch.float32, device=dev)
    ld_f, g_dtype = 0, torch.float32
    if gate:
        xf = _vec_ok(xf)
        ld_f = _rows(xf, "xf")
        g_dtype = dg.dtype
        dg = dg.contiguous()
        dt_bias = dt_bias.to(torch.float32).contiguous()
        A_log = A_log.to(torch.float32).contiguous()
        dxf = torch.empty((B, T, HD), dtype=dt, device=dev)
        ddt = torch.empty((HD,), **f32)
        dA = torch.empty((H,), **f32)
    else:
        dg = dt_bias = A_log = dxf = ddt = dA = None
    dqkv = torch.empty((B, T, 3 * HD), dtype=dt, device=dev)
    dxb = torch.empty((B, T, H), dtype=dt, device=dev)
    dconv_w = torch.empty((3, HD, CONV_TAPS), **f32)
    dconv_b = None if conv_b is None else torch.empty((3, HD), **f32)
    lib = _lib.load()
    nws = lib.kda_layer_workspace_size(_lib.KDA_LAYER_PRODUCER, B, T, H, D)
    ws = torch.empty(max(nws, 256), dtype=torch.uint8, device=dev)
    es = qkv.element_size()
    base, dbase = qkv.data_ptr(), dqkv.data_ptr()
    rc = lib.kda_layer_producer_bwd(
        base, base + HD * es, base + 2 * HD * es, _ptr(xf), _ptr(xb), ld_x, ld_f, ld_b,
        _ptr(conv_w), _ptr(conv_b), _ptr(dt_bias), _ptr(A_log),
        _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dg), _ptr(dbeta),
        dbase, dbase + HD * es, dbase + 2 * HD * es, _ptr(dxf), _ptr(dxb), 3 * HD, HD if gate else 0, H,
        _ptr(dconv_w), _ptr(dconv_b), _ptr(ddt), _ptr(dA),
        B, T, H, D, float(scale), float(beta_mult), _DTYPE_CODE[dt], _DTYPE_CODE[g_dtype],
        _ptr(ws), ws.numel(), _stream(dev))
    _lib.check(rc, "kda_layer_producer_bwd")
    return dqkv, dxf, dxb, dconv_w, dconv_b, ddt, dA


def gated_rmsnorm_forward(o: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """rms_norm(o) * weight * sigmoid(z) per head: o (B, T, H, D), z (B, T, H*D)
    -> (B, T, H*D) in o's dtype."""
    B, T, H, D = o.shape
    o = o.contiguous()
    z = _vec_ok(z)
    if tuple(z.shape) != (B, T, H * D):
        raise ValueError(f"gate shape {tuple(z.shape)} != {(B, T, H * D)}")
    _check_dtype("gate", z, o.dtype)
    w = weight.to(torch.float32).contiguous()
    y = torch.empty((B, T, H * D), dtype=o.dtype, device=o.device)
    rc = _lib.load().kda_layer_gated_rmsnorm_fwd(_ptr(o), _ptr(z), _rows(z, "gate"), _ptr(w), _ptr(y), H * D,
                                                 B * T, H, D, float(eps), _DTYPE_CODE[o.dtype], _stream(o.device))
    _lib.check(rc, "kda_layer_gated_rmsnorm_fwd")
    return y


def gated_rmsnorm_backward(o, z, weight, eps, dy):
    """VJP of ``gated_rmsnorm_forward``: returns (do, dz, dweight fp32)."""
    B, T, H, D = o.shape
    o = o.contiguous()
    z = _vec_ok(z)
    dy = _vec_ok(dy.to(o.dtype))
    w = weight.to(torch.float32).contiguous()
    dev = o.device
    do = torch.empty_like(o)
    dz = torch.empty((B, T, H * D), dtype=o.dtype, device=dev)
    dw = torch.empty((D,), dtype=torch.float32, device=dev)
    lib = _lib.load()
    nws = lib.kda_layer_workspace_size(_lib.KDA_LAYER_RMSNORM, B, T, H, D)
    ws = torch.empty(max(nws, 256), dtype=torch.uint8, device=dev)
    rc = lib.kda_layer_gated_rmsnorm_bwd(_ptr(o), _ptr(z), _rows(z, "gate"), _ptr(w), _ptr(dy), _rows(dy, "dy"),
                                         _ptr(do), _ptr(dz), H * D, _ptr(dw), B * T, H, D, float(eps),
                                         _DTYPE_CODE[o.dtype], _ptr(ws), ws.numel(), _stream(dev))
    _lib.check(rc, "kda_layer_gated_rmsnorm_bwd")
    return do, dz, dw


class ProducerFunction(torch.autograd.Function):
    """Autograd wrapper of the producer kernels."""

    @staticmethod
    def forward(ctx, qkv, xf, xb, conv_w, conv_b, dt_bias, A_log, num_heads, head_dim, scale, beta_mult,
                g_dtype):
        out = producer_forward(qkv, xf, xb, conv_w, conv_b, dt_bias, A_log, num_heads, head_dim, scale,
                               beta_mult, g_dtype)
        ctx.save_for_backward(qkv, xf, xb, conv_w, conv_b, dt_bias, A_log)
        ctx.cfg = (num_heads, head_dim, scale, beta_mult)
        ctx.pdtypes = tuple(None if t is None else t.dtype for t in (conv_w, conv_b, dt_bias, A_log))
        return out

    @staticmethod
    def backward(ctx, dq, dk, dv, dg, dbeta):
        qkv, xf, xb, conv_w, conv_b, dt_bias, A_log = ctx.saved_tensors
        H, D, scale, beta_mult = ctx.cfg
        B, T, _ = qkv.shape
        z = dict(device=qkv.device)
        dq = torch.zeros((B, T, H, D), dtype=qkv.dtype, **z) if dq is None else dq
        dk = torch.zeros((B, T, H, D), dtype=qkv.dtype, **z) if dk is None else dk
        dv = torch.zeros((B, T, H, D), dtype=qkv.dtype, **z) if dv is None else dv
        if xf is not None and dg is None:
            dg = torch.zeros((B, T, H, D), dtype=torch.float32, **z)
        dbeta = torch.zeros((B, T, H), dtype=qkv.dtype, **z) if dbeta is None else dbeta
        dqkv, dxf, dxb, dcw, dcb, ddt, dA = producer_backward(
            qkv, xf, xb, conv_w, conv_b, dt_bias, A_log, dq, dk, dv, dg, dbeta, H, D, scale, beta_mult)
        wt, bt, dtt, at = ctx.pdtypes
        cast = lambda t, d: None if t is None else t.to(d)  # noqa: E731
        return (dqkv, dxf, dxb, dcw.to(wt), cast(dcb, bt), cast(ddt, dtt), cast(dA, at),
                None, None, None, None, None)


class GatedRMSNormFunction(torch.autograd.Function):
    """Autograd wrapper of the gated RMSNorm kernels."""

    @staticmethod
    def forward(ctx, o, z, weight, eps):
        y = gated_rmsnorm_forward(o, z, weight, eps)
        ctx.save_for_backward(o, z, weight)
        ctx.eps = eps
        return y

    @staticmethod
    def backward(ctx, dy):
        o, z, weight = ctx.saved_tensors
        do, dz, dw = gated_rmsnorm_backward(o, z, weight, ctx.eps, dy)
        return do, dz, dw.to(weight.dtype), None


class ChunkKDAGatedFunction(torch.autograd.Function):
    """The recurrence and the output norm as one autograd node: the forward
    runs ``kda_fwd_gated`` (norm fused into the store of o; with a gradient
    needed, the training forward, whose workspace the backward reuses), the
    backward runs the norm's adjoint and then the recurrence's VJP."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, initial_state, gate, norm_weight, eps):
        train = any(ctx.needs_input_grad)
        y, o, s_final, ws = kda_forward_gated(q, k, v, g, beta, initial_state, gate, norm_weight, eps, train=train)
        ctx.save_for_backward(q, k, v, g, beta, initial_state, o, gate, norm_weight)
        ctx.ws = ws if train else None
        ctx.eps = eps
        ctx.has_state = initial_state is not None
        return y, s_final

    @staticmethod
    def backward(ctx, dy, ds_final):
        q, k, v, g, beta, s0, o, gate, w = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros(gate.shape, dtype=o.dtype, device=o.device)
        do, dz, dw = gated_rmsnorm_backward(o, gate, w, ctx.eps, dy)
        if ctx.ws is not None:
            dq, dk, dv, dg, dbeta, ds0 = kda_backward_train(q, k, v, g, beta, s0, do, ds_final, ctx.ws)
            ctx.ws = None
        else:
            dq, dk, dv, dg, dbeta, ds0 = kda_backward(q, k, v, g, beta, s0, do, ds_final)
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype), dbeta.to(beta.dtype),
                ds0 if ctx.has_state else None, dz.to(gate.dtype), dw.to(w.dtype), None)


class ShortCausalConv1d(nn.Module):
    """Parameter holder of one depthwise causal conv (nope_gdn_mlx.py:409-431):
    ``weight (channels, kernel_size, 1)`` U(+-1/sqrt(K)), ``bias (channels,)``
    zeros.  The convolution itself runs inside the producer kernel."""

    def __init__(self, channels: int, kernel_size: int = CONV_TAPS, bias: bool = True):
        super().__init__()
        if kernel_size != CONV_TAPS:
            raise ValueError(f"kernel_size={kernel_size}: the producer kernel implements {CONV_TAPS} taps")
        self.channels = channels
        self.kernel_size = kernel_size
        s = 1.0 / math.sqrt(kernel_size)
        self.weight = nn.Parameter(torch.empty(channels, kernel_size, 1).uniform_(-s, s))
        self.bias = nn.Parameter(torch.zeros(channels)) if bias else None


class RMSNormGated(nn.Module):
    """Parameter holder of the output norm (nope_gdn_mlx.py:353-366)."""

    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        """x (B, T, H, D), gate (B, T, H*D) -> (B, T, H*D)."""
        return GatedRMSNormFunction.apply(x, gate, self.weight, self.eps)


class GatedDeltaLayer(nn.Module):
    """Channel-wise KDA layer (nope_gdn_mlx.py:653-885) on the HIP path.

    ``forward(x, state=None, compute_path=None) -> (out, new_state)`` with
    x (B, L, hidden_size) and state (B, H, D, D) fp32 or None.  Construction
    raises ``ValueError`` for configurations the HIP path cannot run, as the
    reference does for its Metal budgets (nope_gdn_mlx.py:693-735).  With
    ``channel_wise_decay=False`` it is the original scalar-alpha GDN
    (``a_proj``, path ``hip_chunkwise_gdn``)."""

    def __init__(self, hidden_size: int, num_heads: int = 6, head_dim: int = 64, chunk_size: int = CHUNK,
                 channel_wise_decay: bool = True, decay_low_rank: Optional[int] = None,
                 allow_neg_eigval: bool = False, compute_path: Optional[str] = None):
        super().__init__()
        if compute_path is None:
            compute_path = HIP_PATH if channel_wise_decay else GDN_HIP_PATH
        if head_dim not in FWD_HEAD_DIMS:
            raise ValueError(f"compute_path='{compute_path}' supports head_dim in {FWD_HEAD_DIMS}; "
                             f"got head_dim={head_dim}")
        if num_heads * head_dim > 2048:
            raise ValueError(f"num_heads * head_dim = {num_heads * head_dim} exceeds the producer's 2048")
        # the output norm gives a head D / 4 lanes rounded up to a power of two,
        # and a row at most 8 waves of 64 lanes
        lanes = 1 << max(0, (head_dim // 4 - 1).bit_length())
        if -(-num_heads // max(1, 64 // lanes)) > 8:
            raise ValueError(f"num_heads={num_heads} heads of head_dim={head_dim} exceed the output norm's "
                             f"512 threads a row")
        self.recurrence = KDARecurrence(num_heads, head_dim, chunk_size, channel_wise_decay, compute_path,
                                        requires_grad=head_dim in BWD_HEAD_DIMS)
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.chunk_size = chunk_size
        self.channel_wise_decay = channel_wise_decay
        self.allow_neg_eigval = allow_neg_eigval
        self.compute_path = compute_path
        self.scale = head_dim ** -0.5
        total = num_heads * head_dim
        self.total_dim = total

        self.q_proj = nn.Linear(hidden_size, total, bias=False)
        self.k_proj = nn.Linear(hidden_size, total, bias=False)
        self.v_proj = nn.Linear(hidden_size, total, bias=False)
        if channel_wise_decay:
            rank = decay_low_rank or head_dim
            self.f_proj_1 = nn.Linear(hidden_size, rank, bias=False)
            self.f_proj_2 = nn.Linear(rank, total, bias=False)
            self.A_log = nn.Parameter(torch.empty(num_heads).uniform_(1.0, 16.0).log_())
            self.dt_bias = nn.Parameter(torch.zeros(total))
        else:
            self.a_proj = nn.Linear(hidden_size, num_heads, bias=False)
        self.b_proj = nn.Linear(hidden_size, num_heads, bias=False)
        self.q_conv1d = ShortCausalConv1d(total, CONV_TAPS)
        self.k_conv1d = ShortCausalConv1d(total, CONV_TAPS)
        self.v_conv1d = ShortCausalConv1d(total, CONV_TAPS)
        self.g_proj_1 = nn.Linear(hidden_size, head_dim, bias=False)
        self.g_proj_2 = nn.Linear(head_dim, total, bias=True)
        self.o_norm = RMSNormGated(head_dim, eps=1e-5)
        self.o_proj = nn.Linear(total, hidden_size, bias=False)
        # True fuses the output norm into the recurrence's store where a kernel
        # has it (kda_fwd_gated).  Off by default: the fused forward measured
        # slower than the plain forward plus the standalone norm kernel
        self.fused_output_norm = False

    def produce(self, x: torch.Tensor):
        """(q, k, v, g, beta) for x (B, L, hidden): the layer's inputs to the
        recurrence (nope_gdn_mlx.py:790-833); g is fp32 as in the reference.
        With scalar-alpha decay the fourth entry is alpha (B, L, H)."""
        H, D = self.num_heads, self.head_dim
        w_qkv = torch.cat([self.q_proj.weight, self.k_proj.weight, self.v_proj.weight], 0)
        qkv = F.linear(x, w_qkv)
        xb = self.b_proj(x)
        convs = (self.q_conv1d, self.k_conv1d, self.v_conv1d)
        conv_w = torch.stack([c.weight.reshape(self.total_dim, CONV_TAPS) for c in convs])
        conv_b = None if convs[0].bias is None else torch.stack([c.bias for c in convs])
        mult = 2.0 if self.allow_neg_eigval else 1.0
        if self.channel_wise_decay:
            xf = self.f_proj_2(self.f_proj_1(x))
            return ProducerFunction.apply(qkv, xf, xb, conv_w, conv_b, self.dt_bias, self.A_log, H, D,
                                          self.scale, mult, torch.float32)
        # scalar-alpha GDN: alpha = sigmoid(a_proj(x)) (nope_gdn_mlx.py:821-823), no decay gate
        q, k, v, _, beta = ProducerFunction.apply(qkv, None, xb, conv_w, conv_b, None, None, H, D, self.scale,
                                                  mult, torch.float32)
        return q, k, v, torch.sigmoid(self.a_proj(x)), beta

    def forward(self, x: torch.Tensor, state: Optional[torch.Tensor] = None,
                compute_path: Optional[str] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        if x.dim() != 3 or x.shape[-1] != self.hidden_size:
            raise ValueError(f"x must be (B, L, {self.hidden_size}); got {tuple(x.shape)}")
        q, k, v, g, beta = self.produce(x)
        gate = self.g_proj_2(self.g_proj_1(x))
        path = compute_path or self.compute_path
        if (self.fused_output_norm and path == HIP_PATH and self.channel_wise_decay and gate.dtype == q.dtype
                and gated_supported(self.head_dim, q.dtype)):
            y, new_state = ChunkKDAGatedFunction.apply(q, k, v, g, beta, state, gate, self.o_norm.weight,
                                                       self.o_norm.eps)
        else:
            o, new_state = self.recurrence(q, k, v, g, beta, state, compute_path)
            y = self.o_norm(o, gate)
        return self.o_proj(y), new_state
