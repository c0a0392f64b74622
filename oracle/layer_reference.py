"""CPU restatement of the GatedDeltaLayer around the KDA recurrence (TEST
INFRASTRUCTURE ONLY: imported by tests/, never by the product path).

Plain torch on the CPU (fp64 in the tests), one function per reference piece:

* ``short_causal_conv1d``   _depthwise_conv1d_manual / ShortCausalConv1d, nope_gdn_mlx.py:369-431
* ``producer_from_projections``  projection outputs to q, k, v, g, beta, nope_gdn_mlx.py:796-833
* ``producer``              the same from x and the layer's parameters, nope_gdn_mlx.py:790-833
* ``gated_rms_norm``        _gated_rms_norm / RMSNormGated, nope_gdn_mlx.py:340-366
* ``layer_forward``         the whole __call__, nope_gdn_mlx.py:775-885, with the
                            recurrence from ``kda_reference.loop_compiled_kda``

Pinned by tests/test_layer_oracle.py against library routines (F.conv1d,
F.rms_norm, F.softplus), closed forms (identity tap, unit row norms) and
finite differences on tiny shapes.
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor

from .kda_reference import l2_normalize, loop_compiled_gdn, loop_compiled_kda, softplus

TAPS = 4


def short_causal_conv1d(x: Tensor, weight: Tensor, bias: Optional[Tensor]) -> Tensor:
    """nope_gdn_mlx.py:369-406: x (B, L, C), weight (C, K, 1) -> (B, L, C).
    K - 1 zeros are prepended along L; out[t] = sum_k w[c, k] x_pad[t + k]."""
    B, L, C = x.shape
    K = weight.shape[1]
    xp = F.pad(x, (0, 0, K - 1, 0))
    w = weight.reshape(C, K)
    out = sum(xp[:, k:k + L, :] * w[:, k] for k in range(K))
    if bias is not None:
        out = out + bias
    return out


def producer_from_projections(xq: Tensor, xk: Tensor, xv: Tensor, xf: Tensor, xb: Tensor,
                              conv_w: Tensor, conv_b: Optional[Tensor], dt_bias: Tensor, A_log: Tensor,
                              H: int, D: int, beta_mult: float = 1.0):
    """nope_gdn_mlx.py:796-833 from the projection outputs: xq, xk, xv, xf
    (B, L, H*D), xb (B, L, H); conv_w (3, H*D, K) and conv_b (3, H*D) or None
    for the q, k, v convs.  Returns q, k, v, g (B, L, H, D) and beta (B, L, H).
    The L2 norms run over the whole H*D row (before the head split)."""
    B, L, HD = xq.shape
    cb = (None, None, None) if conv_b is None else conv_b
    convs = [short_causal_conv1d(x, conv_w[i].unsqueeze(-1), cb[i]) for i, x in enumerate((xq, xk, xv))]
    q = l2_normalize(F.silu(convs[0]), dim=-1) * (D ** -0.5)
    k = l2_normalize(F.silu(convs[1]), dim=-1)
    v = F.silu(convs[2])
    g = xf.reshape(B, L, H, D) + dt_bias.reshape(H, D)
    g = -torch.exp(A_log).reshape(1, 1, H, 1) * softplus(g)
    beta = torch.sigmoid(xb) * beta_mult
    return q.reshape(B, L, H, D), k.reshape(B, L, H, D), v.reshape(B, L, H, D), g, beta


def producer(params: Dict[str, Tensor], x: Tensor, H: int, D: int,
             allow_neg_eigval: bool = False) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """nope_gdn_mlx.py:790-833: the projections, then ``producer_from_projections``.
    For the scalar-alpha layer (an ``a_proj.weight`` parameter) the fourth
    result is alpha = sigmoid(a_proj(x)) (B, L, H)."""
    p = params
    HD = H * D
    conv_w = torch.stack([p[f"{n}_conv1d.weight"].reshape(HD, TAPS) for n in "qkv"])
    conv_b = torch.stack([p[f"{n}_conv1d.bias"] for n in "qkv"]) if "q_conv1d.bias" in p else None
    mult = 2.0 if allow_neg_eigval else 1.0
    if "a_proj.weight" in p:
        # scalar-alpha GDN (nope_gdn_mlx.py:821-823): alpha = sigmoid(a_proj(x)) in place of g
        B, L, _ = x.shape
        zeros = torch.zeros(B, L, HD, dtype=x.dtype)
        q, k, v, _, beta = producer_from_projections(
            x @ p["q_proj.weight"].T, x @ p["k_proj.weight"].T, x @ p["v_proj.weight"].T, zeros,
            x @ p["b_proj.weight"].T, conv_w, conv_b, torch.zeros(HD, dtype=x.dtype),
            torch.zeros(H, dtype=x.dtype), H, D, mult)
        return q, k, v, torch.sigmoid(x @ p["a_proj.weight"].T), beta
    return producer_from_projections(
        x @ p["q_proj.weight"].T, x @ p["k_proj.weight"].T, x @ p["v_proj.weight"].T,
        (x @ p["f_proj_1.weight"].T) @ p["f_proj_2.weight"].T, x @ p["b_proj.weight"].T,
        conv_w, conv_b, p["dt_bias"], p["A_log"], H, D, mult)


def gated_rms_norm(x: Tensor, weight: Tensor, gate: Tensor, eps: float) -> Tensor:
    """nope_gdn_mlx.py:340-350: rms_norm(x, weight, eps) * sigmoid(gate) over the last axis."""
    r = torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + eps)
    return x * r * weight * torch.sigmoid(gate)


def layer_forward(params: Dict[str, Tensor], x: Tensor, H: int, D: int, state: Optional[Tensor] = None,
                  allow_neg_eigval: bool = False, eps: float = 1e-5,
                  keep: Optional[dict] = None) -> Tuple[Tensor, Tensor]:
    """nope_gdn_mlx.py:775-885 with the 'compiled' recurrence: (out, new_state).
    keep: if a dict, receives the decay gate g (B, L, H, D) of the graph, so a
    caller can read its gradient."""
    B, L, _ = x.shape
    q, k, v, g, beta = producer(params, x, H, D, allow_neg_eigval)
    if keep is not None:
        keep["g"] = g
    if "a_proj.weight" in params:   # g is alpha (B, L, H)
        o, new_state = loop_compiled_gdn(q, k, v, g, beta, state, compute_dtype=x.dtype)
    else:
        o, new_state = loop_compiled_kda(q, k, v, g, beta, state, compute_dtype=x.dtype)
    gate = ((x @ params["g_proj_1.weight"].T) @ params["g_proj_2.weight"].T
            + params["g_proj_2.bias"]).reshape(B, L, H, D)
    y = gated_rms_norm(o.reshape(B, L, H, D), params["o_norm.weight"], gate, eps)
    return y.reshape(B, L, H * D) @ params["o_proj.weight"].T, new_state
