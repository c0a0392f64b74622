"""Torch CPU restatement of the reference's KDA recurrence -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may use this module.  It is the checker, never the product.

Every function names the reference code it restates (paths are relative to the
HananKibria/MLX_VIT repository).  The reference runs on MLX, which is absent
here, so each MLX primitive is replaced by its torch equivalent:
``mx.cumsum(reverse=True)`` by a flipped cumsum, ``mx.swapaxes`` by
``transpose``, the Metal triangular-solve kernels by the same per-column
substitution loops.

All functions are dtype-generic: pass float64 tensors for golden values, float32
tensors to reproduce the reference's own fp32 arithmetic (the CPU baseline).

Layouts follow the reference: layer-level tensors are ``(B, L, H, D)``; the
chunkwise functions take heads folded into the batch, ``(B*H, L, D)``.  The
recurrent state is ``S[b, h, i_v, j_k]``: rows index value channels and columns
index key channels, so the per-token output is ``o_t = S_t q_t``.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Tuple

import torch

Tensor = torch.Tensor


# --------------------------------------------------------------------------
# Utilities (nope_gdn_mlx.py:77-86)
# --------------------------------------------------------------------------

def l2_normalize(x: Tensor, dim: int = -1, eps: float = 1e-12) -> Tensor:
    """nope_gdn_mlx.py:77-80: ``x / max(||x||_2, eps)`` over ``dim``."""
    norm = torch.sqrt(torch.sum(x * x, dim=dim, keepdim=True))
    return x / torch.clamp(norm, min=eps)


def softplus(x: Tensor, beta: float = 1.0) -> Tensor:
    """nope_gdn_mlx.py:83-86: stable ``log(1 + exp(beta x)) / beta``."""
    bx = beta * x
    return (torch.log1p(torch.exp(-torch.abs(bx))) + torch.clamp(bx, min=0)) / beta


# --------------------------------------------------------------------------
# Benchmark inputs (the configs' distributions; draw order is fixed)
# --------------------------------------------------------------------------

def make_inputs(B: int, T: int, H: int, D: int, *, dtype: torch.dtype = torch.float32,
                seed: int = 0, with_state: bool = False, state_std: float = 0.02,
                with_grad: bool = False, g_scale: float = 0.1) -> Dict[str, Optional[Tensor]]:
    """Seeded inputs for the KDA op, drawn in fp32 on the CPU and cast to ``dtype``.

    One ``torch.Generator('cpu')`` seeded with ``seed``; draw order q, k, v,
    beta-logits, g-logits, [S0], [dO].  q and k are N(0,1) then L2-normalised
    over D (as the layer does before the op, nope_gdn_mlx.py:796-797); v is
    N(0,1); beta = sigmoid(N(0,1)); g = -softplus(N(0,1)) * g_scale with shape
    (B, T, H, D); S0 ~ N(0, state_std^2) in the reference ``[v, k]``
    orientation, kept fp32; dO ~ N(0,1) in ``dtype``.
    """
    gen = torch.Generator(device="cpu").manual_seed(seed)
    shp = (B, T, H, D)
    q = l2_normalize(torch.randn(shp, generator=gen, dtype=torch.float32))
    k = l2_normalize(torch.randn(shp, generator=gen, dtype=torch.float32))
    v = torch.randn(shp, generator=gen, dtype=torch.float32)
    beta = torch.sigmoid(torch.randn((B, T, H), generator=gen, dtype=torch.float32))
    g = -softplus(torch.randn(shp, generator=gen, dtype=torch.float32)) * g_scale
    s0 = None
    if with_state:
        s0 = torch.randn((B, H, D, D), generator=gen, dtype=torch.float32) * state_std
    do = None
    if with_grad:
        do = torch.randn(shp, generator=gen, dtype=torch.float32).to(dtype)
    return dict(q=q.to(dtype), k=k.to(dtype), v=v.to(dtype), g=g.to(dtype),
                beta=beta.to(dtype), s0=s0, do=do)


def input_checksum(t: Tensor) -> float:
    """Order-sensitive checksum used to detect generator drift in fixtures."""
    x = t.detach().to(torch.float64).reshape(-1)
    w = torch.arange(1, x.numel() + 1, dtype=torch.float64) % 997 + 1.0
    return float(torch.sum(x * w))


# --------------------------------------------------------------------------
# Step recurrence: the 'compiled' / 'naive' paths
# --------------------------------------------------------------------------

def kda_step(state: Tensor, q_t: Tensor, k_t: Tensor, v_t: Tensor, g_t: Tensor,
             beta_t: Tensor, I: Tensor) -> Tuple[Tensor, Tensor]:
    """nope_gdn_mlx.py:616-638 (``_kda_step_fused``), op for op.

    Column-scale the state by exp(g_t), apply the delta rule in its D x D x D
    matmul form ``S (I - beta k k^T) + beta v k^T`` and read out with the
    post-update state, ``o_t = S q_t``.
    """
    decay = torch.exp(g_t)
    state = state * decay[..., None, :]
    b = beta_t[..., None, None]
    k_outer = k_t[..., :, None] @ k_t[..., None, :]
    state = state @ (I - b * k_outer)
    state = state + b * (v_t[..., :, None] @ k_t[..., None, :])
    out = (state @ q_t[..., :, None]).squeeze(-1)
    return state, out


def loop_compiled_kda(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor,
                      state: Optional[Tensor] = None,
                      compute_dtype: torch.dtype = torch.float32) -> Tuple[Tensor, Tensor]:
    """nope_gdn_mlx.py:890-917 (``_loop_compiled_kda``); same math as the naive
    loop, nope_gdn_mlx.py:2870-2892.

    q, k, v: (B, L, H, D); g: (B, L, H, D) log-decay; beta: (B, L, H);
    state: (B, H, D, D) or None.  Inputs are cast to ``compute_dtype`` (the
    reference uses fp32; the reference leaves ``g`` uncast -- it is fp32 inside
    the layer -- here it is cast too), the state starts at zero when None, and
    the output is cast back to ``q.dtype``.  Returns (o, final_state).
    """
    B, L, H, D = q.shape
    cd = compute_dtype
    q32, k32, v32, g32, b32 = (t.to(cd) for t in (q, k, v, g, beta))
    if state is None:
        state = torch.zeros((B, H, D, D), dtype=cd)
    else:
        state = state.to(cd)
    I = torch.eye(D, dtype=cd)
    outs: List[Tensor] = []
    for t in range(L):
        state, o_t = kda_step(state, q32[:, t], k32[:, t], v32[:, t], g32[:, t], b32[:, t], I)
        outs.append(o_t)
    if L == 0:
        return torch.zeros_like(q), state
    return torch.stack(outs, dim=1).to(q.dtype), state


def gdn_step(state: Tensor, q_t: Tensor, k_t: Tensor, v_t: Tensor, alpha_t: Tensor, beta_t: Tensor,
             I: Tensor) -> Tuple[Tensor, Tensor]:
    """nope_gdn_mlx.py:641-650 (``_gdn_step_fused``): scalar-alpha step,
    ``S (alpha (I - beta k k^T)) + beta v k^T``, then ``o_t = S q_t``."""
    a = alpha_t[..., None, None]
    b = beta_t[..., None, None]
    k_outer = k_t[..., :, None] @ k_t[..., None, :]
    state = state @ (a * (I - b * k_outer))
    state = state + b * (v_t[..., :, None] @ k_t[..., None, :])
    out = (state @ q_t[..., :, None]).squeeze(-1)
    return state, out


def loop_compiled_gdn(q: Tensor, k: Tensor, v: Tensor, alpha: Tensor, beta: Tensor,
                      state: Optional[Tensor] = None,
                      compute_dtype: torch.dtype = torch.float32) -> Tuple[Tensor, Tensor]:
    """nope_gdn_mlx.py:919-947 (``_loop_compiled_gdn``): q, k, v (B, L, H, D),
    alpha, beta (B, L, H); casts to ``compute_dtype``, zero state when None,
    output cast back to q's dtype.  Returns (o, final_state)."""
    B, L, H, D = q.shape
    cd = compute_dtype
    q32, k32, v32, a32, b32 = (t.to(cd) for t in (q, k, v, alpha, beta))
    state = torch.zeros((B, H, D, D), dtype=cd) if state is None else state.to(cd)
    I = torch.eye(D, dtype=cd)
    outs: List[Tensor] = []
    for t in range(L):
        state, o_t = gdn_step(state, q32[:, t], k32[:, t], v32[:, t], a32[:, t], b32[:, t], I)
        outs.append(o_t)
    if L == 0:
        return torch.zeros_like(q), state
    return torch.stack(outs, dim=1).to(q.dtype), state


def step_forward_rank1(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor,
                       state: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """Rank-1 form of the same step, nope_gdn_mlx.py:3003-3019 and 3724-3735.

    ``S' = S diag(e^g); u = beta (v - S' k); S = S' + u k^T; o = S q``.
    Folded layout: q, k, v, g (BH, L, D); beta (BH, L); state (BH, D, D).
    Returns (o, S_final, u) -- ``u`` is what the metal forward saves for its
    backward.
    """
    BH, L, D = q.shape
    S = state.clone()
    outs, us = [], []
    for t in range(L):
        S = S * torch.exp(g[:, t])[:, None, :]
        Sk = torch.einsum("bij,bj->bi", S, k[:, t])
        u = beta[:, t, None] * (v[:, t] - Sk)
        S = S + u[:, :, None] * k[:, t, None, :]
        outs.append(torch.einsum("bij,bj->bi", S, q[:, t]))
        us.append(u)
    o = torch.stack(outs, 1) if L else torch.zeros_like(q)
    u = torch.stack(us, 1) if L else torch.zeros_like(q)
    return o, S, u


def python_backward_full(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor,
                         u: Tensor, state_init: Tensor, dout: Tensor,
                         dstate_final: Tensor) -> Tuple[Tensor, ...]:
    """nope_gdn_mlx.py:3185-3295 (``_kda_python_backward_full``).

    Replays the forward from the saved ``u`` to materialise every state, then
    walks time backwards.  Folded layout (BH, L, D).  Returns
    (dq, dk, dv, dg, dbeta, dstate_init).
    """
    BH, L, D = q.shape
    S_list = [state_init]
    S_cur = state_init
    for t in range(L):
        S_prime = S_cur * torch.exp(g[:, t])[:, None, :]
        S_cur = S_prime + u[:, t, :, None] * k[:, t, None, :]
        S_list.append(S_cur)
    gS = dstate_final
    dq_r, dk_r, dv_r, dg_r, db_r = [], [], [], [], []
    for t in range(L - 1, -1, -1):
        q_t, k_t, v_t, g_t, u_t = q[:, t], k[:, t], v[:, t], g[:, t], u[:, t]
        beta_t, do_t = beta[:, t], dout[:, t]
        decay = torch.exp(g_t)
        S_t = S_list[t + 1]
        S_prime = S_t - u_t[:, :, None] * k_t[:, None, :]
        gS = gS + do_t[:, :, None] * q_t[:, None, :]
        ud = torch.sum(u_t * do_t, dim=-1, keepdim=True)
        dq_r.append(torch.einsum("blj,bl->bj", S_prime, do_t) + k_t * ud)
        du = torch.einsum("bij,bj->bi", gS, k_t)
        dk_outer = torch.einsum("bij,bi->bj", gS, u_t)
        Sk = torch.einsum("bij,bj->bi", S_prime, k_t)
        w = v_t - Sk
        db_r.append(torch.sum(du * w, dim=-1))
        dw = beta_t[:, None] * du
        dv_r.append(dw)
        dS_prime = gS - dw[:, :, None] * k_t[:, None, :]
        dk_r.append(dk_outer - torch.einsum("blj,bl->bj", S_prime, dw))
        dg_r.append(torch.sum(dS_prime * S_prime, dim=-2))
        gS = dS_prime * decay[:, None, :]

    def _st(lst):
        return torch.stack(lst[::-1], 1) if lst else torch.zeros_like(q)
    dbeta = torch.stack(db_r[::-1], 1) if db_r else torch.zeros_like(beta)
    return _st(dq_r), _st(dk_r), _st(dv_r), _st(dg_r), dbeta, gS


# --------------------------------------------------------------------------
# Triangular solves (the Metal kernels' substitution order)
# --------------------------------------------------------------------------

def solve_unit_lower(L: Tensor, b: Tensor) -> Tensor:
    """nope_gdn_mlx.py:1098-1140 (``_tri_solve_metal_source``): ``y = L^-1 b``
    for unit-lower L (BH, C, C) -- only the strict lower part of L is read --
    by per-column forward substitution, row i after rows < i."""
    BH, C, _ = L.shape
    y = torch.zeros_like(b)
    for i in range(C):
        yi = b[:, i, :].clone()
        if i:
            yi = yi - torch.einsum("bk,bkd->bd", L[:, i, :i], y[:, :i, :])
        y[:, i, :] = yi
    return y


def solve_unit_upper(U: Tensor, b: Tensor) -> Tensor:
    """nope_gdn_mlx.py:1209-1242 (``_tri_solve_upper_metal_source``): ``y = U^-1 b``
    for unit-upper U by back substitution, row C-1 first."""
    BH, C, _ = U.shape
    y = torch.zeros_like(b)
    for i in range(C - 1, -1, -1):
        yi = b[:, i, :].clone()
        if i + 1 < C:
            yi = yi - torch.einsum("bk,bkd->bd", U[:, i, i + 1:], y[:, i + 1:, :])
        y[:, i, :] = yi
    return y


# --------------------------------------------------------------------------
# Chunkwise WY algebra (forward and hand-derived backward)
# --------------------------------------------------------------------------

def chunk_consts(C: int, dtype: torch.dtype) -> Dict[str, Tensor]:
    """nope_gdn_mlx.py:453-470: identity, inclusive causal, strict-lower and
    inclusive-upper masks."""
    ones = torch.ones((C, C), dtype=dtype)
    return {"I_CC": torch.eye(C, dtype=dtype), "causal": torch.tril(ones),
            "A_mask": torch.tril(ones, -1), "O_mask": torch.triu(ones, 0)}


def chunk_preamble(g_c: Tensor, k_c: Tensor, v_c: Tensor, beta_c: Tensor):
    """nope_gdn_mlx.py:549-582 (``_kda_chunk_preamble_no_M``): gamma = in-chunk
    cumsum of g; exp(gamma); K_proj = e^gamma K; K_back = e^(gamma_C - gamma) K;
    beta V."""
    gamma = torch.cumsum(g_c, dim=-2)
    exp_gamma = torch.exp(gamma)
    K_proj = exp_gamma * k_c
    K_back = torch.exp(gamma[..., -1:, :] - gamma) * k_c
    rhs_pre = beta_c[..., :, None] * v_c
    return gamma, exp_gamma, K_proj, K_back, rhs_pre


def compute_M_Moq(K: Tensor, Q: Tensor, gamma: Tensor) -> Tuple[Tensor, Tensor]:
    """nope_gdn_mlx.py:1301-1336 (``_M_kernel_source``):
    ``M[s,t] = sum_d K[s,d] K[t,d] exp(min(gamma[t,d]-gamma[s,d], 0))`` and the
    same with Q[t] for ``M_oq``.  Pairwise exponent, never factorised."""
    diff = gamma[..., None, :, :] - gamma[..., :, None, :]      # [..., s, t, d] = g_t - g_s
    ed = torch.exp(torch.clamp(diff, max=0.0))
    M = torch.einsum("...sd,...td,...std->...st", K, K, ed)
    M_oq = torch.einsum("...sd,...td,...std->...st", K, Q, ed)
    return M, M_oq


def build_IA_and_Moq_T(M, M_oq, beta_c, A_mask, I_C, O_mask):
    """nope_gdn_mlx.py:585-597: ``IA = I + beta_i M^T`` (strict lower) and the
    inclusive-lower masked ``M_oq^T``."""
    A = beta_c[..., :, None] * M.transpose(-1, -2) * A_mask
    return I_C + A, M_oq.transpose(-1, -2) * O_mask.transpose(-1, -2)


def _pad_folded(q, k, v, g, beta, C):
    """nope_gdn_mlx.py:2354-2361: pad L to a multiple of C with g=0, beta=0
    (and zero q/k/v), so padded steps neither decay nor write."""
    BH, L, D = q.shape
    pad = (C - L % C) % C
    if pad:
        z = lambda t: torch.zeros((BH, pad) + t.shape[2:], dtype=t.dtype)
        q, k, v, g, beta = (torch.cat([t, z(t)], 1) for t in (q, k, v, g, beta))
    return q, k, v, g, beta, pad


def chunkwise_forward(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor,
                      state: Optional[Tensor], C: int, return_traj: bool = False):
    """nope_gdn_mlx.py:2318-2456 (``_chunkwise_kda_forward``) and 2484-2571
    (``_chunkwise_kda_with_traj``), unfused variant (rhs 600-603, solve,
    finalize 606-613).  Folded layout (BH, L, D); returns (o, S_final) or, with
    ``return_traj``, (o, S_final, U_traj, S_traj)."""
    BH, L, D = q.shape
    dt = q.dtype
    q, k, v, g, beta, pad = _pad_folded(q, k, v, g, beta, C)
    nc = q.shape[1] // C
    q_c, k_c, v_c, g_c = (t.reshape(BH, nc, C, D) for t in (q, k, v, g))
    beta_c = beta.reshape(BH, nc, C)
    state = torch.zeros((BH, D, D), dtype=dt) if state is None else state.to(dt)
    cs = chunk_consts(C, dt)
    gamma, exp_gamma, K_proj, K_back, rhs_pre = chunk_preamble(g_c, k_c, v_c, beta_c)
    M, M_oq = compute_M_Moq(k_c, q_c, gamma)
    IA, MoqT = build_IA_and_Moq_T(M, M_oq, beta_c, cs["A_mask"], cs["I_CC"], cs["O_mask"])
    Q_prime = exp_gamma * q_c
    outs, Us, Ss = [], [], [state]
    for ci in range(nc):
        rhs = rhs_pre[:, ci] - beta_c[:, ci, :, None] * (K_proj[:, ci] @ state.transpose(-1, -2))
        U = solve_unit_lower(IA[:, ci], rhs)
        O = Q_prime[:, ci] @ state.transpose(-1, -2) + MoqT[:, ci] @ U
        state = exp_gamma[:, ci, -1, :][:, None, :] * state + U.transpose(-1, -2) @ K_back[:, ci]
        outs.append(O); Us.append(U); Ss.append(state)
    o = torch.cat(outs, 1)[:, :L] if nc else torch.zeros((BH, 0, D), dtype=dt)
    if return_traj:
        return o, state, torch.stack(Us, 1), torch.stack(Ss, 1)
    return o, state


def _M_Moq_backward(K, Q, gamma, dM, dM_oq):
    """Adjoint of ``compute_M_Moq`` (the job of nope_gdn_mlx.py:2080-2229),
    written from the pairwise definition: the clipped exponent has zero
    derivative where ``gamma_t - gamma_s > 0``."""
    diff = gamma[..., None, :, :] - gamma[..., :, None, :]      # [s, t, d]
    active = (diff <= 0).to(K.dtype)
    ed = torch.exp(torch.clamp(diff, max=0.0))
    dK = (torch.einsum("...st,...td,...std->...sd", dM, K, ed)
          + torch.einsum("...st,...sd,...std->...td", dM, K, ed)
          + torch.einsum("...st,...td,...std->...sd", dM_oq, Q, ed))
    dQ = torch.einsum("...st,...sd,...std->...td", dM_oq, K, ed)
    # d/dgamma of exp(gamma_t - gamma_s) on the active set
    w = (torch.einsum("...st,...sd,...td->...std", dM, K, K)
         + torch.einsum("...st,...sd,...td->...std", dM_oq, K, Q)) * ed * active
    dgamma = w.sum(dim=-3) - w.sum(dim=-2)                       # +d/dg_t, -d/dg_s
    return dK, dQ, dgamma


def chunkwise_backward(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor,
                       state: Optional[Tensor], dout: Tensor,
                       dstate_final: Optional[Tensor], C: int):
    """nope_gdn_mlx.py:2579-2720 (``_chunkwise_kda_backward``) with the padding
    and cotangent handling of 2746-2808.  Folded layout.  Returns
    (dq, dk, dv, dg, dbeta, dstate_init), unpadded."""
    BH, L, D = q.shape
    dt = q.dtype
    _, _, U_traj, S_traj = chunkwise_forward(q, k, v, g, beta, state, C, return_traj=True)
    q, k, v, g, beta, pad = _pad_folded(q, k, v, g, beta, C)
    if pad:
        dout = torch.cat([dout, torch.zeros((BH, pad, D), dtype=dout.dtype)], 1)
    nc = q.shape[1] // C
    q_c, k_c, v_c, g_c, dO_all = (t.reshape(BH, nc, C, D) for t in (q, k, v, g, dout))
    beta_c = beta.reshape(BH, nc, C)
    cs = chunk_consts(C, dt)
    I_C, A_mask, O_mask = cs["I_CC"], cs["A_mask"], cs["O_mask"]
    dstate = torch.zeros((BH, D, D), dtype=dt) if dstate_final is None else dstate_final.to(dt)
    res = {n: [] for n in ("dq", "dk", "dv", "dg", "db")}
    for ci in range(nc - 1, -1, -1):
        S, U = S_traj[:, ci], U_traj[:, ci]
        Qc, Kc, Vc, Gc, Bc = q_c[:, ci], k_c[:, ci], v_c[:, ci], g_c[:, ci], beta_c[:, ci]
        gamma = torch.cumsum(Gc, dim=-2)
        gamma_last = gamma[:, -1, :]
        exp_gamma = torch.exp(gamma)
        exp_gamma_last = exp_gamma[:, -1, :]
        K_proj = exp_gamma * Kc
        Q_prime = exp_gamma * Qc
        K_back = torch.exp(gamma_last[:, None, :] - gamma) * Kc
        M, M_oq = compute_M_Moq(Kc, Qc, gamma)
        IA = I_C + Bc[:, :, None] * M.transpose(-1, -2) * A_mask
        MoqT = M_oq.transpose(-1, -2) * O_mask.transpose(-1, -2)
        y = Vc - K_proj @ S.transpose(-1, -2)
        dO = dO_all[:, ci]
        # (1) state update
        dexp_last_S = torch.sum(S * dstate, dim=-2)
        dS_decay = exp_gamma_last[..., None, :] * dstate
        dU_S = K_back @ dstate.transpose(-1, -2)
        dK_back = U @ dstate
        # (2) output
        dQ_prime = dO @ S
        dS_O = dO.transpose(-1, -2) @ Q_prime
        dMoqT = dO @ U.transpose(-1, -2)
        dU_O = MoqT.transpose(-1, -2) @ dO
        dU = dU_S + dU_O
        # (3) solve
        drhs = solve_unit_upper(IA.transpose(-1, -2), dU)
        dIA = -torch.tril(drhs @ U.transpose(-1, -2), -1)
        # (4) rhs = beta * y
        db_rhs = torch.sum(drhs * y, dim=-1)
        dy = drhs * Bc[..., None]
        dK_proj = -dy @ S
        dS_rhs = -dy.transpose(-1, -2) @ K_proj
        # (5) IA
        dM = (dIA * Bc[..., None] * A_mask).transpose(-1, -2)
        db_IA = torch.sum(dIA * M.transpose(-1, -2) * A_mask, dim=-1)
        # (6) M_oq
        dM_oq = dMoqT.transpose(-1, -2) * O_mask
        # (7) pairwise products
        dK_M, dQ_M, dgam_M = _M_Moq_backward(Kc, Qc, gamma, dM, dM_oq)
        # (8)-(9) exponentials
        dgam = dgam_M + dK_proj * K_proj + dQ_prime * Q_prime - dK_back * K_back
        dgam_last = torch.sum(dK_back * K_back, dim=-2) + dexp_last_S * exp_gamma_last
        dgam = torch.cat([dgam[:, :-1], dgam[:, -1:] + dgam_last[:, None, :]], 1)
        # (10) reverse cumsum
        res["dg"].append(torch.flip(torch.cumsum(torch.flip(dgam, [1]), 1), [1]))
        res["dv"].append(dy)
        res["dk"].append(dK_M + dK_proj * exp_gamma
                         + dK_back * torch.exp(gamma_last[:, None, :] - gamma))
        res["dq"].append(dQ_M + dQ_prime * exp_gamma)
        res["db"].append(db_rhs + db_IA)
        # (13) carry
        dstate = dS_decay + dS_O + dS_rhs
    out = []
    for n in ("dq", "dk", "dv", "dg"):
        out.append(torch.cat(res[n][::-1], 1)[:, :L] if nc else torch.zeros((BH, 0, D), dtype=dt))
    dbeta = torch.cat(res["db"][::-1], 1)[:, :L] if nc else torch.zeros((BH, 0), dtype=dt)
    return out[0], out[1], out[2], out[3], dbeta, dstate


# --------------------------------------------------------------------------
# Head folding (nope_gdn_mlx.py:2841-2854, 2858-2865)
# --------------------------------------------------------------------------

def fold_heads(x: Tensor) -> Tensor:
    """(B, L, H, D) -> (B*H, L, D); (B, L, H) -> (B*H, L)."""
    if x.dim() == 4:
        B, L, H, D = x.shape
        return x.permute(0, 2, 1, 3).reshape(B * H, L, D)
    B, L, H = x.shape
    return x.permute(0, 2, 1).reshape(B * H, L)


def unfold_heads(x: Tensor, B: int, H: int) -> Tensor:
    """Inverse of ``fold_heads``."""
    if x.dim() == 3:
        BH, L, D = x.shape
        return x.reshape(B, H, L, D).permute(0, 2, 1, 3)
    BH, L = x.shape
    return x.reshape(B, H, L).permute(0, 2, 1)


def autograd_reference(q, k, v, g, beta, s0, do, ds_final=None,
                       compute_dtype: torch.dtype = torch.float64):
    """Gradients of ``loop_compiled_kda`` by torch autograd -- the derivative MLX
    autograd takes through ``_kda_step_fused``.  Layer layout.  Returns a dict
    with o, s_final, dq, dk, dv, dg, dbeta, ds0 (all in ``compute_dtype``)."""
    cd = compute_dtype
    leaves = [t.detach().to(cd).requires_grad_(True) for t in (q, k, v, g, beta)]
    B, L, H, D = q.shape
    st = (torch.zeros((B, H, D, D), dtype=cd) if s0 is None else s0.detach().to(cd))
    st = st.requires_grad_(True)
    o, sf = loop_compiled_kda(*leaves, st, compute_dtype=cd)
    loss = torch.sum(o * do.to(cd))
    if ds_final is not None:
        loss = loss + torch.sum(sf * ds_final.to(cd))
    grads = torch.autograd.grad(loss, leaves + [st], allow_unused=True)
    out = dict(o=o.detach(), s_final=sf.detach())
    for n, gr, ref in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), grads, leaves + [st]):
        out[n] = torch.zeros_like(ref) if gr is None else gr.detach()
    return out


def rel_l2(a: Tensor, b: Tensor) -> float:
    """``||a - b||_2 / max(||b||_2, tiny)`` in float64."""
    a = a.detach().to(torch.float64)
    b = b.detach().to(torch.float64)
    den = float(torch.linalg.vector_norm(b))
    num = float(torch.linalg.vector_norm(a - b))
    return num / max(den, 1e-300) if den > 0 else num
