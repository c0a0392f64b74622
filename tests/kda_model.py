"""Float64 model of the HIP kernel decomposition (test helper, CPU only).

This is *not* the oracle.  It restates, in torch, exactly the staging the HIP
library uses -- so that a mismatch between the HIP path and the oracle can be
localised to one kernel by comparing that kernel's workspace output with the
matching tensor here.  Tests check this model against the oracle first.

State orientation inside the model and the kernels is ``Sig = S^T`` with shape
``[dk, dv]``; the reference orientation ``S[v, k]`` is restored at the ends.

Per chunk of C rows (gamma = in-chunk cumsum of g, G = gamma of the last row):

  prep      Akk[t,s] = sum_d k_t k_s e^{gamma_t - gamma_s}  (s < t)
            Aqk[t,s] = sum_d q_t k_s e^{gamma_t - gamma_s}  (s <= t)
            computed per 16-row block i with the anchor row r = 16 i:
            (k_t e^{gamma_t - gamma_r}) . (k_s e^{gamma_r - gamma_s}); every
            factor is <= 1 except on the diagonal block, where it is bounded
            by the block's decay span.
            L = diag(beta) Akk;  [W | U] = (I + L)^-1 [beta e^gamma K | beta V]
            by block forward substitution with inverted 16 x 16 diagonal blocks.
            Qp = e^gamma Q;  Kb = e^{G - gamma} K;  eG = e^G
  recur     Vp = U - W Sig;  O = Qp Sig + Aqk Vp;  Sig <- eG Sig + Kb^T Vp
  dh        dVp = Aqk^T dO + Kb dSig;  dSig <- eG dSig + Qp^T dO - W^T dVp
  local     the remaining chunk-parallel adjoints (see ``local_backward``).
"""
from __future__ import annotations

import torch

BS = 16


def _cumsum_chunks(g_c):
    return torch.cumsum(g_c, dim=-2)


def prep(q_c, k_c, v_c, g_c, beta_c):
    """Inputs (N, C, D) / (N, C) float64 (N = chunks).  Returns a dict."""
    N, C, D = k_c.shape
    gam = _cumsum_chunks(g_c)
    G = gam[:, -1, :]
    Akk = torch.zeros((N, C, C), dtype=k_c.dtype)
    Aqk = torch.zeros((N, C, C), dtype=k_c.dtype)
    for i in range(C // BS):
        r = BS * i
        t = slice(r, r + BS)
        Kl = k_c[:, t] * torch.exp(gam[:, t] - gam[:, r:r + 1])
        Ql = q_c[:, t] * torch.exp(gam[:, t] - gam[:, r:r + 1])
        Kr = k_c[:, :r + BS] * torch.exp(gam[:, r:r + 1] - gam[:, :r + BS])
        Akk[:, t, :r + BS] = Kl @ Kr.transpose(-1, -2)
        Aqk[:, t, :r + BS] = Ql @ Kr.transpose(-1, -2)
    Akk = torch.tril(Akk, -1)
    Aqk = torch.tril(Aqk, 0)
    L = beta_c[:, :, None] * Akk
    I16 = torch.eye(BS, dtype=k_c.dtype)
    Tii = [torch.linalg.inv(I16 + L[:, BS * i:BS * i + BS, BS * i:BS * i + BS]) for i in range(C // BS)]
    R = torch.cat([beta_c[:, :, None] * torch.exp(gam) * k_c, beta_c[:, :, None] * v_c], -1)
    X = []
    for i in range(C // BS):
        Y = R[:, BS * i:BS * i + BS].clone()
        for j in range(i):
            Y = Y - L[:, BS * i:BS * i + BS, BS * j:BS * j + BS] @ X[j]
        X.append(Tii[i] @ Y)
    X = torch.cat(X, 1)
    return dict(gam=gam, G=G, Akk=Akk, Aqk=Aqk, L=L, Tii=Tii, W=X[:, :, :D], U=X[:, :, D:],
                Qp=q_c * torch.exp(gam), Kb=k_c * torch.exp(G[:, None, :] - gam),
                eG=torch.exp(G), Kt=R[:, :, :D])


def forward(q, k, v, g, beta, s0, C=64):
    """Folded inputs (BH, L, D) / (BH, L); s0 (BH, D, D) reference orientation
    or None.  Returns (o, s_final, aux)."""
    BH, L, D = q.shape
    pad = (C - L % C) % C
    z = lambda t: torch.cat([t, torch.zeros((BH, pad) + t.shape[2:], dtype=t.dtype)], 1)
    if pad:
        q, k, v, g, beta = (z(t) for t in (q, k, v, g, beta))
    nc = q.shape[1] // C
    P = prep(*(t.reshape((BH * nc, C) + t.shape[2:]) for t in (q, k, v, g, beta)))
    rs = lambda t: t.reshape((BH, nc) + t.shape[1:])
    W, U, Qp, Kb, Aqk, eG = (rs(P[n]) for n in ("W", "U", "Qp", "Kb", "Aqk", "eG"))
    Sig = torch.zeros((BH, D, D), dtype=q.dtype) if s0 is None else s0.transpose(-1, -2).clone()
    outs, hs, vps = [], [], []
    for n in range(nc):
        hs.append(Sig)
        Vp = U[:, n] - W[:, n] @ Sig
        outs.append(Qp[:, n] @ Sig + Aqk[:, n] @ Vp)
        Sig = eG[:, n, :, None] * Sig + Kb[:, n].transpose(-1, -2) @ Vp
        vps.append(Vp)
    o = torch.cat(outs, 1)[:, :L]
    aux = dict(P=P, h=torch.stack(hs, 1), Vp=torch.stack(vps, 1), nc=nc, pad=pad,
               padded=(q, k, v, g, beta))
    return o, Sig.transpose(-1, -2), aux


def backward(q, k, v, g, beta, s0, do, dsf=None, C=64, return_aux=False):
    """Returns (dq, dk, dv, dg, dbeta, ds0) for folded inputs; with
    ``return_aux`` also a dict of the per-chunk intermediates (prep outputs,
    h, Vp, dh, dVp) in the kernels' chunk order."""
    BH, L, D = q.shape
    _, _, aux = forward(q, k, v, g, beta, s0, C)
    nc, pad = aux["nc"], aux["pad"]
    qp, kp, vp_, gp, bp = aux["padded"]
    if pad:
        do = torch.cat([do, torch.zeros((BH, pad, D), dtype=do.dtype)], 1)
    P = aux["P"]
    rs = lambda t: t.reshape((BH, nc) + t.shape[1:])
    W, Qp, Kb, Aqk, eG = (rs(P[n]) for n in ("W", "Qp", "Kb", "Aqk", "eG"))
    dO = do.reshape(BH, nc, C, D)
    dSig = torch.zeros((BH, D, D), dtype=q.dtype) if dsf is None else dsf.transpose(-1, -2).clone()
    dh, dvps = [None] * nc, [None] * nc
    for n in range(nc - 1, -1, -1):
        dh[n] = dSig
        dVp = Aqk[:, n].transpose(-1, -2) @ dO[:, n] + Kb[:, n] @ dSig
        dSig = eG[:, n, :, None] * dSig + Qp[:, n].transpose(-1, -2) @ dO[:, n] \
            - W[:, n].transpose(-1, -2) @ dVp
        dvps[n] = dVp
    ds0 = dSig.transpose(-1, -2)
    f = lambda t: t.reshape((BH * nc,) + t.shape[2:])
    grads = local_backward(
        q_c=f(qp.reshape(BH, nc, C, D)), k_c=f(kp.reshape(BH, nc, C, D)),
        v_c=f(vp_.reshape(BH, nc, C, D)), g_c=f(gp.reshape(BH, nc, C, D)),
        beta_c=f(bp.reshape(BH, nc, C)), dO=f(dO), h=f(aux["h"]), dh=f(torch.stack(dh, 1)),
        Vp=f(aux["Vp"]), dVp=f(torch.stack(dvps, 1)))
    out = []
    for gname in ("dq", "dk", "dv", "dg"):
        out.append(grads[gname].reshape(BH, nc * C, D)[:, :L])
    out.append(grads["dbeta"].reshape(BH, nc * C)[:, :L])
    out.append(ds0)
    if return_aux:
        aux2 = dict(P=P, h=f(aux["h"]), Vp=f(aux["Vp"]), dh=f(torch.stack(dh, 1)),
                    dVp=f(torch.stack(dvps, 1)), local=grads)
        return tuple(out), aux2
    return tuple(out)


def local_backward(q_c, k_c, v_c, g_c, beta_c, dO, h, dh, Vp, dVp):
    """Chunk-parallel adjoints.  h = Sig at chunk start, dh = dL/dSig at chunk
    end, Vp / dVp the chunk's V' and its adjoint.  All (N, C, D) / (N, D, D)."""
    N, C, D = k_c.shape
    P = prep(q_c, k_c, v_c, g_c, beta_c)
    gam, G, L, Tii, W, U = P["gam"], P["G"], P["L"], P["Tii"], P["W"], P["U"]
    eg = torch.exp(gam)
    ebk = torch.exp(G[:, None, :] - gam)
    # products with K = dv
    dQp = dO @ h.transpose(-1, -2)                        # (C, D)
    dKb = Vp @ dh.transpose(-1, -2)
    dW = -dVp @ h.transpose(-1, -2)
    dAqk = torch.tril(dO @ Vp.transpose(-1, -2), 0)
    dG = torch.exp(G) * torch.sum(dh * h, dim=-1)         # state decay term
    # solve adjoint: dR = (I + L)^-T [dW | dU] by block back substitution
    dX = torch.cat([dW, dVp], -1)
    nb = C // BS
    dR = [None] * nb
    for i in range(nb - 1, -1, -1):
        Y = dX[:, BS * i:BS * i + BS].clone()
        for j in range(i + 1, nb):
            Y = Y - L[:, BS * j:BS * j + BS, BS * i:BS * i + BS].transpose(-1, -2) @ dR[j]
        dR[i] = Tii[i].transpose(-1, -2) @ Y
    dR = torch.cat(dR, 1)
    X = torch.cat([W, U], -1)
    dL = -torch.tril(dR @ X.transpose(-1, -2), -1)
    dKt, dVt = dR[:, :, :D], dR[:, :, D:]
    # R = [beta e^gam K | beta V]
    dv = beta_c[:, :, None] * dVt
    dbeta = torch.sum(dVt * v_c, -1) + torch.sum(dKt * eg * k_c, -1)
    dk = beta_c[:, :, None] * eg * dKt
    dgam = dKt * (beta_c[:, :, None] * eg * k_c)
    # L = diag(beta) Akk
    Akk = P["Akk"]
    dbeta = dbeta + torch.sum(dL * Akk, -1)
    dP = beta_c[:, :, None] * dL
    # anchored products: P = Kl Kr^T, Aqk = Ql Kr^T per block row i
    dq = dQp * eg
    dgam = dgam + dQp * (q_c * eg)
    dk = dk + dKb * ebk
    dgam = dgam - dKb * (k_c * ebk)
    dG = dG + torch.sum(dKb * k_c * ebk, dim=1)
    for i in range(nb):
        r = BS * i
        t = slice(r, r + BS)
        el = torch.exp(gam[:, t] - gam[:, r:r + 1])
        er = torch.exp(gam[:, r:r + 1] - gam[:, :r + BS])
        Kl, Ql, Kr = k_c[:, t] * el, q_c[:, t] * el, k_c[:, :r + BS] * er
        dPi, dAi = dP[:, t, :r + BS], dAqk[:, t, :r + BS]
        dKl = dPi @ Kr
        dQl = dAi @ Kr
        dKr = dPi.transpose(-1, -2) @ Kl + dAi.transpose(-1, -2) @ Ql
        dk[:, t] += dKl * el
        dq[:, t] += dQl * el
        dgam[:, t] += dKl * Kl + dQl * Ql
        dk[:, :r + BS] += dKr * er
        dgam[:, :r + BS] -= dKr * Kr
    dgam[:, -1, :] += dG
    dg = torch.flip(torch.cumsum(torch.flip(dgam, [1]), 1), [1])
    return dict(dq=dq, dk=dk, dv=dv, dg=dg, dbeta=dbeta, dQp=dQp, dKb=dKb, dW=dW, dAqk=dAqk,
                dR=dR, dL=dL)
