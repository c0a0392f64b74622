"""Pins the CPU oracle (CPU only, float64).

Every check below is fixed by mathematics or by an equivalence the reference
itself states, and is chosen so that a plausible slip -- decaying rows instead
of columns, reading the state transposed, dropping the beta factor, an
off-by-one in the cumsum or the causal mask -- fails at least one of them.
"""
import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import cref
from oracle import kda_reference as R
from tests import kda_model as M

F64 = torch.float64


def _rand_case(B, T, H, D, seed, g_scale=0.3, state_std=0.3):
    x = R.make_inputs(B, T, H, D, dtype=F64, seed=seed, with_state=True, with_grad=True,
                      g_scale=g_scale, state_std=state_std)
    x["s0"] = x["s0"].to(F64)
    return x


# ---------------------------------------------------------------- forward invariants

def test_beta_zero_is_pure_column_decay():
    """beta = 0: S_t = S_0 diag(exp(sum_{tau<=t} g_tau)) -- columns (key channels)
    decay, and o_t = S_t q_t."""
    x = _rand_case(1, 9, 2, 5, seed=1)
    beta = torch.zeros_like(x["beta"])
    o, sf = R.loop_compiled_kda(x["q"], x["k"], x["v"], x["g"], beta, x["s0"], compute_dtype=F64)
    G = torch.cumsum(x["g"], 1)
    S = x["s0"][:, None] * torch.exp(G)[:, :, :, None, :]
    assert torch.allclose(sf, S[:, -1], rtol=1e-12, atol=1e-14)
    assert torch.allclose(o, torch.einsum("bthij,bthj->bthi", S, x["q"]), rtol=1e-12, atol=1e-14)
    # a row decay would differ for a non-symmetric S0
    S_row = x["s0"][:, None] * torch.exp(G)[:, :, :, :, None]
    assert not torch.allclose(sf, S_row[:, -1], rtol=1e-3)


def test_single_token_zero_state_closed_form():
    """T = 1, S_0 = 0: S_1 = beta v k^T, o = beta (k . q) v (output reads the
    post-update state; the state is [v, k])."""
    x = _rand_case(2, 1, 3, 6, seed=2)
    o, sf = R.loop_compiled_kda(x["q"], x["k"], x["v"], x["g"], x["beta"], None, compute_dtype=F64)
    b = x["beta"][:, 0, :, None]
    kq = torch.sum(x["k"][:, 0] * x["q"][:, 0], -1, keepdim=True)
    assert torch.allclose(o[:, 0], b * kq * x["v"][:, 0], rtol=1e-12, atol=1e-15)
    S1 = b[..., None] * x["v"][:, 0, :, :, None] * x["k"][:, 0, :, None, :]
    assert torch.allclose(sf, S1, rtol=1e-12, atol=1e-15)


def test_orthonormal_keys_overwrite_exactly():
    """g = 0, beta = 1, orthonormal keys: each step writes its value exactly, so
    S_T k_t = v_t for every t (delta rule = exact associative overwrite)."""
    D, T = 8, 6
    gen = torch.Generator().manual_seed(3)
    Qm, _ = torch.linalg.qr(torch.randn(D, D, generator=gen, dtype=F64))
    k = Qm[:T].reshape(1, T, 1, D)
    v = torch.randn(1, T, 1, D, generator=gen, dtype=F64)
    q = torch.randn(1, T, 1, D, generator=gen, dtype=F64)
    g = torch.zeros_like(k)
    beta = torch.ones(1, T, 1, dtype=F64)
    _, sf = R.loop_compiled_kda(q, k, v, g, beta, None, compute_dtype=F64)
    recalled = torch.einsum("ij,tj->ti", sf[0, 0], k[0, :, 0])
    assert torch.allclose(recalled, v[0, :, 0], atol=1e-12)


def test_transition_matrix_closed_form():
    """Unrolled recurrence with A_t = diag(e^{g_t}) (I - beta_t k_t k_t^T):
    S_T = S_0 A_1 ... A_T + sum_t beta_t v_t k_t^T A_{t+1} ... A_T (numpy)."""
    x = _rand_case(1, 7, 1, 5, seed=4)
    q, k, v, g, beta, s0 = (x[n][0, :, 0].numpy() if x[n].dim() == 4 else x[n] for n in
                            ("q", "k", "v", "g", "beta", "s0"))
    beta = x["beta"][0, :, 0].numpy()
    S0 = x["s0"][0, 0].numpy()
    T, D = k.shape
    A = [np.diag(np.exp(g[t])) @ (np.eye(D) - beta[t] * np.outer(k[t], k[t])) for t in range(T)]
    S = S0.copy()
    for t in range(T):
        S = S @ A[t]
    for t in range(T):
        P = np.eye(D)
        for tau in range(t + 1, T):
            P = P @ A[tau]
        S = S + beta[t] * np.outer(v[t], k[t]) @ P
    _, sf = R.loop_compiled_kda(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], compute_dtype=F64)
    assert np.allclose(sf[0, 0].numpy(), S, rtol=1e-11, atol=1e-13)


def test_linear_in_state_and_values():
    """For fixed q, k, g, beta the map (S_0, v) -> (o, S_T) is linear."""
    x = _rand_case(1, 12, 2, 6, seed=5)
    y = _rand_case(1, 12, 2, 6, seed=6)
    a, b = 0.7, -1.3
    f = lambda s0, v: R.loop_compiled_kda(x["q"], x["k"], v, x["g"], x["beta"], s0, compute_dtype=F64)
    o1, s1 = f(x["s0"], x["v"])
    o2, s2 = f(y["s0"], y["v"])
    o3, s3 = f(a * x["s0"] + b * y["s0"], a * x["v"] + b * y["v"])
    assert torch.allclose(o3, a * o1 + b * o2, atol=1e-12)
    assert torch.allclose(s3, a * s1 + b * s2, atol=1e-12)


def test_matrix_step_equals_rank1_step():
    """nope_gdn_mlx.py:3724-3735: S (I - b k k^T) + b v k^T == S + b (v - S k) k^T."""
    x = _rand_case(2, 15, 2, 7, seed=7)
    o, sf = R.loop_compiled_kda(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], compute_dtype=F64)
    f = R.fold_heads
    o1, s1, _ = R.step_forward_rank1(f(x["q"]), f(x["k"]), f(x["v"]), f(x["g"]), f(x["beta"]),
                                     x["s0"].reshape(4, 7, 7))
    assert R.rel_l2(R.unfold_heads(o1, 2, 2), o) < 1e-13
    assert R.rel_l2(s1.reshape(2, 2, 7, 7), sf) < 1e-13


def test_c_oracle_forward_matches_torch():
    x = _rand_case(2, 77, 3, 16, seed=8)
    o, sf = R.loop_compiled_kda(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], compute_dtype=F64)
    c = cref.forward(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"])
    assert R.rel_l2(c["o"], o) < 1e-13 and R.rel_l2(c["s_final"], sf) < 1e-13


# ---------------------------------------------------------------- gradients

def test_gradcheck_step_oracle():
    """Finite differences pin the autograd gradient of the step form."""
    x = _rand_case(1, 5, 1, 3, seed=9)
    leaves = [x[n].clone().requires_grad_(True) for n in ("q", "k", "v", "g", "beta", "s0")]
    w = torch.randn(1, 5, 1, 3, dtype=F64, generator=torch.Generator().manual_seed(1))
    ws = torch.randn(1, 1, 3, 3, dtype=F64, generator=torch.Generator().manual_seed(2))

    def fn(q, k, v, g, beta, s0):
        o, sf = R.loop_compiled_kda(q, k, v, g, beta, s0, compute_dtype=F64)
        return (o * w).sum() + (sf * ws).sum()
    assert torch.autograd.gradcheck(fn, leaves, eps=1e-6, atol=1e-7, rtol=1e-5)


@pytest.mark.parametrize("B,T,H,D", [(1, 37, 2, 8), (2, 70, 1, 16), (1, 1, 1, 4)])
def test_c_oracle_backward_matches_autograd(B, T, H, D):
    x = _rand_case(B, T, H, D, seed=10)
    dsf = torch.randn(B, H, D, D, dtype=F64, generator=torch.Generator().manual_seed(3))
    ref = R.autograd_reference(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], x["do"], dsf)
    c = cref.backward(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], x["do"], dsf)
    for n in ("dq", "dk", "dv", "dg", "dbeta", "ds0"):
        assert R.rel_l2(c[n], ref[n]) < 1e-12, n


def test_python_backward_full_matches_autograd():
    """Restated nope_gdn_mlx.py:3185-3295 equals autograd of the step form."""
    B, T, H, D = 1, 30, 2, 6
    x = _rand_case(B, T, H, D, seed=11)
    dsf = torch.randn(B, H, D, D, dtype=F64, generator=torch.Generator().manual_seed(4))
    ref = R.autograd_reference(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], x["do"], dsf)
    f = R.fold_heads
    _, _, u = R.step_forward_rank1(f(x["q"]), f(x["k"]), f(x["v"]), f(x["g"]), f(x["beta"]),
                                   x["s0"].reshape(B * H, D, D))
    out = R.python_backward_full(f(x["q"]), f(x["k"]), f(x["v"]), f(x["g"]), f(x["beta"]), u,
                                 x["s0"].reshape(B * H, D, D), f(x["do"]), dsf.reshape(B * H, D, D))
    for i, n in enumerate(("dq", "dk", "dv", "dg", "dbeta")):
        assert R.rel_l2(R.unfold_heads(out[i], B, H), ref[n]) < 1e-12, n
    assert R.rel_l2(out[5].reshape(B, H, D, D), ref["ds0"]) < 1e-12


# ---------------------------------------------------------------- chunkwise algebra

@pytest.mark.parametrize("C", [4, 8, 16, 64])
def test_chunkwise_equals_step(C):
    """The reference's own equivalence criterion (nope_gdn_mlx.py:4905-4914) for
    chunk sizes that do and do not divide T."""
    B, T, H, D = 1, 50, 2, 8
    x = _rand_case(B, T, H, D, seed=12)
    o, sf = R.loop_compiled_kda(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], compute_dtype=F64)
    f = R.fold_heads
    oc, sc = R.chunkwise_forward(f(x["q"]), f(x["k"]), f(x["v"]), f(x["g"]), f(x["beta"]),
                                 x["s0"].reshape(B * H, D, D), C)
    assert R.rel_l2(R.unfold_heads(oc, B, H), o) < 1e-12
    assert R.rel_l2(sc.reshape(B, H, D, D), sf) < 1e-12


def test_padding_is_invisible():
    """Appending tokens with g = 0 and beta = 0 leaves o[:T] and S_T unchanged
    (the padding rule of nope_gdn_mlx.py:2354-2361)."""
    x = _rand_case(1, 20, 1, 6, seed=13)
    o, sf = R.loop_compiled_kda(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], compute_dtype=F64)
    pad = lambda t, val=0.0: torch.cat([t, torch.full((1, 9) + t.shape[2:], val, dtype=t.dtype)], 1)
    gen = torch.Generator().manual_seed(5)
    qp = torch.cat([x["q"], torch.randn(1, 9, 1, 6, generator=gen, dtype=F64)], 1)
    kp = torch.cat([x["k"], torch.randn(1, 9, 1, 6, generator=gen, dtype=F64)], 1)
    vp = torch.cat([x["v"], torch.randn(1, 9, 1, 6, generator=gen, dtype=F64)], 1)
    o2, sf2 = R.loop_compiled_kda(qp, kp, vp, pad(x["g"]), pad(x["beta"]), x["s0"], compute_dtype=F64)
    assert torch.allclose(o2[:, :20], o, atol=1e-14) and torch.allclose(sf2, sf, atol=1e-14)


@pytest.mark.parametrize("C", [4, 16])
def test_chunkwise_backward_matches_autograd(C):
    """The restated hand-derived adjoints (nope_gdn_mlx.py:2579-2720)."""
    B, T, H, D = 1, 37, 2, 6
    x = _rand_case(B, T, H, D, seed=14)
    dsf = torch.randn(B, H, D, D, dtype=F64, generator=torch.Generator().manual_seed(6))
    ref = R.autograd_reference(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], x["do"], dsf)
    f = R.fold_heads
    out = R.chunkwise_backward(f(x["q"]), f(x["k"]), f(x["v"]), f(x["g"]), f(x["beta"]),
                               x["s0"].reshape(B * H, D, D), f(x["do"]), dsf.reshape(B * H, D, D), C)
    for i, n in enumerate(("dq", "dk", "dv", "dg", "dbeta")):
        assert R.rel_l2(R.unfold_heads(out[i], B, H), ref[n]) < 1e-12, n
    assert R.rel_l2(out[5].reshape(B, H, D, D), ref["ds0"]) < 1e-12


# ---------------------------------------------------------------- triangular solves

def test_solve_kat_matches_numpy():
    """The reference's KAT (nope_gdn_mlx.py:4793-4835): numpy seed 0 per C,
    L = tril(randn*0.1, -1) + I, b = randn(BH, C, C), rel-max < 1e-4."""
    BH = 4
    for C in [4, 8, 16, 32, 40, 48, 56, 64]:
        np.random.seed(0)
        L = np.tril(np.random.randn(BH, C, C).astype(np.float32) * 0.1, k=-1) + np.eye(C, dtype=np.float32)
        b = np.random.randn(BH, C, C).astype(np.float32)
        y_np = np.stack([np.linalg.solve(L[i], b[i]) for i in range(BH)])
        y = R.solve_unit_lower(torch.from_numpy(L).double(), torch.from_numpy(b).double()).numpy()
        rel = np.max(np.abs(y - y_np)) / (np.max(np.abs(y_np)) + 1e-9)
        assert rel < 1e-4, (C, rel)
        U = np.ascontiguousarray(np.transpose(L, (0, 2, 1)))
        yu = R.solve_unit_upper(torch.from_numpy(U).double(), torch.from_numpy(b).double()).numpy()
        yu_ref = np.stack([scipy.linalg.solve_triangular(U[i].astype(np.float64), b[i], lower=False,
                                                         unit_diagonal=True) for i in range(BH)])
        assert np.max(np.abs(yu - yu_ref)) / np.max(np.abs(yu_ref)) < 1e-12


def test_solve_reads_only_the_strict_triangle():
    gen = torch.Generator().manual_seed(7)
    L = torch.randn(2, 10, 10, generator=gen, dtype=F64)
    b = torch.randn(2, 10, 3, generator=gen, dtype=F64)
    y = R.solve_unit_lower(L, b)
    Lu = torch.tril(L, -1) + torch.eye(10, dtype=F64)
    assert torch.allclose(Lu @ y, b, atol=1e-10)


# ---------------------------------------------------------------- the kernel decomposition model

@pytest.mark.parametrize("T,D,g_scale", [(37, 16, 0.5), (130, 32, 0.3), (64, 64, 1.0)])
def test_decomposition_model_matches_oracle(T, D, g_scale):
    """The float64 model of the HIP staging (anchored sub-blocks, block
    substitution, W/U form, reverse state recurrence, local adjoints)."""
    B, H = 1, 2
    x = _rand_case(B, T, H, D, seed=15, g_scale=g_scale)
    dsf = torch.randn(B, H, D, D, dtype=F64, generator=torch.Generator().manual_seed(8))
    ref = R.autograd_reference(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], x["do"], dsf)
    f = R.fold_heads
    o, sf, _ = M.forward(f(x["q"]), f(x["k"]), f(x["v"]), f(x["g"]), f(x["beta"]), x["s0"].reshape(B * H, D, D))
    assert R.rel_l2(R.unfold_heads(o, B, H), ref["o"]) < 1e-12
    assert R.rel_l2(sf.reshape(B, H, D, D), ref["s_final"]) < 1e-12
    gr = M.backward(f(x["q"]), f(x["k"]), f(x["v"]), f(x["g"]), f(x["beta"]), x["s0"].reshape(B * H, D, D),
                    f(x["do"]), dsf.reshape(B * H, D, D))
    for i, n in enumerate(("dq", "dk", "dv", "dg", "dbeta")):
        assert R.rel_l2(R.unfold_heads(gr[i], B, H), ref[n]) < 1e-11, n
    assert R.rel_l2(gr[5].reshape(B, H, D, D), ref["ds0"]) < 1e-11


# ---------------------------------------------------------------- inputs

def test_input_distributions():
    x = R.make_inputs(2, 300, 3, 64, dtype=torch.float32, seed=0, with_state=True)
    assert torch.allclose(torch.linalg.vector_norm(x["q"], dim=-1), torch.ones(2, 300, 3), atol=1e-5)
    assert torch.allclose(torch.linalg.vector_norm(x["k"], dim=-1), torch.ones(2, 300, 3), atol=1e-5)
    assert bool((x["beta"] > 0).all() and (x["beta"] < 1).all())
    assert bool((x["g"] <= 0).all())
    # E[softplus(N(0,1))] = 0.806...; g = -0.1 softplus
    assert abs(float(x["g"].mean()) + 0.0806) < 0.003
    assert abs(float(x["s0"].std()) - 0.02) < 0.001
