"""CPU checks of the GatedDeltaLayer restatement (oracle/layer_reference.py) and
of the layer's host-side validation.  The restatement is pinned against library
routines (F.conv1d, F.rms_norm, F.softplus) and closed forms, so a transposed
tap order, a per-head instead of per-row norm or a dropped scale fails here."""
import pytest
import torch
import torch.nn.functional as F

from oracle import kda_reference as R
from oracle import layer_reference as LR

D64 = torch.float64


def _gen(seed=0):
    return torch.Generator().manual_seed(seed)


def test_short_conv_matches_conv1d():
    g = _gen(1)
    B, L, C, K = 2, 13, 6, 4
    x = torch.randn(B, L, C, generator=g, dtype=D64)
    w = torch.randn(C, K, 1, generator=g, dtype=D64)
    b = torch.randn(C, generator=g, dtype=D64)
    ref = F.conv1d(x.transpose(1, 2), w.reshape(C, 1, K), b, padding=K - 1, groups=C)[..., :L].transpose(1, 2)
    torch.testing.assert_close(LR.short_causal_conv1d(x, w, b), ref, rtol=1e-12, atol=1e-12)


def test_short_conv_identity_and_shift_taps():
    g = _gen(2)
    x = torch.randn(1, 9, 4, generator=g, dtype=D64)
    w = torch.zeros(4, 4, 1, dtype=D64)
    w[:, 3] = 1.0   # the last tap multiplies the current token
    torch.testing.assert_close(LR.short_causal_conv1d(x, w, None), x)
    w.zero_()
    w[:, 0] = 1.0   # the first tap reads three tokens back, zeros before the start
    out = LR.short_causal_conv1d(x, w, None)
    torch.testing.assert_close(out[:, 3:], x[:, :-3])
    assert torch.all(out[:, :3] == 0)


def test_gated_rms_norm_matches_library():
    g = _gen(3)
    x = torch.randn(2, 5, 3, 16, generator=g, dtype=D64)
    z = torch.randn(2, 5, 3, 16, generator=g, dtype=D64)
    w = torch.randn(16, generator=g, dtype=D64)
    ref = F.rms_norm(x, (16,), w, 1e-5) * torch.sigmoid(z)
    torch.testing.assert_close(LR.gated_rms_norm(x, w, z, 1e-5), ref, rtol=1e-12, atol=1e-12)


def test_softplus_matches_library():
    # F.softplus switches to the identity above its threshold (20), where the
    # exact value differs by log1p(e^-x) < 2.1e-9
    x = torch.linspace(-40, 20, 601, dtype=D64)
    torch.testing.assert_close(R.softplus(x), F.softplus(x), rtol=1e-12, atol=1e-12)
    x = torch.linspace(20, 60, 41, dtype=D64)
    torch.testing.assert_close(R.softplus(x), x + torch.log1p(torch.exp(-x)), rtol=1e-14, atol=0)


def _proj_inputs(B, L, H, D, seed=0, bias=True):
    g = _gen(seed)
    HD = H * D
    r = lambda *s: torch.randn(*s, generator=g, dtype=D64)  # noqa: E731
    return dict(xq=r(B, L, HD), xk=r(B, L, HD), xv=r(B, L, HD), xf=r(B, L, HD), xb=r(B, L, H),
                conv_w=torch.rand(3, HD, 4, generator=g, dtype=D64) - 0.5,
                conv_b=0.1 * r(3, HD) if bias else None, dt_bias=0.1 * r(HD),
                A_log=torch.log(1 + 15 * torch.rand(H, generator=g, dtype=D64)))


def test_producer_closed_forms():
    B, L, H, D = 2, 11, 3, 8
    x = _proj_inputs(B, L, H, D)
    q, k, v, g, beta = LR.producer_from_projections(**x, H=H, D=D, beta_mult=2.0)
    # the L2 norm spans the whole H*D row, after SiLU; q carries D^-1/2
    torch.testing.assert_close(q.reshape(B, L, -1).norm(dim=-1), torch.full((B, L), D ** -0.5, dtype=D64))
    torch.testing.assert_close(k.reshape(B, L, -1).norm(dim=-1), torch.ones(B, L, dtype=D64))
    assert not torch.allclose(k.norm(dim=-1), torch.ones(B, L, H, dtype=D64))
    # v is SiLU of the conv output: with the identity tap and no bias, silu(xv)
    xi = dict(x, conv_w=torch.zeros(3, H * D, 4, dtype=D64), conv_b=None)
    xi["conv_w"][:, :, 3] = 1.0
    _, _, v1, _, _ = LR.producer_from_projections(**xi, H=H, D=D)
    torch.testing.assert_close(v1.reshape(B, L, -1), x["xv"] * torch.sigmoid(x["xv"]))
    # g = -exp(A_log) softplus(xf + dt_bias) <= 0 per head; beta in (0, 2)
    A = torch.exp(x["A_log"])
    gref = -A.reshape(1, 1, H, 1) * F.softplus(x["xf"].reshape(B, L, H, D) + x["dt_bias"].reshape(H, D))
    torch.testing.assert_close(g, gref)
    assert torch.all(g <= 0)
    torch.testing.assert_close(beta, 2 * torch.sigmoid(x["xb"]))


def test_layer_forward_t1_closed_form():
    """One token, zero state: the recurrence gives o = beta (k . q) v, so the
    layer output is fixed by the producer and the epilogue alone."""
    torch.manual_seed(0)
    H, D, hidden = 2, 4, 8
    g = _gen(5)
    p = {n: torch.randn(*s, generator=g, dtype=D64) * 0.3 for n, s in {
        "q_proj.weight": (H * D, hidden), "k_proj.weight": (H * D, hidden), "v_proj.weight": (H * D, hidden),
        "f_proj_1.weight": (D, hidden), "f_proj_2.weight": (H * D, D), "b_proj.weight": (H, hidden),
        "q_conv1d.weight": (H * D, 4, 1), "k_conv1d.weight": (H * D, 4, 1), "v_conv1d.weight": (H * D, 4, 1),
        "q_conv1d.bias": (H * D,), "k_conv1d.bias": (H * D,), "v_conv1d.bias": (H * D,),
        "g_proj_1.weight": (D, hidden), "g_proj_2.weight": (H * D, D), "g_proj_2.bias": (H * D,),
        "o_norm.weight": (D,), "o_proj.weight": (hidden, H * D), "dt_bias": (H * D,), "A_log": (H,)}.items()}
    x = torch.randn(1, 1, hidden, generator=g, dtype=D64)
    out, state = LR.layer_forward(p, x, H, D)
    q, k, v, _, beta = LR.producer(p, x, H, D)
    o = beta[..., None] * (k * q).sum(-1, keepdim=True) * v
    gate = ((x @ p["g_proj_1.weight"].T) @ p["g_proj_2.weight"].T + p["g_proj_2.bias"]).reshape(1, 1, H, D)
    y = F.rms_norm(o, (D,), p["o_norm.weight"], 1e-5) * torch.sigmoid(gate)
    torch.testing.assert_close(out, y.reshape(1, 1, H * D) @ p["o_proj.weight"].T)
    # S_1 = beta v k^T (reference [v, k] orientation)
    torch.testing.assert_close(state[0], beta[0, 0, :, None, None] * v[0, 0, :, :, None] * k[0, 0, :, None, :])


def test_layer_construction_validation():
    from mlx_vit_amd.layer import GatedDeltaLayer
    with pytest.raises(ValueError, match="channel-wise"):
        GatedDeltaLayer(64, 2, 32, channel_wise_decay=False, compute_path="hip_chunkwise_kda")
    scalar = GatedDeltaLayer(64, 2, 32, channel_wise_decay=False)
    names = dict(scalar.named_parameters())
    assert names["a_proj.weight"].shape == (2, 64) and "A_log" not in names and "f_proj_1.weight" not in names
    assert scalar.recurrence.compute_path == "hip_chunkwise_gdn"
    with pytest.raises(ValueError, match="head_dim"):
        GatedDeltaLayer(64, 2, 48)
    with pytest.raises(ValueError, match="chunk_size"):
        GatedDeltaLayer(64, 2, 32, chunk_size=48)
    assert GatedDeltaLayer(64, 2, 32, chunk_size=32).chunk_size == 32
    with pytest.raises(ValueError, match="Unknown compute_path"):
        GatedDeltaLayer(64, 2, 32, compute_path="metal")
    with pytest.raises(ValueError, match="2048"):
        GatedDeltaLayer(64, 32, 128)
    layer = GatedDeltaLayer(96, 3, 32, allow_neg_eigval=True)
    names = dict(layer.named_parameters())
    # the reference's parameter names and shapes (nope_gdn_mlx.py:736-772)
    assert names["q_conv1d.weight"].shape == (96, 4, 1)
    assert names["A_log"].shape == (3,) and names["dt_bias"].shape == (96,)
    assert names["o_norm.weight"].shape == (32,) and names["g_proj_2.bias"].shape == (96,)
    assert torch.all(names["A_log"] >= 0) and torch.all(names["A_log"] <= torch.log(torch.tensor(16.0)))
    with pytest.raises(ValueError, match="x must be"):
        layer(torch.zeros(1, 4, 95))


def test_producer_host_checks():
    from mlx_vit_amd.layer import producer_forward
    qkv = torch.zeros(1, 4, 3 * 64)
    with pytest.raises(ValueError, match="columns"):
        producer_forward(qkv, torch.zeros(1, 4, 64), torch.zeros(1, 4, 2), torch.zeros(3, 64, 4), None,
                         torch.zeros(64), torch.zeros(2), 2, 16, 0.25)
    with pytest.raises(ValueError, match="do not match"):
        producer_forward(torch.zeros(1, 4, 96), torch.zeros(1, 5, 32), torch.zeros(1, 4, 2),
                         torch.zeros(3, 32, 4), None, torch.zeros(32), torch.zeros(2), 2, 16, 0.25)


def test_gdn_step_is_kda_step_with_broadcast_log_alpha():
    """The scalar-alpha step (nope_gdn_mlx.py:641-650) is the KDA step
    (nope_gdn_mlx.py:616-638) with every channel's decay e^g = alpha; also
    pinned by the closed form of one step from a zero state."""
    g = _gen(7)
    B, H, D = 2, 3, 5
    S = torch.randn(B, H, D, D, generator=g, dtype=D64)
    q, k, v = (torch.randn(B, H, D, generator=g, dtype=D64) for _ in range(3))
    alpha = torch.rand(B, H, generator=g, dtype=D64) * 0.9 + 0.05
    beta = torch.rand(B, H, generator=g, dtype=D64)
    I = torch.eye(D, dtype=D64)
    s1, o1 = R.gdn_step(S, q, k, v, alpha, beta, I)
    s2, o2 = R.kda_step(S, q, k, v, torch.log(alpha)[..., None].expand(B, H, D), beta, I)
    torch.testing.assert_close(s1, s2)
    torch.testing.assert_close(o1, o2)
    s0, o0 = R.gdn_step(torch.zeros_like(S), q, k, v, alpha, beta, I)
    torch.testing.assert_close(s0, beta[..., None, None] * v[..., :, None] * k[..., None, :])
    torch.testing.assert_close(o0, beta[..., None] * (k * q).sum(-1, keepdim=True) * v)
