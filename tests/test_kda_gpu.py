"""GPU parity tests: the HIP path through the C ABI against the CPU oracle.

Bars: rel-L2 <= 1e-4 with fp32 inputs, <= 1e-2 with bf16 inputs (the oracle
runs in fp64 on the same bf16-rounded values).  Outputs o, final state and the
gradients dq, dk, dv, dg, dbeta, dS0 are all checked.
"""
import numpy as np
import pytest
import torch

from oracle import cref
from oracle import kda_reference as R
from tests import kda_model as M

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.bfloat16: 1e-2}
DEV = "cuda"


def _kda():
    import mlx_vit_amd
    return mlx_vit_amd


def _inputs(B, T, H, D, dtype, seed=0, with_state=False, g_scale=0.1, grad=False):
    x = R.make_inputs(B, T, H, D, dtype=dtype, seed=seed, with_state=with_state,
                      with_grad=grad, g_scale=g_scale)
    return x


def _dev(x, names=("q", "k", "v", "g", "beta")):
    return [x[n].to(DEV) for n in names]


def _fwd_errors(x, dtype):
    kda = _kda()
    q, k, v, g, beta = _dev(x)
    s0 = x["s0"].to(DEV) if x["s0"] is not None else None
    o, sf = kda.kda_forward(q, k, v, g, beta, s0)
    torch.cuda.synchronize()
    ref = cref.forward(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"])
    return {"o": R.rel_l2(o.cpu(), ref["o"]), "s_final": R.rel_l2(sf.cpu(), ref["s_final"])}


def _bwd_errors(x, dtype, dsf=None):
    kda = _kda()
    q, k, v, g, beta = _dev(x)
    s0 = x["s0"].to(DEV) if x["s0"] is not None else None
    do = x["do"].to(DEV)
    grads = kda.kda_backward(q, k, v, g, beta, s0, do, None if dsf is None else dsf.to(DEV))
    torch.cuda.synchronize()
    ref = cref.backward(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], x["do"], dsf)
    names = ("dq", "dk", "dv", "dg", "dbeta", "ds0")
    return {n: R.rel_l2(gr.cpu(), ref[n]) for n, gr in zip(names, grads)}


def _assert_all(errs, tol, case):
    print(case, {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    bad = {k: v for k, v in errs.items() if not (v <= tol)}
    assert not bad, f"{case}: rel-L2 above {tol}: {bad}"


# ---------------------------------------------------------------- stage checks

def _ws_view(ws, off, shape):
    n = int(np.prod(shape))
    return ws[off:off + 4 * n].view(torch.float32).reshape(shape)


def test_prep_workspace_matches_model():
    """The forward prep kernel's workspace equals the float64 decomposition model."""
    kda = _kda()
    B, T, H, D = 1, 100, 2, 64
    x = _inputs(B, T, H, D, torch.float32, seed=5, g_scale=0.5)
    q, k, v, g, beta = _dev(x)
    ws = torch.zeros(kda.workspace_bytes(0, B, T, H, D, torch.float32), dtype=torch.uint8, device=DEV)
    kda.kda_forward(q, k, v, g, beta, None, workspace=ws)
    torch.cuda.synchronize()
    off = kda.workspace_offsets(0, B, T, H, D)
    nc = (T + 63) // 64
    N = B * H * nc
    f = lambda t: R.fold_heads(t.double())
    pad = nc * 64 - T
    z = lambda t: torch.cat([t, torch.zeros((t.shape[0], pad) + t.shape[2:], dtype=t.dtype)], 1)
    qf, kf, vf, gf, bf = (z(f(x[n])) for n in ("q", "k", "v", "g", "beta"))
    P = M.prep(qf.reshape(N, 64, D), kf.reshape(N, 64, D), vf.reshape(N, 64, D), gf.reshape(N, 64, D),
               bf.reshape(N, 64))
    wsc = ws.cpu()
    errs = {
        "W": R.rel_l2(_ws_view(wsc, off["W"], (N, 64, D)), P["W"]),
        "U": R.rel_l2(_ws_view(wsc, off["U"], (N, 64, D)), P["U"]),
        "Qp": R.rel_l2(_ws_view(wsc, off["Qp"], (N, 64, D)), P["Qp"]),
        "KbT": R.rel_l2(_ws_view(wsc, off["KbT"], (N, D, 64)), P["Kb"].transpose(-1, -2)),
        "Aqk": R.rel_l2(_ws_view(wsc, off["Aqk"], (N, 64, 64)), P["Aqk"]),
        "eG": R.rel_l2(_ws_view(wsc, off["eG"], (N, D)), P["eG"]),
    }
    _assert_all(errs, 1e-4, "prep fp32")


def test_bwd_workspace_matches_model():
    """Backward intermediates (recomputed states, dh, V', dV') equal the model."""
    kda = _kda()
    B, T, H, D = 1, 130, 2, 64
    x = _inputs(B, T, H, D, torch.float32, seed=6, with_state=True, grad=True, g_scale=0.3)
    q, k, v, g, beta = _dev(x)
    s0, do = x["s0"].to(DEV), x["do"].to(DEV)
    ws = torch.zeros(kda.workspace_bytes(1, B, T, H, D, torch.float32), dtype=torch.uint8, device=DEV)
    kda.kda_backward(q, k, v, g, beta, s0, do, None, workspace=ws)
    torch.cuda.synchronize()
    off = kda.workspace_offsets(1, B, T, H, D)
    nc = (T + 63) // 64
    N = B * H * nc
    f = lambda t: R.fold_heads(t.double())
    _, aux = M.backward(f(x["q"]), f(x["k"]), f(x["v"]), f(x["g"]), f(x["beta"]),
                        x["s0"].double().reshape(B * H, D, D), f(x["do"]), None, return_aux=True)
    P = aux["P"]
    wsc = ws.cpu()
    errs = {
        "W": R.rel_l2(_ws_view(wsc, off["W"], (N, 64, D)), P["W"]),
        "WT": R.rel_l2(_ws_view(wsc, off["WT"], (N, D, 64)), P["W"].transpose(-1, -2)),
        "QpT": R.rel_l2(_ws_view(wsc, off["QpT"], (N, D, 64)), P["Qp"].transpose(-1, -2)),
        "Kb": R.rel_l2(_ws_view(wsc, off["Kb"], (N, 64, D)), P["Kb"]),
        "AqkT": R.rel_l2(_ws_view(wsc, off["AqkT"], (N, 64, 64)), P["Aqk"].transpose(-1, -2)),
        "Akk": R.rel_l2(_ws_view(wsc, off["Akk"], (N, 64, 64)), P["Akk"]),
        "h": R.rel_l2(_ws_view(wsc, off["h"], (N, D, D)), aux["h"]),
        "Vp": R.rel_l2(_ws_view(wsc, off["Vp"], (N, 64, D)), aux["Vp"]),
        "dh": R.rel_l2(_ws_view(wsc, off["dh"], (N, D, D)), aux["dh"]),
        "dVp": R.rel_l2(_ws_view(wsc, off["dVp"], (N, 64, D)), aux["dVp"]),
    }
    _assert_all(errs, 1e-4, "bwd workspace fp32")


# ---------------------------------------------------------------- forward parity

@pytest.mark.parametrize("B,T,H,D,with_state", [
    (1, 256, 2, 64, False),     # config 0
    (1, 256, 2, 64, True),
    (2, 100, 3, 64, True),      # ragged last chunk
    (1, 1, 1, 64, True),        # single token
    (1, 63, 2, 32, False),
    (1, 65, 2, 32, True),
    (1, 200, 2, 128, True),
])
def test_fwd_parity_fp32(B, T, H, D, with_state):
    x = _inputs(B, T, H, D, torch.float32, seed=1, with_state=with_state)
    _assert_all(_fwd_errors(x, torch.float32), TOL[torch.float32], f"fwd fp32 {B},{T},{H},{D},{with_state}")


@pytest.mark.parametrize("B,T,H,D,with_state", [
    (2, 300, 4, 64, True),
    (1, 129, 2, 128, False),
    (1, 64, 3, 32, True),
])
def test_fwd_parity_bf16(B, T, H, D, with_state):
    x = _inputs(B, T, H, D, torch.bfloat16, seed=2, with_state=with_state)
    _assert_all(_fwd_errors(x, torch.bfloat16), TOL[torch.bfloat16], f"fwd bf16 {B},{T},{H},{D},{with_state}")


@pytest.mark.parametrize("B,T,H,D,with_state", [
    (1, 2000, 2, 128, True),     # 8 segments of 4 chunks, ragged last chunk
    (1, 2340, 2, 128, False),    # 8 segments, the last of 2 chunks
    (2, 2500, 3, 128, True),     # 10 segments for each of six (b, h)
    (5, 12288, 8, 128, True),    # 40 (b, h): 6 segments of 32 chunks
])
def test_fwd_parity_bf16_segmented(B, T, H, D, with_state):
    """The bf16 forward at D = 128 split over segments of the sequence: segment
    maps (chain from zero / from the identity), the start-state scan, and the
    forward of every segment from its start state."""
    kda = _kda()
    assert kda.workspace_offsets(0, B, T, H, D, torch.bfloat16)["SegX"] >= 0, "segmented path not taken"
    x = _inputs(B, T, H, D, torch.bfloat16, seed=21, with_state=with_state)
    _assert_all(_fwd_errors(x, torch.bfloat16), TOL[torch.bfloat16], f"fwd bf16 segmented {B},{T},{H},{D},{with_state}")


def test_fwd_parity_config1_full():
    """Config 1: B=8, H=12, T=1568, D=64, bf16 -- full size against the fp64 oracle."""
    x = _inputs(8, 1568, 12, 64, torch.bfloat16, seed=0)
    _assert_all(_fwd_errors(x, torch.bfloat16), TOL[torch.bfloat16], "config1 fwd")


def test_fwd_parity_config3_long():
    """Config 3: B=1, H=16, T=32768, D=128, bf16, nonzero fp32 initial state."""
    x = _inputs(1, 32768, 16, 128, torch.bfloat16, seed=0, with_state=True)
    _assert_all(_fwd_errors(x, torch.bfloat16), TOL[torch.bfloat16], "config3 fwd")


def test_fwd_strong_decay_pairwise_path():
    """Decays beyond the anchored span guard take the pairwise path; still exact."""
    x = _inputs(1, 160, 2, 64, torch.float32, seed=3, with_state=True, g_scale=6.0)
    _assert_all(_fwd_errors(x, torch.float32), TOL[torch.float32], "fwd strong decay")


def test_fwd_moderate_decay_anchored_path():
    """Spans up to the guard stay on the anchored MFMA path."""
    x = _inputs(1, 160, 2, 64, torch.float32, seed=4, with_state=True, g_scale=2.0)
    _assert_all(_fwd_errors(x, torch.float32), TOL[torch.float32], "fwd moderate decay")


def test_fwd_beta_zero_is_pure_decay():
    """beta = 0: no writes, the state only decays and o_t = S_t q_t."""
    kda = _kda()
    x = _inputs(1, 70, 2, 64, torch.float32, seed=7, with_state=True)
    x["beta"] = torch.zeros_like(x["beta"])
    q, k, v, g, beta = _dev(x)
    o, sf = kda.kda_forward(q, k, v, g, beta, x["s0"].to(DEV))
    G = torch.cumsum(x["g"].double(), 1)                                  # (B, T, H, D)
    S = x["s0"].double()[:, None] * torch.exp(G)[:, :, :, None, :]      # (B, T, H, D, D)
    o_ref = torch.einsum("bthij,bthj->bthi", S, x["q"].double())
    assert R.rel_l2(o.cpu(), o_ref) <= 1e-5
    assert R.rel_l2(sf.cpu(), S[:, -1]) <= 1e-5


# ---------------------------------------------------------------- backward parity

@pytest.mark.parametrize("B,T,H,D,with_state,with_dsf", [
    (1, 256, 2, 64, False, False),
    (1, 256, 2, 64, True, True),
    (2, 100, 3, 64, True, True),
    (1, 1, 1, 64, True, True),
    (1, 65, 2, 32, True, False),
])
def test_bwd_parity_fp32(B, T, H, D, with_state, with_dsf):
    x = _inputs(B, T, H, D, torch.float32, seed=11, with_state=with_state, grad=True)
    dsf = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(9)) if with_dsf else None
    _assert_all(_bwd_errors(x, torch.float32, dsf), TOL[torch.float32],
                f"bwd fp32 {B},{T},{H},{D},{with_state},{with_dsf}")


def test_bwd_strong_decay_pairwise_path():
    x = _inputs(1, 130, 2, 64, torch.float32, seed=12, with_state=True, grad=True, g_scale=6.0)
    _assert_all(_bwd_errors(x, torch.float32), TOL[torch.float32], "bwd strong decay")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("g_scale", [0.5, 1.0, 2.0, 3.0])
def test_bwd_dg_independent_of_decay_span(dtype, g_scale):
    """Strong decays that still take the anchored path (16-row spans up to the
    guard): dgamma sums row and column contributions of every pair that cancel
    in the reverse cumsum, so both sides must use identical operand values.
    With mismatched roundings the dg error grew with the span (bf16 4.8e-2,
    fp32 1e-4 at g_scale 3); it must stay at the level of dq, dk, dv.
    g is fp32, as the layer produces it (D = 64, D = 32 with fp32 inputs)."""
    for D in ((64, 32) if dtype == torch.float32 else (64,)):
        x = _inputs(2, 128, 2, D, dtype, seed=21, grad=True, g_scale=g_scale)
        x["g"] = x["g"].float()
        errs = _bwd_errors(x, dtype)
        _assert_all(errs, TOL[dtype], f"bwd decay span {dtype} g_scale={g_scale} D={D}")
        assert errs["dg"] <= 3 * max(errs["dq"], errs["dk"], errs["dv"]), errs


@pytest.mark.parametrize("g_scale", [8.0, 12.0, 16.0])
def test_bwd_dg_pairwise_strong_decay(g_scale):
    """Per-step decays of -6 to -13 (the reference layer's initial A = e^{A_log}
    up to 16 gives such heads): the pairwise path with in-chunk cumulative
    decays of several hundred, fp32 inputs and fp32 g."""
    x = _inputs(2, 128, 2, 64, torch.float32, seed=22, grad=True, g_scale=g_scale)
    _assert_all(_bwd_errors(x, torch.float32), TOL[torch.float32], f"bwd pairwise strong decay g_scale={g_scale}")


def _block_scaled(x, scales):
    """g scaled per 16-row block of each 64-token chunk (scales[i] for block i), so
    that some diagonal blocks exceed the anchored span guard and others do not."""
    T = x["g"].shape[1]
    f = torch.tensor([scales[(t % 64) // 16] for t in range(T)], dtype=torch.float32)
    x["g"] = (x["g"].float() * f[None, :, None, None]).to(x["g"].dtype)
    return x


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("scales", [(12.0, 0.1, 12.0, 0.1), (0.1, 0.1, 0.1, 14.0), (16.0, 16.0, 0.3, 6.0)])
def test_mixed_span_blocks(dtype, scales):
    """Per-block decays: 16-row blocks beyond the span guard (their diagonal
    tiles pair by pair) next to weakly decaying ones (MFMA), with the block-end
    factors between them spanning hundreds of nats.  Forward and backward."""
    x = _inputs(2, 200, 2, 64, dtype, seed=31, with_state=True, grad=True, g_scale=1.0)
    x = _block_scaled(x, scales)
    x["g"] = x["g"].float()
    _assert_all(_fwd_errors(x, dtype), TOL[dtype], f"fwd mixed spans {dtype} {scales}")
    _assert_all(_bwd_errors(x, dtype), TOL[dtype], f"bwd mixed spans {dtype} {scales}")


@pytest.mark.parametrize("scales", [(12.0, 0.1, 12.0, 0.1), (0.1, 0.1, 0.1, 14.0), (16.0, 16.0, 0.3, 6.0)])
def test_mixed_span_blocks_d128(scales):
    """bf16 at D = 128 (the wide local-adjoint kernel): 16-row blocks beyond the
    span guard next to weakly decaying ones.  Their diagonal tiles go pair by
    pair within the block and the other tiles take exact per-lane factors;
    forward and backward against the fp64 oracle."""
    x = _inputs(1, 200, 2, 128, torch.bfloat16, seed=33, with_state=True, grad=True, g_scale=1.0)
    x = _block_scaled(x, scales)
    x["g"] = x["g"].float()
    _assert_all(_fwd_errors(x, torch.bfloat16), TOL[torch.bfloat16], f"fwd mixed spans D128 {scales}")
    _assert_all(_bwd_errors(x, torch.bfloat16), TOL[torch.bfloat16], f"bwd mixed spans D128 {scales}")


@pytest.mark.parametrize("D", [96, 64])
def test_layer_init_decay(D):
    """The SSv2 layer's decay at initialisation, g = -A_h softplus(N(0, 0.5^2))
    with A_h ~ U[1, 16] per head (nope_gdn_mlx.py:749): nearly every 16-row
    block beyond the span guard, bf16, through the training pair -- at D = 96
    (the SSv2 heads, wide local-adjoint kernel) and D = 64 (config 2's heads,
    the sub-anchored diagonal tiles of the D <= 64 kernel)."""
    kda = _kda()
    B, T, H = 1, 300, 4
    x = _inputs(B, T, H, D, torch.bfloat16, seed=34, with_state=True, grad=True)
    gen = torch.Generator().manual_seed(35)
    A = torch.linspace(1.0, 16.0, H)
    x["g"] = (-A[None, None, :, None] * torch.nn.functional.softplus(0.5 * torch.randn(B, T, H, D, generator=gen))
              ).to(torch.bfloat16)
    q, k, v, g, beta = _dev(x)
    s0, do = x["s0"].to(DEV), x["do"].to(DEV)
    o, sf, ws = kda.kda_forward_train(q, k, v, g, beta, s0)
    grads = kda.kda_backward_train(q, k, v, g, beta, s0, do, None, ws)
    torch.cuda.synchronize()
    ref = cref.forward(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"])
    refb = cref.backward(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], x["do"])
    errs = {"o": R.rel_l2(o.cpu(), ref["o"]), "s_final": R.rel_l2(sf.cpu(), ref["s_final"])}
    errs.update({n: R.rel_l2(gr.cpu(), refb[n]) for n, gr in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), grads)})
    _assert_all(errs, TOL[torch.bfloat16], f"layer-init decay D{D}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_positive_decay_chunks(dtype):
    """g > 0 in some chunks (outside the layer's domain, but the op and the
    reference's step loop accept it): those chunks are evaluated pair by pair
    from the exact exp(gamma_t - gamma_s); the others stay anchored."""
    x = _inputs(1, 260, 2, 64, dtype, seed=32, with_state=True, grad=True, g_scale=0.3)
    g = x["g"].float()
    gen = torch.Generator().manual_seed(33)
    g[:, 64:128] = torch.randn(g[:, 64:128].shape, generator=gen) * 0.05     # chunk 1: mixed signs
    g[:, 200:203] = 0.02                                                      # chunk 3: a few positive rows
    x["g"] = g
    _assert_all(_fwd_errors(x, dtype), TOL[dtype], f"fwd positive decay {dtype}")
    _assert_all(_bwd_errors(x, dtype), TOL[dtype], f"bwd positive decay {dtype}")


def test_bwd_parity_bf16_small():
    x = _inputs(2, 300, 4, 64, torch.bfloat16, seed=13, with_state=True, grad=True)
    _assert_all(_bwd_errors(x, torch.bfloat16), TOL[torch.bfloat16], "bwd bf16 small")


@pytest.mark.parametrize("B,T,H,D,with_state,with_dsf,g_scale", [
    (2, 100, 3, 64, True, True, 0.1),      # ragged last chunk, state + final-state cotangent
    (1, 1, 1, 64, True, False, 0.1),       # single token
    (1, 65, 2, 32, True, True, 0.1),       # D = 32, one-token tail chunk
    (1, 130, 2, 64, True, False, 6.0),     # strong decay: pairwise path
])
def test_bwd_parity_bf16_cases(B, T, H, D, with_state, with_dsf, g_scale):
    x = _inputs(B, T, H, D, torch.bfloat16, seed=14, with_state=with_state, grad=True, g_scale=g_scale)
    dsf = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(9)) if with_dsf else None
    _assert_all(_bwd_errors(x, torch.bfloat16, dsf), TOL[torch.bfloat16],
                f"bwd bf16 {B},{T},{H},{D},{with_state},{with_dsf},{g_scale}")


@pytest.mark.parametrize("B,T,H,D,with_state,with_dsf,g_scale", [
    (1, 200, 2, 128, True, True, 0.1),     # ragged last chunk, state + final-state cotangent
    (2, 64, 3, 128, False, False, 0.1),    # one full chunk, six (b, h)
    (2, 1, 4, 128, True, False, 0.1),      # single token (eight sequences: one token's rel-L2 over
                                           # 128 channels is dominated by single bf16 roundings)
    (1, 130, 2, 128, True, False, 6.0),    # strong decay: every pair pair by pair
    (1, 150, 2, 128, False, True, 1.0),    # strong but anchored decay
])
def test_bwd_parity_bf16_d128(B, T, H, D, with_state, with_dsf, g_scale):
    """The backward at D = 128 (bf16): the generic state recompute (which writes
    V'), the generic reverse carry, and the wide local-adjoint kernel reading
    A_kk and the diagonal inverses from the prep."""
    x = _inputs(B, T, H, D, torch.bfloat16, seed=24, with_state=with_state, grad=True, g_scale=g_scale)
    dsf = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(9)) if with_dsf else None
    _assert_all(_bwd_errors(x, torch.bfloat16, dsf), TOL[torch.bfloat16],
                f"bwd bf16 D128 {B},{T},{H},{D},{with_state},{with_dsf},{g_scale}")


@pytest.mark.parametrize("B,T,H,D,with_state,with_dsf,g_scale", [
    (1, 2000, 2, 128, True, True, 0.1),    # 8 segments of 4 chunks, ragged last chunk
    (2, 2500, 3, 128, True, False, 0.1),   # 10 segments for each of six (b, h)
    (1, 2340, 2, 128, False, True, 1.0),   # 8 segments, the last of 2 chunks; strong decay
    (1, 2560, 2, 96, True, True, 0.1),     # D = 96: 10 segments of the padded state
])
def test_bwd_parity_bf16_segmented_states(B, T, H, D, with_state, with_dsf, g_scale):
    """The bf16 backward at D = 128 (and 96) with its recurrences split over
    segments of the sequence (few long sequences: at least 8 segments): the
    state recompute (segment maps, start states, then each segment's
    chunk-start states h and V') and the reverse carry (each segment's reverse
    map, a reverse scan through the maps' transposes from ds_final, then each
    segment's dh, dV' and dS0)."""
    kda = _kda()
    assert kda.workspace_offsets(1, B, T, H, D, torch.bfloat16)["SegX"] >= 0, "segmented recompute not taken"
    x = _inputs(B, T, H, D, torch.bfloat16, seed=29, with_state=with_state, grad=True, g_scale=g_scale)
    dsf = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(9)) if with_dsf else None
    _assert_all(_bwd_errors(x, torch.bfloat16, dsf), TOL[torch.bfloat16],
                f"bwd bf16 segmented states {B},{T},{H},{D},{with_state},{with_dsf},{g_scale}")


@pytest.mark.parametrize("B,T,H,D,with_state,with_dsf,g_scale", [
    (1, 200, 2, 128, True, True, 0.1),     # ragged last chunk, state + final-state cotangent
    (2, 64, 3, 128, False, False, 0.1),    # one full chunk
    (1, 130, 2, 128, True, False, 6.0),    # strong decay: every pair pair by pair
])
def test_bwd_parity_fp32_d128(B, T, H, D, with_state, with_dsf, g_scale):
    """The fp32 backward at D = 128: the state recompute, the reverse carry on
    four column slices of the state per (batch, head), and the wide
    local-adjoint kernel with split-bf16 products accurate to fp32."""
    x = _inputs(B, T, H, D, torch.float32, seed=26, with_state=with_state, grad=True, g_scale=g_scale)
    dsf = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(9)) if with_dsf else None
    _assert_all(_bwd_errors(x, torch.float32, dsf), TOL[torch.float32],
                f"bwd fp32 D128 {B},{T},{H},{D},{with_state},{with_dsf},{g_scale}")


# ---------------------------------------------------------------- head dimension 96

D96_FWD = [
    (1, 150, 2, torch.float32, True),
    (2, 70, 3, torch.float32, False),      # ragged last chunk
    (1, 1, 1, torch.float32, True),        # single token
    (2, 300, 4, torch.bfloat16, True),
    (1, 129, 2, torch.bfloat16, False),
    (2, 1568, 8, torch.bfloat16, True),    # the reference's SSv2 layer: 8 heads x 96, 1568 tokens
]


@pytest.mark.parametrize("B,T,H,dtype,with_state", D96_FWD)
def test_fwd_parity_d96(B, T, H, dtype, with_state):
    """D = 96 (the reference's SSv2 model, train_mlx_ssv2.py:71-80): the library
    pads to 128 channels in its workspace, runs the D = 128 kernels and crops."""
    kda = _kda()
    assert kda.workspace_offsets(0, B, T, H, 96, dtype)["Pad"] >= 0
    x = _inputs(B, T, H, 96, dtype, seed=27, with_state=with_state)
    _assert_all(_fwd_errors(x, dtype), TOL[dtype], f"fwd D96 {B},{T},{H},{dtype},{with_state}")


@pytest.mark.parametrize("B,T,H,dtype,with_state,with_dsf,g_scale", [
    (1, 150, 2, torch.float32, True, True, 0.1),
    (2, 70, 3, torch.float32, False, False, 0.1),    # ragged last chunk
    (1, 1, 1, torch.float32, True, True, 0.1),       # single token
    (1, 130, 2, torch.float32, True, False, 6.0),    # strong decay
    (2, 100, 3, torch.bfloat16, True, True, 0.1),
    (1, 130, 2, torch.bfloat16, True, False, 6.0),
    (2, 300, 8, torch.bfloat16, False, True, 1.0),
])
def test_bwd_parity_d96(B, T, H, dtype, with_state, with_dsf, g_scale):
    D = 96
    x = _inputs(B, T, H, D, dtype, seed=28, with_state=with_state, grad=True, g_scale=g_scale)
    dsf = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(9)) if with_dsf else None
    _assert_all(_bwd_errors(x, dtype, dsf), TOL[dtype], f"bwd D96 {B},{T},{H},{dtype},{with_state},{with_dsf},{g_scale}")


def test_d96_zero_channels_leave_d128_results():
    """Padding is exact: D = 96 inputs zero-padded to 128 by hand give, through
    the D = 128 path, the D = 96 call's outputs and gradients in their first
    96 channels (bit for bit: the library runs the same kernels on the same
    padded values)."""
    kda = _kda()
    B, T, H = 1, 100, 2
    x = _inputs(B, T, H, 96, torch.bfloat16, seed=29, with_state=True, grad=True)
    pad = lambda t: torch.nn.functional.pad(t, (0, 32))                                   # noqa: E731
    pads = lambda t: torch.nn.functional.pad(t, (0, 32, 0, 32))                           # noqa: E731
    q, k, v, g, beta = _dev(x)
    s0, do = x["s0"].to(DEV), x["do"].to(DEV)
    o96, sf96 = kda.kda_forward(q, k, v, g, beta, s0)
    gr96 = kda.kda_backward(q, k, v, g, beta, s0, do, None)
    o128, sf128 = kda.kda_forward(pad(q), pad(k), pad(v), pad(g), beta, pads(s0))
    gr128 = kda.kda_backward(pad(q), pad(k), pad(v), pad(g), beta, pads(s0), pad(do), None)
    torch.cuda.synchronize()
    assert torch.equal(o96, o128[..., :96]) and torch.equal(sf96, sf128[..., :96, :96])
    for n, a, b in zip(("dq", "dk", "dv", "dg"), gr96[:4], gr128[:4]):
        assert torch.equal(a, b[..., :96]), n
    assert torch.equal(gr96[4], gr128[4]) and torch.equal(gr96[5], gr128[5][..., :96, :96])
    # the padded channels' outputs are zero
    assert not o128[..., 96:].any() and not sf128[..., 96:, :].any() and not sf128[..., :, 96:].any()


def test_bwd_d128_fp32_gate():
    """D = 128 with bf16 q/k/v/beta and a float32 g: dg comes back float32."""
    x = _inputs(1, 100, 2, 128, torch.bfloat16, seed=25, with_state=True, grad=True)
    x["g"] = x["g"].float()
    _assert_all(_bwd_errors(x, torch.bfloat16), TOL[torch.bfloat16], "bwd bf16 D128, fp32 g")


def test_bwd_bf16_operands_fp32_gate():
    """bf16 q/k/v/beta with a float32 g: dg comes back float32."""
    x = _inputs(1, 200, 2, 64, torch.bfloat16, seed=15, with_state=True, grad=True)
    x["g"] = x["g"].float() * (1.0 + 1e-3 * torch.rand(x["g"].shape, generator=torch.Generator().manual_seed(3)))
    errs = _bwd_errors(x, torch.bfloat16)
    _assert_all(errs, TOL[torch.bfloat16], "bwd bf16 operands, fp32 g")


def test_bwd_parity_config2_full():
    """Config 2: fwd + VJP at B=8, H=12, T=1568, D=64 bf16, dO ~ N(0,1) bf16,
    through both the standalone kda_bwd and the training pair that a training
    step (and the benchmark) runs: kda_fwd_train, then kda_bwd_train on its
    workspace.  Both against the fp64 oracle; the pair bit-identical to the
    standalone calls at this full size too."""
    kda = _kda()
    x = _inputs(8, 1568, 12, 64, torch.bfloat16, seed=0, grad=True)
    q, k, v, g, beta = _dev(x)
    do = x["do"].to(DEV)
    o1, sf1 = kda.kda_forward(q, k, v, g, beta, None)
    g1 = kda.kda_backward(q, k, v, g, beta, None, do, None)
    o2, sf2, ws = kda.kda_forward_train(q, k, v, g, beta, None)
    g2 = kda.kda_backward_train(q, k, v, g, beta, None, do, None, ws)
    torch.cuda.synchronize()
    ref = cref.forward(x["q"], x["k"], x["v"], x["g"], x["beta"], None)
    refb = cref.backward(x["q"], x["k"], x["v"], x["g"], x["beta"], None, x["do"])
    names = ("dq", "dk", "dv", "dg", "dbeta", "ds0")
    for label, o, sf, grads in (("config2 standalone", o1, sf1, g1), ("config2 training pair", o2, sf2, g2)):
        errs = {"o": R.rel_l2(o.cpu(), ref["o"]), "s_final": R.rel_l2(sf.cpu(), ref["s_final"])}
        errs.update({n: R.rel_l2(gr.cpu(), refb[n]) for n, gr in zip(names, grads)})
        _assert_all(errs, TOL[torch.bfloat16], label)
    assert torch.equal(o1, o2) and torch.equal(sf1, sf2)
    for n, a, b in zip(names, g1, g2):
        assert torch.equal(a, b), n


# ---------------------------------------------------------------- training pair

@pytest.mark.parametrize("B,T,H,D,dtype,g_scale", [
    (2, 100, 3, 64, torch.bfloat16, 0.1),
    (1, 130, 2, 64, torch.bfloat16, 6.0),     # pairwise path writes both A_qk layouts directly
    (2, 333, 3, 64, torch.bfloat16, 0.1),     # six chunks: the recurrences' LDS sets wrap
    (1, 65, 2, 32, torch.float32, 0.1),
    (1, 1, 1, 64, torch.float32, 0.1),
    (1, 150, 2, 128, torch.bfloat16, 0.1),    # D = 128
    (1, 100, 2, 128, torch.float32, 0.1),
    (1, 150, 2, 96, torch.bfloat16, 0.1),     # D = 96: padded inputs in the pair's workspace
    (2, 70, 2, 96, torch.float32, 0.1),
    (1, 2560, 2, 128, torch.bfloat16, 0.1),   # forward and backward over 10 segments
    (1, 2560, 2, 96, torch.bfloat16, 0.1),
])
def test_training_pair_equals_standalone_calls(B, T, H, D, dtype, g_scale):
    """kda_fwd_train / kda_bwd_train reproduce kda_fwd / kda_bwd bit for bit."""
    kda = _kda()
    x = _inputs(B, T, H, D, dtype, seed=16, with_state=True, grad=True, g_scale=g_scale)
    q, k, v, g, beta = _dev(x)
    s0, do = x["s0"].to(DEV), x["do"].to(DEV)
    dsf = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(4)).to(DEV)
    o1, sf1 = kda.kda_forward(q, k, v, g, beta, s0)
    g1 = kda.kda_backward(q, k, v, g, beta, s0, do, dsf)
    o2, sf2, ws = kda.kda_forward_train(q, k, v, g, beta, s0)
    g2 = kda.kda_backward_train(q, k, v, g, beta, s0, do, dsf, ws)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(sf1, sf2)
    for n, a, b in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), g1, g2):
        assert torch.equal(a, b), n


@pytest.mark.parametrize("B,T,H,D,dtype", [
    (2, 100, 3, 64, torch.bfloat16),
    (1, 65, 2, 32, torch.float32),
    (1, 150, 2, 128, torch.bfloat16),
    (1, 100, 2, 128, torch.float32),
    (1, 150, 2, 96, torch.bfloat16),          # PAD kept, PADB the backward's
    (1, 2560, 2, 128, torch.bfloat16),        # segmented state recompute: the segment regions
    (1, 2560, 2, 96, torch.bfloat16),         # are the backward's
])
def test_training_pair_kept_part_and_split_scratch(B, T, H, D, dtype):
    """kda_fwd_train writes nothing past the kept part of the pair's workspace
    (kda_train_kept_size bytes); kda_bwd_train leaves the kept part as it was;
    kda_bwd_train_split on a copy of the kept part and a separate scratch
    buffer full of NaN bytes gives kda_bwd_train's gradients bit for bit."""
    from mlx_vit_amd import _lib
    from mlx_vit_amd import kda as K
    kda = _kda()
    lib = _lib.load()
    x = _inputs(B, T, H, D, dtype, seed=17, with_state=True, grad=True)
    q, k, v, g, beta = _dev(x)
    s0, do = x["s0"].to(DEV), x["do"].to(DEV)
    total = kda.workspace_bytes(2, B, T, H, D, dtype)
    kept = kda.train_kept_bytes(B, T, H, D, dtype)
    assert 0 < kept < total
    ws = torch.full((total,), 0x5A, dtype=torch.uint8, device=DEV)
    kda.kda_forward_train(q, k, v, g, beta, s0, workspace=ws)
    torch.cuda.synchronize()
    assert bool((ws[kept:] == 0x5A).all()), "the training forward wrote past the kept part"
    kept_copy = ws[:kept].clone()
    g1 = kda.kda_backward_train(q, k, v, g, beta, s0, do, None, ws)     # one buffer: kda_bwd_train
    torch.cuda.synchronize()
    assert torch.equal(ws[:kept], kept_copy), "the backward wrote into the kept part"
    scratch = torch.full((total - kept,), 0xFF, dtype=torch.uint8, device=DEV)   # NaN in fp32 and bf16
    g2 = [torch.empty_like(t) for t in (q, k, v, g, beta)] + [torch.empty_like(s0)]
    rc = lib.kda_bwd_train_split(*(K._ptr(t) for t in (q, k, v, g, beta, s0, do)), None,
                                 *(K._ptr(t) for t in g2), B, T, H, D, 64, K._DTYPE_CODE[dtype],
                                 K._DTYPE_CODE[g.dtype], K._ptr(kept_copy), kept, K._ptr(scratch),
                                 scratch.numel(), K._stream(q.device))
    _lib.check(rc, "kda_bwd_train_split")
    torch.cuda.synchronize()
    for n, a, b in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), g1, g2):
        assert torch.equal(a, b), n


@pytest.mark.parametrize("B,T,H,D,with_state,g_scale", [
    (2, 200, 3, 64, True, 0.1),
    (1, 130, 2, 32, False, 0.1),
    (1, 140, 2, 64, True, 6.0),      # strong decay: the pairwise diagonal tiles
])
def test_head_decay_equals_broadcast(B, T, H, D, with_state, g_scale):
    """g of shape (B, T, H) -- one fp32 decay per head, the scalar-alpha GDN's --
    gives what the same g broadcast over the channels gives: o, S_T and dq, dk,
    dv, dbeta, dS0 bit for bit (standalone calls and the training pair).  dg is
    the channel sum, formed in fp32 in the kernel: the broadcast path's fp32
    per-channel dg summed afterwards (another summation order), and within the
    bf16 bar of the fp64 oracle's channel sum."""
    kda = _kda()
    x = _inputs(B, T, H, D, torch.bfloat16, seed=41, with_state=with_state, grad=True, g_scale=g_scale)
    gen = torch.Generator().manual_seed(42)
    gh = -torch.nn.functional.softplus(torch.randn(B, T, H, generator=gen)) * g_scale
    q, k, v, beta = _dev(x, ("q", "k", "v", "beta"))
    s0 = x["s0"].to(DEV) if with_state else None
    do = x["do"].to(DEV)
    dsf = torch.randn(B, H, D, D, generator=gen).to(DEV)
    g_h = gh.to(DEV)
    g_b = gh[..., None].expand(B, T, H, D).contiguous().to(DEV)
    names = ("dq", "dk", "dv", "dg", "dbeta", "ds0")
    o_h, sf_h = kda.kda_forward(q, k, v, g_h, beta, s0)
    o_b, sf_b = kda.kda_forward(q, k, v, g_b, beta, s0)
    gr_h = kda.kda_backward(q, k, v, g_h, beta, s0, do, dsf)
    gr_b = kda.kda_backward(q, k, v, g_b, beta, s0, do, dsf)
    o_t, sf_t, ws = kda.kda_forward_train(q, k, v, g_h, beta, s0)
    gr_t = kda.kda_backward_train(q, k, v, g_h, beta, s0, do, dsf, ws)
    torch.cuda.synchronize()
    assert torch.equal(o_h, o_b) and torch.equal(sf_h, sf_b)
    assert torch.equal(o_t, o_h) and torch.equal(sf_t, sf_h)
    assert gr_h[3].shape == (B, T, H) and gr_h[3].dtype == torch.float32
    ref = cref.backward(x["q"], x["k"], x["v"], gh[..., None].expand(B, T, H, D), x["beta"], x["s0"], x["do"],
                        dsf.cpu())["dg"].sum(-1)
    for n, a, b, t in zip(names, gr_h, gr_b, gr_t):
        assert torch.equal(a, t), n
        if n == "dg":
            err_hb = R.rel_l2(a.double().cpu(), b.double().sum(-1).cpu())
            err_h = R.rel_l2(a.double().cpu(), ref)
            print("dg channel sum: head vs broadcast", f"{err_hb:.2e}", "head vs fp64 oracle", f"{err_h:.2e}")
            assert err_hb <= 1e-5 and err_h <= TOL[torch.bfloat16], (err_hb, err_h)
        else:
            assert torch.equal(a, b), n


# ---------------------------------------------------------------- committed golden fixtures

def _golden(name):
    import os
    return dict(np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name)))


def test_golden_config0_forward():
    """Config 0 (B1 T256 H2 D64 fp32, zero state) against tests/golden/kda_cfg0.npz."""
    from tests.golden import make_golden as MG
    f, x = _golden("kda_cfg0.npz"), MG.cfg0_inputs()
    np.testing.assert_allclose(MG.checksums(x, MG.NAMES), f["checksums"], rtol=MG.CHECKSUM_RTOL)
    o, sf = _kda().kda_forward(*_dev(x), None)
    torch.cuda.synchronize()
    _assert_all({"o": R.rel_l2(o.cpu(), torch.from_numpy(f["o"])),
                 "s_final": R.rel_l2(sf.cpu(), torch.from_numpy(f["s_final"]))}, 1e-4, "golden cfg0")


def test_golden_backward_d32():
    """B1 T70 H2 D32 fp32 with S0 and dS_final against tests/golden/kda_grads_d32.npz."""
    from tests.golden import make_golden as MG
    f, x = _golden("kda_grads_d32.npz"), MG.grads_inputs()
    np.testing.assert_allclose(MG.checksums(x, MG.NAMES + ("s0", "do", "dsf")), f["checksums"], rtol=MG.CHECKSUM_RTOL)
    kda = _kda()
    q, k, v, g, beta = _dev(x)
    o, sf = kda.kda_forward(q, k, v, g, beta, x["s0"].to(DEV))
    grads = kda.kda_backward(q, k, v, g, beta, x["s0"].to(DEV), x["do"].to(DEV), x["dsf"].to(DEV))
    torch.cuda.synchronize()
    errs = {"o": R.rel_l2(o.cpu(), torch.from_numpy(f["o"])),
            "s_final": R.rel_l2(sf.cpu(), torch.from_numpy(f["s_final"]))}
    for n, gr in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), grads):
        errs[n] = R.rel_l2(gr.cpu(), torch.from_numpy(f[n]))
    _assert_all(errs, 1e-4, "golden d32 backward")


# ---------------------------------------------------------------- autograd / API

def test_autograd_function_matches_direct_backward():
    kda = _kda()
    B, T, H, D = 1, 90, 2, 64
    x = _inputs(B, T, H, D, torch.float32, seed=21, with_state=True, grad=True)
    leaves = [t.to(DEV).requires_grad_(True) for t in (x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"])]
    o, sf = kda.chunk_kda(*leaves)
    dsf = torch.randn(B, H, D, D, device=DEV)
    (o * x["do"].to(DEV)).sum().backward(retain_graph=True)
    g1 = [t.grad.clone() for t in leaves]
    for t in leaves:
        t.grad = None
    ((o * x["do"].to(DEV)).sum() + (sf * dsf).sum()).backward()
    direct = kda.kda_backward(*[t.detach() for t in leaves[:5]], leaves[5].detach(), x["do"].to(DEV), dsf)
    for a, b in zip([t.grad for t in leaves], direct):
        assert R.rel_l2(a.cpu(), b.cpu()) < 1e-6
    ref = R.autograd_reference(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], x["do"])
    for a, n in zip(g1, ("dq", "dk", "dv", "dg", "dbeta", "ds0")):
        assert R.rel_l2(a.cpu(), ref[n]) <= 1e-4, n


def test_recurrence_dispatch_matches_op():
    kda = _kda()
    x = _inputs(1, 64, 2, 64, torch.bfloat16, seed=22)
    q, k, v, g, beta = _dev(x)
    rec = kda.KDARecurrence(num_heads=2, head_dim=64)
    o1, s1 = rec(q, k, v, g, beta)
    o2, s2 = kda.kda_forward(q, k, v, g, beta)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    with pytest.raises(ValueError):
        rec(q, k, v, g, beta, compute_path="metal")


def test_host_arguments_on_other_devices_are_rejected():
    """Tensors the library reads through device pointers must be on q's
    device: a host do, ds_final or workspace is refused before any launch, as
    is a workspace that is not a contiguous byte tensor."""
    kda = _kda()
    x = _inputs(1, 64, 2, 64, torch.bfloat16, seed=23)
    q, k, v, g, beta = _dev(x)
    do = torch.randn(1, 64, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="do is on"):
        kda.kda_backward(q, k, v, g, beta, None, do)
    with pytest.raises(ValueError, match="ds_final is on"):
        kda.kda_backward(q, k, v, g, beta, None, do.to(DEV), torch.zeros(1, 2, 64, 64))
    n = kda.workspace_bytes(0, 1, 64, 2, 64)
    with pytest.raises(ValueError, match="workspace is on"):
        kda.kda_forward(q, k, v, g, beta, workspace=torch.empty(n, dtype=torch.uint8))
    with pytest.raises(ValueError, match="uint8"):
        kda.kda_forward(q, k, v, g, beta, workspace=torch.empty(n // 4 + 1, dtype=torch.float32, device=DEV))
    o, _ = kda.kda_forward(q, k, v, g, beta, workspace=torch.empty(n, dtype=torch.uint8, device=DEV))
    assert torch.equal(o, kda.kda_forward(q, k, v, g, beta)[0])


def test_empty_sequence():
    kda = _kda()
    q = torch.zeros(1, 0, 2, 64, device=DEV)
    beta = torch.zeros(1, 0, 2, device=DEV)
    s0 = torch.randn(1, 2, 64, 64, device=DEV)
    o, sf = kda.kda_forward(q, q, q, q, beta, s0)
    assert o.shape == (1, 0, 2, 64) and torch.equal(sf, s0)


def test_deterministic_repeat():
    kda = _kda()
    x = _inputs(2, 200, 3, 64, torch.bfloat16, seed=23, grad=True)
    q, k, v, g, beta = _dev(x)
    a = kda.kda_forward(q, k, v, g, beta)
    b = kda.kda_forward(q, k, v, g, beta)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    ga = kda.kda_backward(q, k, v, g, beta, None, x["do"].to(DEV))
    gb = kda.kda_backward(q, k, v, g, beta, None, x["do"].to(DEV))
    for u, w in zip(ga, gb):
        assert torch.equal(u, w)


@pytest.mark.parametrize("C", [8, 16, 32])
def test_reference_chunk_sizes_match_chunkwise_oracle(C):
    """chunk_size 8 / 16 / 32 (the reference's other blockings): forward and
    VJP against the oracle's chunkwise restatement of the reference's algorithm
    at that C (nope_gdn_mlx.py:2318-2456, 2579-2720), fp32 to 1e-4 with a ragged
    last chunk and an initial state; the kernels block at 64 whatever C is, so
    the result also equals the chunk_size=64 call bit for bit."""
    kda = _kda()
    B, T, H, D = 1, 100, 2, 64
    x = _inputs(B, T, H, D, torch.float32, seed=29, with_state=True, grad=True)
    q, k, v, g, beta = _dev(x)
    s0, do = x["s0"].to(DEV), x["do"].to(DEV)
    o, sf = kda.kda_forward(q, k, v, g, beta, s0, chunk_size=C)
    grads = kda.kda_backward(q, k, v, g, beta, s0, do, None, chunk_size=C)
    o64, sf64 = kda.kda_forward(q, k, v, g, beta, s0)
    grads64 = kda.kda_backward(q, k, v, g, beta, s0, do, None)
    torch.cuda.synchronize()
    assert torch.equal(o, o64) and torch.equal(sf, sf64)
    for u, w in zip(grads, grads64):
        assert torch.equal(u, w)
    fo = [R.fold_heads(x[n].double()) for n in ("q", "k", "v", "g", "beta")]
    s0f = x["s0"].double().reshape(B * H, D, D)
    ro, rs = R.chunkwise_forward(*fo, s0f, C)
    rg = R.chunkwise_backward(*fo, s0f, R.fold_heads(x["do"].double()), None, C)
    errs = {"o": R.rel_l2(o.cpu(), R.unfold_heads(ro, B, H)), "s_final": R.rel_l2(sf.cpu(), rs.reshape(B, H, D, D))}
    for n, gr, rr in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), grads, rg):
        rr = rr.reshape(B, H, D, D) if n == "ds0" else R.unfold_heads(rr, B, H)
        errs[n] = R.rel_l2(gr.cpu(), rr)
    _assert_all(errs, TOL[torch.float32], f"chunk_size {C}")


# ---------------------------------------------------------------- triangular solve KAT

@pytest.mark.parametrize("upper", [False, True])
def test_solve_triangular_kat(upper):
    """nope_gdn_mlx.py:4793-4835: numpy seed 0 per C, L = tril(randn*0.1, -1) + I,
    b = randn(BH, C, C), rel-max error < 1e-4 against numpy.linalg.solve."""
    kda = _kda()
    BH = 4
    for C in [4, 8, 16, 32, 40, 48, 56, 64]:
        np.random.seed(0)
        Lm = np.tril(np.random.randn(BH, C, C).astype(np.float32) * 0.1, k=-1) + np.eye(C, dtype=np.float32)
        b = np.random.randn(BH, C, C).astype(np.float32)
        Mm = np.ascontiguousarray(np.transpose(Lm, (0, 2, 1))) if upper else Lm
        y_np = np.stack([np.linalg.solve(Mm[i], b[i]) for i in range(BH)])
        y = kda.solve_unit_triangular(torch.from_numpy(Mm).to(DEV), torch.from_numpy(b).to(DEV), upper=upper)
        rel = float(np.max(np.abs(y.cpu().numpy() - y_np))) / (float(np.max(np.abs(y_np))) + 1e-9)
        assert rel < 1e-4, (C, rel)


# ---------------------------------------------------------------- randomized sweep

def _sweep_cases(n=44, seed=20261202):
    """Seeded random shapes: D in {32, 64, 96, 128}, fp32 (D <= 64) or bf16,
    T from 1 to 2600 (ragged and chunk-aligned, single- and multi-segment),
    with or without S0 and dS_T, and three decays: the default, a scaled one
    (g_scale up to 2.5) and the layer's initial decay per head."""
    import random
    rng = random.Random(seed)
    out = []
    for i in range(n):
        D = rng.choice([32, 64, 64, 96, 128, 128])
        dt = "bf16" if (D > 64 or rng.random() < 0.7) else "fp32"
        T = rng.choice([1, 63, 64, 65, 130, 777, 1568, 2100, 2600])
        H = rng.randint(1, 5)
        B = rng.randint(1, 3)
        st = rng.random() < 0.5
        dsf_on = rng.random() < 0.4
        mode = rng.choice(["default", "scaled", "layer"])
        gs = rng.choice([0.1, 0.5, 1.0, 2.5]) if mode == "scaled" else 0.1
        out.append((i, B, T, H, D, dt, st, dsf_on, mode, gs))
    return out


@pytest.mark.parametrize("case", _sweep_cases(), ids=lambda c: f"{c[0]}-B{c[1]}T{c[2]}H{c[3]}D{c[4]}-{c[5]}-{c[8]}")
def test_random_sweep(case):
    """Forward, standalone backward and the training pair on one seeded random
    case, every output and gradient against the fp64 oracle."""
    i, B, T, H, D, dt, st, dsf_on, mode, gs = case
    dtype = torch.bfloat16 if dt == "bf16" else torch.float32
    kda = _kda()
    x = _inputs(B, T, H, D, dtype, seed=100 + i, with_state=st, grad=True, g_scale=gs)
    if mode == "layer":
        gen = torch.Generator().manual_seed(200 + i)
        A = torch.empty(H).uniform_(1.0, 16.0, generator=gen)
        x["g"] = (-A[None, None, :, None] * torch.nn.functional.softplus(
            0.5 * torch.randn(B, T, H, D, generator=gen))).to(x["g"].dtype)
    dsf = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(5)) if dsf_on else None
    errs = {"f_" + k: v for k, v in _fwd_errors(x, dtype).items()}
    errs.update({"b_" + k: v for k, v in _bwd_errors(x, dtype, dsf).items()})
    q, k, v, g, beta = _dev(x)
    s0 = x["s0"].to(DEV) if x["s0"] is not None else None
    o, sf, ws = kda.kda_forward_train(q, k, v, g, beta, s0)
    grads = kda.kda_backward_train(q, k, v, g, beta, s0, x["do"].to(DEV),
                                   None if dsf is None else dsf.to(DEV), ws)
    torch.cuda.synchronize()
    ref = cref.forward(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"])
    refb = cref.backward(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], x["do"], dsf)
    errs["t_o"] = R.rel_l2(o.cpu(), ref["o"])
    errs["t_s_final"] = R.rel_l2(sf.cpu(), ref["s_final"])
    for n, gr in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), grads):
        if gr is not None and refb.get(n) is not None:
            errs["t_" + n] = R.rel_l2(gr.cpu(), refb[n])
    _assert_all(errs, TOL[dtype], f"random sweep {case}")
