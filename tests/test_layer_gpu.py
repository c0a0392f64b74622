"""GPU parity of the GatedDeltaLayer kernels (producer, gated RMSNorm) and of
the whole layer, through the C ABI, against the CPU restatement in
oracle/layer_reference.py evaluated in fp64 on the same (dtype-rounded) inputs.

Bars: rel-L2 <= 1e-4 with fp32 activations, <= 1e-2 with bf16 activations,
for every output and every gradient (inputs and parameters)."""
import pytest
import torch

from oracle import kda_reference as R
from oracle import layer_reference as LR

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float32: 1e-4, torch.bfloat16: 1e-2}


def _rel(a, b):
    return R.rel_l2(a.detach().cpu().double(), b.detach().cpu().double())


def _check(errs, tol, case):
    print(case, {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    bad = {k: v for k, v in errs.items() if not (v <= tol)}
    assert not bad, f"{case}: {bad} above {tol}"


def _prod_inputs(B, T, H, D, dtype, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    HD = H * D
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    acts = dict(qkv=r(B, T, 3 * HD), xf=r(B, T, HD), xb=r(B, T, H))
    acts = {n: t.to(dtype) for n, t in acts.items()}
    params = dict(conv_w=torch.rand(3, HD, 4, generator=g) - 0.5,
                  conv_b=0.1 * r(3, HD) if bias else None, dt_bias=0.1 * r(HD),
                  A_log=torch.log(1 + 15 * torch.rand(H, generator=g)))
    cots = dict(dq=r(B, T, H, D).to(dtype), dk=r(B, T, H, D).to(dtype), dv=r(B, T, H, D).to(dtype),
                dg=r(B, T, H, D), dbeta=r(B, T, H).to(dtype))
    return acts, params, cots


def _prod_reference(acts, params, cots, H, D, mult):
    HD = H * D
    leaves = {n: t.double().requires_grad_() for n, t in acts.items()}
    leaves.update({n: t.double().requires_grad_() for n, t in params.items() if t is not None})
    xq, xk, xv = leaves["qkv"].split(HD, -1)
    outs = LR.producer_from_projections(xq, xk, xv, leaves["xf"], leaves["xb"], leaves["conv_w"],
                                        leaves.get("conv_b"), leaves["dt_bias"], leaves["A_log"], H, D, mult)
    loss = sum((o * cots[n].double()).sum() for o, n in zip(outs, ("dq", "dk", "dv", "dg", "dbeta")))
    loss.backward()
    return outs, {n: t.grad for n, t in leaves.items()}


PRODUCER_CASES = [
    # B, T, H, D, dtype, bias, beta_mult
    (2, 37, 3, 64, torch.float32, True, 1.0),      # H*D = 192: one wave, a quarter of its lanes idle
    (1, 100, 12, 64, torch.float32, True, 1.0),    # H*D = 768: three waves per row
    (2, 5, 2, 32, torch.float32, True, 1.0),       # T shorter than a strip
    (1, 1, 6, 64, torch.float32, True, 1.0),       # T = 1
    (1, 70, 16, 128, torch.float32, True, 1.0),    # H*D = 2048: eight waves
    (3, 33, 4, 32, torch.float32, False, 2.0),     # no conv bias, allow_neg_eigval
    (2, 77, 12, 64, torch.bfloat16, True, 1.0),
    (1, 40, 6, 64, torch.bfloat16, False, 2.0),
    # enough row segments (>= 16) that the parameter-gradient column sums run
    # as two passes over row slices
    (2, 300, 4, 64, torch.float32, True, 1.0),
    (4, 260, 3, 64, torch.bfloat16, True, 1.0),
    (2, 37, 8, 96, torch.float32, True, 1.0),      # the SSv2 layer's 8 heads x 96
]


@pytest.mark.parametrize("B,T,H,D,dtype,bias,mult", PRODUCER_CASES)
def test_producer_parity(B, T, H, D, dtype, bias, mult):
    from mlx_vit_amd import producer_backward, producer_forward
    acts, params, cots = _prod_inputs(B, T, H, D, dtype, seed=B * 1000 + T, bias=bias)
    case = f"producer B={B} T={T} H={H} D={D} {dtype} bias={bias} mult={mult}"
    print(case, flush=True)
    da = {n: t.to(DEV) for n, t in acts.items()}
    dp = {n: (None if t is None else t.to(DEV)) for n, t in params.items()}
    dc = {n: t.to(DEV) for n, t in cots.items()}
    outs = producer_forward(da["qkv"], da["xf"], da["xb"], dp["conv_w"], dp["conv_b"], dp["dt_bias"],
                            dp["A_log"], H, D, D ** -0.5, mult, torch.float32)
    grads = producer_backward(da["qkv"], da["xf"], da["xb"], dp["conv_w"], dp["conv_b"], dp["dt_bias"],
                              dp["A_log"], dc["dq"], dc["dk"], dc["dv"], dc["dg"], dc["dbeta"], H, D, D ** -0.5,
                              mult)
    torch.cuda.synchronize()
    ref_outs, ref_grads = _prod_reference(acts, params, cots, H, D, mult)
    errs = {n: _rel(o, r) for n, o, r in zip(("q", "k", "v", "g", "beta"), outs, ref_outs)}
    names = ("qkv", "xf", "xb", "conv_w", "conv_b", "dt_bias", "A_log")
    for n, gr in zip(names, grads):
        if n == "conv_b" and not bias:
            assert gr is None
            continue
        errs["d" + n] = _rel(gr, ref_grads[n])
    _check(errs, TOL[dtype], case)


def test_producer_strided_rows():
    """q/k/v read from column slices of a wider fused projection output."""
    from mlx_vit_amd import producer_forward
    B, T, H, D = 2, 50, 4, 32
    HD = H * D
    acts, params, _ = _prod_inputs(B, T, H, D, torch.float32, seed=7)
    wide = torch.randn(B, T, 3 * HD + 64)
    wide[..., 32:32 + 3 * HD] = acts["qkv"]
    d = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    out_wide = producer_forward(d(wide)[..., 32:32 + 3 * HD], d(acts["xf"]), d(acts["xb"]), d(params["conv_w"]),
                                d(params["conv_b"]), d(params["dt_bias"]), d(params["A_log"]), H, D, 0.5)
    out_ref = producer_forward(d(acts["qkv"]), d(acts["xf"]), d(acts["xb"]), d(params["conv_w"]),
                               d(params["conv_b"]), d(params["dt_bias"]), d(params["A_log"]), H, D, 0.5)
    for a, b in zip(out_wide, out_ref):
        assert torch.equal(a, b)


def test_producer_full_size_properties():
    """Config-2 shape in bf16 (B=8, T=1568, H=12, D=64): every q row has norm
    D^-1/2 and every k row norm 1 (to bf16 rounding), g <= 0, 0 < beta < 1,
    and the forward matches the fp32 torch restatement on the GPU."""
    from mlx_vit_amd import producer_forward
    B, T, H, D = 8, 1568, 12, 64
    acts, params, _ = _prod_inputs(B, T, H, D, torch.bfloat16, seed=11)
    da = {n: t.to(DEV) for n, t in acts.items()}
    dp = {n: t.to(DEV) for n, t in params.items()}
    q, k, v, g, beta = producer_forward(da["qkv"], da["xf"], da["xb"], dp["conv_w"], dp["conv_b"], dp["dt_bias"],
                                        dp["A_log"], H, D, D ** -0.5)
    qn = q.float().reshape(B, T, -1).norm(dim=-1)
    kn = k.float().reshape(B, T, -1).norm(dim=-1)
    assert torch.allclose(qn, torch.full_like(qn, D ** -0.5), rtol=4e-3)
    assert torch.allclose(kn, torch.ones_like(kn), rtol=4e-3)
    assert bool((g <= 0).all()) and bool((beta > 0).all()) and bool((beta < 1).all())
    HD = H * D
    xq, xk, xv = da["qkv"].float().split(HD, -1)
    ref = LR.producer_from_projections(xq, xk, xv, da["xf"].float(), da["xb"].float(), dp["conv_w"],
                                       dp["conv_b"], dp["dt_bias"], dp["A_log"], H, D)
    errs = {n: _rel(o.float(), r) for n, o, r in zip(("q", "k", "v", "g", "beta"), (q, k, v, g, beta), ref)}
    _check(errs, TOL[torch.bfloat16], "producer full size")


NORM_CASES = [
    (2, 37, 3, 64, torch.float32),
    (1, 100, 12, 64, torch.float32),
    (2, 5, 4, 32, torch.float32),
    (1, 9, 16, 128, torch.float32),
    (1, 130, 2, 4, torch.float32),
    (4, 65, 12, 64, torch.bfloat16),
    (2, 37, 8, 96, torch.float32),     # D = 96: 32-lane head groups, 24 live lanes each
    (1, 20, 5, 96, torch.float32),     # an odd head count: half of the last wave idle
    (2, 30, 16, 96, torch.bfloat16),   # 16 heads of 96: eight waves
]


@pytest.mark.parametrize("B,T,H,D,dtype", NORM_CASES)
def test_gated_rmsnorm_parity(B, T, H, D, dtype):
    from mlx_vit_amd import gated_rmsnorm_backward, gated_rmsnorm_forward
    case = f"gated_rmsnorm B={B} T={T} H={H} D={D} {dtype}"
    print(case, flush=True)
    g = torch.Generator().manual_seed(T + D)
    o = torch.randn(B, T, H, D, generator=g).to(dtype)
    wide = torch.randn(B, T, H * D + 8, generator=g).to(dtype)   # the gate as a strided column slice
    w = 1 + 0.1 * torch.randn(D, generator=g)
    dy = torch.randn(B, T, H * D, generator=g).to(dtype)
    z = wide[..., 8:]
    y = gated_rmsnorm_forward(o.to(DEV), wide.to(DEV)[..., 8:], w.to(DEV), 1e-5)
    do, dz, dw = gated_rmsnorm_backward(o.to(DEV), wide.to(DEV)[..., 8:], w.to(DEV), 1e-5, dy.to(DEV))
    torch.cuda.synchronize()
    lo, lz, lw = (t.double().requires_grad_() for t in (o, z, w))
    ref = LR.gated_rms_norm(lo, lw, lz.reshape(B, T, H, D), 1e-5).reshape(B, T, H * D)
    (ref * dy.double()).sum().backward()
    errs = {"y": _rel(y, ref), "do": _rel(do, lo.grad), "dz": _rel(dz, lz.grad), "dw": _rel(dw, lw.grad)}
    _check(errs, TOL[dtype], case)


GATED_CASES = [
    # B, T, H, D, dtype, with_state, train, gate column offset (a strided gate)
    (2, 100, 3, 64, torch.bfloat16, True, False, 8),     # ragged last chunk
    (1, 1, 4, 64, torch.bfloat16, False, True, 0),       # T = 1
    (3, 64, 2, 64, torch.bfloat16, False, True, 8),      # one whole chunk
    (2, 200, 12, 64, torch.bfloat16, True, True, 0),     # four chunks (the LDS sets wrap)
    (2, 100, 3, 64, torch.float32, True, True, 4),
    (1, 77, 2, 32, torch.float32, False, False, 0),
]


@pytest.mark.parametrize("B,T,H,D,dtype,with_state,train,pad", GATED_CASES)
def test_fwd_gated_parity(B, T, H, D, dtype, with_state, train, pad):
    """kda_fwd_gated: y against the fp64 C oracle's o followed by the fp64
    gated RMSNorm; o and the final state bit-identical to the unfused forward
    (kda_fwd / kda_fwd_train); y against the standalone norm kernel on that o;
    with the training pass, kda_bwd_train on its workspace bit-identical to the
    unfused training pair."""
    from oracle import cref
    from mlx_vit_amd import (gated_rmsnorm_forward, kda_backward_train, kda_forward, kda_forward_gated,
                             kda_forward_train)
    case = f"fwd_gated B={B} T={T} H={H} D={D} {dtype} state={with_state} train={train} pad={pad}"
    print(case, flush=True)
    x = R.make_inputs(B, T, H, D, dtype=dtype, seed=T + D, with_state=with_state, with_grad=True)
    gen = torch.Generator().manual_seed(11)
    wide = torch.randn(B, T, H * D + pad, generator=gen).to(dtype)
    w = 1 + 0.1 * torch.randn(D, generator=gen)
    d = {n: (None if t is None else t.to(DEV)) for n, t in x.items()}
    args = (d["q"], d["k"], d["v"], d["g"], d["beta"], d["s0"])
    wd = wide.to(DEV)
    y, o, sf, ws = kda_forward_gated(*args, wd[..., pad:], w.to(DEV), 1e-5, train=train)
    if train:
        o_u, sf_u, ws_u = kda_forward_train(*args)
    else:
        o_u, sf_u = kda_forward(*args)
    y_u = gated_rmsnorm_forward(o_u, wd[..., pad:], w.to(DEV), 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(o, o_u), f"{case}: o differs from the unfused forward"
    assert torch.equal(sf, sf_u), f"{case}: final state differs from the unfused forward"
    ref_o = cref.forward(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"])["o"]
    z = wide[..., pad:].double().reshape(B, T, H, D)
    ref = LR.gated_rms_norm(ref_o, w.double(), z, 1e-5).reshape(B, T, H * D)
    errs = {"y": _rel(y, ref), "y_vs_standalone": _rel(y, y_u)}
    if train:
        g1 = kda_backward_train(*args, d["do"], None, ws)
        g2 = kda_backward_train(*args, d["do"], None, ws_u)
        torch.cuda.synchronize()
        for n, a, b in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), g1, g2):
            assert torch.equal(a, b), f"{case}: {n} from the gated forward's workspace differs"
    _check(errs, TOL[dtype], case)
    assert errs["y_vs_standalone"] <= (2e-3 if dtype == torch.bfloat16 else 1e-6), case


def test_fwd_gated_rejects():
    """Unsupported head sizes and bad gate strides raise ValueError."""
    from mlx_vit_amd import kda_forward_gated
    x = R.make_inputs(1, 10, 2, 32, dtype=torch.bfloat16, seed=1)
    d = {n: (None if t is None else t.to(DEV)) for n, t in x.items()}
    z = torch.randn(1, 10, 64, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="no fused kernel"):
        kda_forward_gated(d["q"], d["k"], d["v"], d["g"], d["beta"], None, z, torch.ones(32, device=DEV), 1e-5)
    x = R.make_inputs(1, 10, 2, 64, dtype=torch.bfloat16, seed=1)
    d = {n: (None if t is None else t.to(DEV)) for n, t in x.items()}
    with pytest.raises(ValueError, match="gate shape"):
        kda_forward_gated(d["q"], d["k"], d["v"], d["g"], d["beta"], None, z, torch.ones(64, device=DEV), 1e-5)


def _layer_params(layer):
    return {n: p.detach().cpu().double() for n, p in layer.named_parameters()}


@pytest.mark.parametrize("dtype,with_state,D,fused", [
    (torch.float32, False, 32, True), (torch.float32, True, 32, True), (torch.bfloat16, False, 32, True),
    (torch.float32, True, 64, True), (torch.float32, True, 64, False), (torch.bfloat16, True, 64, True),
    (torch.bfloat16, True, 64, False)])
def test_layer_parity(dtype, with_state, D, fused):
    """The whole GatedDeltaLayer (projections, producer, HIP recurrence, gated
    RMSNorm, o_proj) forward and backward against the fp64 restatement with
    the step recurrence (nope_gdn_mlx.py:775-885 on the 'compiled' path), with
    the output norm fused into the recurrence's store where a kernel has it
    (fused) or as the standalone kernel."""
    _layer_case(dtype, with_state, D, fused, B=2, L=100, H=3, hidden=3 * D)


@pytest.mark.parametrize("dtype,with_state", [(torch.float32, True), (torch.bfloat16, True),
                                              (torch.bfloat16, False)])
def test_layer_parity_ssv2_d96(dtype, with_state):
    """The reference's SSv2 layer, GatedDeltaLayer(768, 8, 96)
    (train_mlx_ssv2.py:71-80): head dimension 96 through the padded recurrence
    and the norm's 32-lane head groups."""
    _layer_case(dtype, with_state, 96, False, B=2, L=100, H=8, hidden=768)


def test_layer_training_step_ssv2_d96():
    """A training step of GatedDeltaLayer(768, 8, 96) in bf16: forward,
    backward, AdamW update; every parameter gets a finite, nonzero gradient,
    the update changes the parameters, and the loss of the next forward on the
    same batch is lower."""
    from mlx_vit_amd import GatedDeltaLayer
    torch.manual_seed(5)
    layer = GatedDeltaLayer(768, 8, 96).to(torch.bfloat16)
    layer.A_log.data = layer.A_log.data.float()
    layer.dt_bias.data = layer.dt_bias.data.float()
    layer = layer.to(DEV)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 1568, 768, generator=g).to(torch.bfloat16).to(DEV)
    target = torch.randn(2, 1568, 768, generator=g).to(torch.bfloat16).to(DEV)
    # lr 1e-2: an AdamW step of about lr moves even a bf16 weight at 1.0 (spacing 2^-7)
    opt = torch.optim.AdamW(layer.parameters(), lr=1e-2)
    before = {n: p.detach().clone() for n, p in layer.named_parameters()}
    losses = []
    for _ in range(2):
        out, _ = layer(x)
        loss = ((out.float() - target.float()) ** 2).mean()
        opt.zero_grad()
        loss.backward()
        if not losses:
            for n, p in layer.named_parameters():
                assert p.grad is not None and torch.isfinite(p.grad).all() and p.grad.abs().sum() > 0, n
        opt.step()
        losses.append(loss.item())
    torch.cuda.synchronize()
    print("ssv2 layer training step losses", losses, flush=True)
    assert losses[1] < losses[0]
    assert all(not torch.equal(before[n], p.detach()) for n, p in layer.named_parameters())


def _layer_case(dtype, with_state, D, fused, B, L, H, hidden):
    from mlx_vit_amd import GatedDeltaLayer
    case = f"layer B={B} L={L} hidden={hidden} H={H} D={D} {dtype} state={with_state} fused={fused}"
    print(case, flush=True)
    torch.manual_seed(3)
    layer = GatedDeltaLayer(hidden, H, D)
    layer.fused_output_norm = fused
    with torch.no_grad():
        layer.dt_bias.normal_(0, 0.1)
        layer.o_norm.weight.normal_(1, 0.1)
    layer = layer.to(dtype)
    # A_log and dt_bias stay fp32 in a bf16 model (nope_gdn_mlx.py:4959-4963)
    layer.A_log.data = layer.A_log.data.float()
    layer.dt_bias.data = layer.dt_bias.data.float()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, L, hidden, generator=g).to(dtype)
    s0 = 0.1 * torch.randn(B, H, D, D, generator=g) if with_state else None
    cot = torch.randn(B, L, hidden, generator=g).to(dtype)
    cot_s = torch.randn(B, H, D, D, generator=g)
    ref_params = _layer_params(layer)
    layer = layer.to(DEV)
    xd = x.to(DEV).requires_grad_()
    s0d = None if s0 is None else s0.to(DEV).requires_grad_()
    out, st = layer(xd, s0d)
    ((out.float() * cot.to(DEV).float()).sum() + (st * cot_s.to(DEV)).sum()).backward()
    torch.cuda.synchronize()

    rp = {n: t.requires_grad_() for n, t in ref_params.items()}
    rx = x.double().requires_grad_()
    rs0 = None if s0 is None else s0.double().requires_grad_()
    keep = {}
    rout, rst = LR.layer_forward(rp, rx, H, D, rs0, keep=keep)
    keep["g"].retain_grad()
    ((rout * cot.double()).sum() + (rst * cot_s.double()).sum()).backward()
    errs = {"out": _rel(out, rout), "state": _rel(st, rst), "dx": _rel(xd.grad, rx.grad)}
    if s0 is not None:
        errs["ds0"] = _rel(s0d.grad, rs0.grad)
    for n, p in layer.named_parameters():
        errs["d" + n] = _rel(p.grad, rp[n].grad)
    # dA_log[h] is the signed sum over (b, t, d) of dg * g (dg/dA_log = g): its
    # error is bounded relative to the sum of the terms' magnitudes, which
    # cancellation can make far larger than the sum itself (the rel-L2 of an
    # H-entry vector of such sums is printed, not asserted)
    terms = (keep["g"].grad * keep["g"]).abs().sum(dim=(0, 1, 3))
    plain = errs.pop("dA_log")
    errs["dA_log/sum|terms|"] = (layer.A_log.grad.detach().cpu().double() - rp["A_log"].grad).norm().item() / \
        terms.norm().item()
    print(case, f"dA_log rel-L2 {plain:.2e}, cancellation factor {terms.norm().item() / rp['A_log'].grad.norm().item():.1f}",
          flush=True)
    _check(errs, TOL[dtype], case)


@pytest.mark.parametrize("B,T,H,D,dtype,with_state,shift", [
    (2, 100, 3, 64, torch.float32, True, 1.5),
    (1, 130, 2, 32, torch.float32, False, 1.5),
    (2, 77, 4, 64, torch.bfloat16, True, 1.5),       # bf16 D <= 64: one decay per (b, t, h) in the kernels
    (1, 150, 2, 32, torch.bfloat16, False, 1.5),
    (1, 130, 2, 64, torch.bfloat16, True, -4.0),     # alpha down to ~0.002: beyond the span guard
])
def test_chunk_gdn_parity(B, T, H, D, dtype, with_state, shift):
    """Scalar-alpha GDN (the reference's original gated delta rule) through the
    KDA kernels against the fp64 step loop (nope_gdn_mlx.py:641-650, 919-947):
    outputs and the gradients of q, k, v, alpha, beta and the initial state."""
    from mlx_vit_amd import chunk_gdn
    case = f"chunk_gdn B={B} T={T} H={H} D={D} {dtype} state={with_state} shift={shift}"
    print(case, flush=True)
    g = torch.Generator().manual_seed(T + D)
    x = R.make_inputs(B, T, H, D, dtype=dtype, seed=T, with_state=with_state, with_grad=True)
    alpha = torch.sigmoid(torch.randn(B, T, H, generator=g) + shift)   # shift 1.5: 0.2 .. 0.98
    cot_s = torch.randn(B, H, D, D, generator=g)
    dev = {n: x[n].to(DEV).requires_grad_() for n in ("q", "k", "v", "beta")}
    a_d = alpha.to(DEV).requires_grad_()
    s0_d = None if x["s0"] is None else x["s0"].to(DEV).requires_grad_()
    o, st = chunk_gdn(dev["q"], dev["k"], dev["v"], a_d, dev["beta"], s0_d)
    ((o.float() * x["do"].to(DEV).float()).sum() + (st * cot_s.to(DEV)).sum()).backward()
    torch.cuda.synchronize()
    ref = {n: x[n].double().requires_grad_() for n in ("q", "k", "v", "beta")}
    a_r = alpha.double().requires_grad_()
    s0_r = None if x["s0"] is None else x["s0"].double().requires_grad_()
    ro, rst = R.loop_compiled_gdn(ref["q"], ref["k"], ref["v"], a_r, ref["beta"], s0_r, compute_dtype=torch.float64)
    ((ro * x["do"].double()).sum() + (rst * cot_s.double()).sum()).backward()
    errs = {"o": _rel(o, ro), "state": _rel(st, rst), "dalpha": _rel(a_d.grad, a_r.grad)}
    for n in ("q", "k", "v", "beta"):
        errs["d" + n] = _rel(dev[n].grad, ref[n].grad)
    if s0_d is not None:
        errs["ds0"] = _rel(s0_d.grad, s0_r.grad)
    _check(errs, TOL[dtype], case)


def test_layer_parity_scalar_alpha():
    """GatedDeltaLayer(channel_wise_decay=False): a_proj gate, producer without
    the decay gate, path hip_chunkwise_gdn, against the fp64 restatement."""
    from mlx_vit_amd import GatedDeltaLayer
    B, L, hidden, H, D = 2, 90, 64, 2, 32
    torch.manual_seed(5)
    layer = GatedDeltaLayer(hidden, H, D, channel_wise_decay=False)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(B, L, hidden, generator=g)
    cot = torch.randn(B, L, hidden, generator=g)
    cot_s = torch.randn(B, H, D, D, generator=g)
    ref_params = _layer_params(layer)
    layer = layer.to(DEV)
    xd = x.to(DEV).requires_grad_()
    out, st = layer(xd)
    ((out * cot.to(DEV)).sum() + (st * cot_s.to(DEV)).sum()).backward()
    torch.cuda.synchronize()
    rp = {n: t.requires_grad_() for n, t in ref_params.items()}
    rx = x.double().requires_grad_()
    rout, rst = LR.layer_forward(rp, rx, H, D)
    ((rout * cot.double()).sum() + (rst * cot_s.double()).sum()).backward()
    errs = {"out": _rel(out, rout), "state": _rel(st, rst), "dx": _rel(xd.grad, rx.grad)}
    for n, p in layer.named_parameters():
        errs["d" + n] = _rel(p.grad, rp[n].grad)
    _check(errs, TOL[torch.float32], "layer scalar alpha")
