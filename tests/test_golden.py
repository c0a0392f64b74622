"""The committed golden fixtures against every CPU implementation of the path.

The fixtures (tests/golden/make_golden.py) come from the fp64 torch step loop
with autograd.  Here they pin the C oracle (the GPU tests' checker), the
chunkwise restatement of nope_gdn_mlx.py:2318-2456 / 2579-2720 and the
per-step adjoint of nope_gdn_mlx.py:3185-3295, and the seeded input generator
itself (checksums).  The GPU side of the same fixtures is in test_kda_gpu.py.
"""
import os
import sys

import numpy as np
import pytest
import torch

from oracle import cref
from oracle import kda_reference as R

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as MG  # noqa: E402

GOLD = os.path.join(HERE, "golden")
BAR = 1e-6      # fixtures are fp64 results stored as float32


def _load(name):
    return dict(np.load(os.path.join(GOLD, name)))


def _t(a):
    return torch.from_numpy(a)


def test_input_generator_matches_fixture_checksums():
    f = _load("kda_cfg0.npz")
    np.testing.assert_allclose(MG.checksums(MG.cfg0_inputs(), MG.NAMES), f["checksums"], rtol=MG.CHECKSUM_RTOL)
    f = _load("kda_grads_d32.npz")
    np.testing.assert_allclose(MG.checksums(MG.grads_inputs(), MG.NAMES + ("s0", "do", "dsf")),
                               f["checksums"], rtol=MG.CHECKSUM_RTOL)


def test_c_oracle_forward_matches_cfg0_fixture():
    f, x = _load("kda_cfg0.npz"), MG.cfg0_inputs()
    ref = cref.forward(*(x[n] for n in MG.NAMES), None)
    assert R.rel_l2(ref["o"], _t(f["o"])) <= BAR
    assert R.rel_l2(ref["s_final"], _t(f["s_final"])) <= BAR


def test_chunkwise_restatement_matches_cfg0_fixture():
    f, x = _load("kda_cfg0.npz"), MG.cfg0_inputs()
    B, T, H, D = x["q"].shape
    fo = [R.fold_heads(x[n].double()) for n in MG.NAMES]
    for C in (16, 64):
        o, sf = R.chunkwise_forward(*fo, None, C)
        assert R.rel_l2(R.unfold_heads(o, B, H), _t(f["o"])) <= BAR
        assert R.rel_l2(sf.reshape(B, H, D, D), _t(f["s_final"])) <= BAR


GRADS = ("dq", "dk", "dv", "dg", "dbeta", "ds0")


def test_c_oracle_backward_matches_grads_fixture():
    f, x = _load("kda_grads_d32.npz"), MG.grads_inputs()
    fw = cref.forward(*(x[n] for n in MG.NAMES), x["s0"])
    assert R.rel_l2(fw["o"], _t(f["o"])) <= BAR
    assert R.rel_l2(fw["s_final"], _t(f["s_final"])) <= BAR
    bw = cref.backward(*(x[n] for n in MG.NAMES), x["s0"], x["do"], x["dsf"])
    for n in GRADS:
        assert R.rel_l2(bw[n], _t(f[n])) <= BAR, n


def test_chunkwise_backward_matches_grads_fixture():
    f, x = _load("kda_grads_d32.npz"), MG.grads_inputs()
    B, T, H, D = x["q"].shape
    fo = [R.fold_heads(x[n].double()) for n in MG.NAMES]
    s0 = x["s0"].double().reshape(B * H, D, D)
    dsf = x["dsf"].double().reshape(B * H, D, D)
    out = R.chunkwise_backward(*fo, s0, R.fold_heads(x["do"].double()), dsf, 64)
    for n, gr in zip(GRADS, out):
        gr = gr.reshape(B, H, D, D) if n == "ds0" else R.unfold_heads(gr, B, H)
        assert R.rel_l2(gr, _t(f[n])) <= BAR, n


def test_step_adjoint_matches_grads_fixture():
    """nope_gdn_mlx.py:3185-3295 replays from the saved u of the rank-1 step."""
    f, x = _load("kda_grads_d32.npz"), MG.grads_inputs()
    B, T, H, D = x["q"].shape
    fo = [R.fold_heads(x[n].double()) for n in MG.NAMES]
    s0 = x["s0"].double().reshape(B * H, D, D)
    o, sf, u = R.step_forward_rank1(*fo, s0)
    assert R.rel_l2(R.unfold_heads(o, B, H), _t(f["o"])) <= BAR
    out = R.python_backward_full(*fo, u, s0, R.fold_heads(x["do"].double()),
                                 x["dsf"].double().reshape(B * H, D, D))
    for n, gr in zip(GRADS, out):
        gr = gr.reshape(B, H, D, D) if n == "ds0" else R.unfold_heads(gr, B, H)
        assert R.rel_l2(gr, _t(f[n])) <= BAR, n


@pytest.mark.parametrize("row", range(len(MG.KAT_SIZES)))
def test_solve_kat_fixture(row):
    """The reference's solve sweep (nope_gdn_mlx.py:4793-4835): inputs regenerate
    from numpy seed 0, and the substitution of the restatement
    reproduces the stored numpy solution."""
    f = _load("solve_kat.npz")
    C, cL, cb, cy = f["table"][row]
    L, b, _ = MG.kat_case(int(C))
    np.testing.assert_allclose([MG.array_checksum(L), MG.array_checksum(b)], [cL, cb], rtol=MG.CHECKSUM_RTOL)
    y = R.solve_unit_lower(torch.from_numpy(L).double(), torch.from_numpy(b).double()).numpy()
    assert abs(MG.array_checksum(y) - cy) <= 1e-9 * abs(cy)
    if int(C) == 16:
        np.testing.assert_allclose(y, f["y16"], rtol=1e-5, atol=1e-6)
