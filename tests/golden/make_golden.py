"""Writes the committed golden fixtures of the KDA path (run from the repo root:
``python tests/golden/make_golden.py``).

The reference's 'compiled' path needs MLX, which is not installable here, and
the reference stores no golden vectors for this op; its only reproducible
known-answer test is the triangular-solve sweep (nope_gdn_mlx.py:4793-4835,
numpy seed 0).  The fixtures are therefore produced by the fp64 torch step
restatement of nope_gdn_mlx.py:616-638 / 890-917 with torch autograd for the
gradients -- an implementation independent of both the C oracle and the HIP
kernels -- on inputs from ``oracle.kda_reference.make_inputs`` (seeded torch
CPU generator, draw order q, k, v, beta, g, [S0], [dO]).  Input checksums are
stored beside the outputs so generator drift is detected instead of silently
changing what the fixtures mean.

Files (float32 outputs, float64 checksums):
  kda_cfg0.npz       config 0: B1 T256 H2 D64 fp32, zero state, seed 0 -- o, s_final
  kda_grads_d32.npz  B1 T70 H2 D32 fp32, S0, dS_final, seed 7 -- o, s_final and
                     dq, dk, dv, dg, dbeta, ds0 for cotangents dO and dS_final
  solve_kat.npz      the reference's solve sweep: per C, checksums of L, b and the
                     numpy solution y (float64), and y itself at C = 16
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import kda_reference as R  # noqa: E402

NAMES = ("q", "k", "v", "g", "beta")
# The generator's fp32 transcendental steps (l2 norm, softplus) may differ in the
# last ulp between CPUs; a drifted generator changes inputs by O(1).
CHECKSUM_RTOL = 1e-6
KAT_SIZES = (4, 8, 16, 32, 40, 48, 56, 64)


def cfg0_inputs():
    return R.make_inputs(1, 256, 2, 64, dtype=torch.float32, seed=0)


def grads_inputs():
    x = R.make_inputs(1, 70, 2, 32, dtype=torch.float32, seed=7, with_state=True, with_grad=True)
    x["dsf"] = torch.randn((1, 2, 32, 32), generator=torch.Generator().manual_seed(8), dtype=torch.float32)
    return x


def checksums(x, names):
    return np.array([R.input_checksum(x[n]) for n in names], dtype=np.float64)


def kat_case(C, BH=4):
    """nope_gdn_mlx.py:4813-4821: L = tril(0.1 N, -1) + I, b = N, numpy seed 0 per C."""
    np.random.seed(0)
    L = np.tril(np.random.randn(BH, C, C).astype(np.float32) * 0.1, k=-1) + np.eye(C, dtype=np.float32)
    b = np.random.randn(BH, C, C).astype(np.float32)
    y = np.stack([np.linalg.solve(L[i].astype(np.float64), b[i].astype(np.float64)) for i in range(BH)])
    return L, b, y


def array_checksum(a):
    return R.input_checksum(torch.from_numpy(np.ascontiguousarray(a)))


def main():
    x = cfg0_inputs()
    o, sf = R.loop_compiled_kda(*(x[n] for n in NAMES), None, compute_dtype=torch.float64)
    np.savez_compressed(os.path.join(HERE, "kda_cfg0.npz"), checksums=checksums(x, NAMES),
                        o=o.numpy().astype(np.float32), s_final=sf.numpy().astype(np.float32))

    x = grads_inputs()
    ref = R.autograd_reference(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], x["do"], x["dsf"])
    out = {n: ref[n].numpy().astype(np.float32) for n in ("o", "s_final", "dq", "dk", "dv", "dg", "dbeta", "ds0")}
    np.savez_compressed(os.path.join(HERE, "kda_grads_d32.npz"),
                        checksums=checksums(x, NAMES + ("s0", "do", "dsf")), **out)

    rows = []
    y16 = None
    for C in KAT_SIZES:
        L, b, y = kat_case(C)
        rows.append([C, array_checksum(L), array_checksum(b), array_checksum(y)])
        if C == 16:
            y16 = y.astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "solve_kat.npz"), table=np.array(rows, dtype=np.float64), y16=y16)
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
