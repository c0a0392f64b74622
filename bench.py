#!/usr/bin/env python3
"""Benchmark of the KDA chunkwise recurrence on one MI355X.

A step is one forward + backward (VJP) pass of the op over one batch of
synthetic inputs already resident in HBM: config 2, B=8, H=12, T=1568, D=64,
chunk 64, bf16 q/k/v/g/beta, dO ~ N(0,1) bf16, zero initial state -- run as a
training step does, through the training pair (kda_fwd_train keeps the
per-chunk factors, kda_bwd_train recomputes the chunk-boundary states from
them).  Prints ONE JSON line.  ``value`` is tokens/s = B*T*steps / wall time of
the timed steps.

Per-kernel durations come from HIP events the library records around each of
its launches (kda_profile_*) during a second pass of the same steps; the
dominant kernel's roofline is reported from them.  The ``cpu_baseline`` leg
times the torch fp32 restatement of the reference's 'compiled' path
(nope_gdn_mlx.py:890-917, autograd for the VJP) on the host cores over a
bounded sample, and checks the HIP outputs against the fp64 C oracle.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--workload cfg2]

``--workload layer`` instead times one GatedDeltaLayer forward + backward
(hidden 768, H12, D64, bf16) and reports the KDA kernels' share of the step;
``--workload model`` times the config-4 training step (12 GDN blocks, 8 clips)
and reports the same share.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

METRIC = "KDA fwd+bwd tokens/sec @B8 H12 T1568 d64 bf16; % MFMA peak; rel-L2 err"
PEAK_HBM = 8.0e12            # B/s, MI355X HBM3E
PEAK_BF16 = 2.5e15           # FLOP/s, MI355X dense bf16 MFMA
C = 64

WORKLOADS = {
    # name: (B, T, H, D, backward, with_state, description)
    "cfg2": (8, 1568, 12, 64, True, False,
             "KDA fwd+VJP (training pair), B8 H12 T1568 D64 bf16 (config 2)"),
    "cfg1": (8, 1568, 12, 64, False, False, "KDA fwd, B8 H12 T1568 D64 bf16 (config 1)"),
    "cfg3": (1, 32768, 16, 128, False, True, "KDA fwd, B1 H16 T32768 D128 bf16, fp32 S0 (config 3)"),
    # config 3's shape trained: 16 long sequences at D = 128 (the backward's
    # state recompute over segments)
    "cfg3-train": (1, 32768, 16, 128, True, True,
                   "KDA fwd+VJP (training pair), B1 H16 T32768 D128 bf16, fp32 S0 (config 3's shape)"),
    # the reference's SSv2 layer (train_mlx_ssv2.py:71-80): 8 heads of 96, 1568 tokens
    "ssv2-d96": (8, 1568, 8, 96, True, False, "KDA fwd+VJP (training pair), B8 H8 T1568 D96 bf16 (SSv2 layer)"),
    # config 2's shape with the decay of the reference layer at initialisation:
    # g = -A_h softplus(x), A_h = e^{A_log} ~ U[1, 16] per head (nope_gdn_mlx.py:749),
    # x ~ N(0, 0.5^2) for the gate projection plus dt_bias (zero at init)
    "cfg2-layerdecay": (8, 1568, 12, 64, True, False,
                        "KDA fwd+VJP (training pair), B8 H12 T1568 D64 bf16, layer-init decay "
                        "g = -A_h softplus(N(0, 0.5^2)), A_h ~ U[1, 16]"),
    "ssv2-d96-layerdecay": (8, 1568, 8, 96, True, False,
                            "KDA fwd+VJP (training pair), B8 H8 T1568 D96 bf16 (SSv2 layer), layer-init decay "
                            "g = -A_h softplus(N(0, 0.5^2)), A_h ~ U[1, 16]"),
    # the scalar-alpha sibling (chunk_gdn, nope_gdn_mlx.py:641-650): one decay per
    # (b, t, h), alpha = e^{-softplus(N(0, 1)) * 0.1}, run as the KDA pair on
    # g = log(alpha) given once per head (bf16, D = 64), with chunk_gdn's host
    # work (the log, d alpha = dg / alpha) inside the timed step
    "gdn-cfg2": (8, 1568, 12, 64, True, False,
                 "scalar-alpha GDN fwd+VJP (chunk_gdn: the KDA pair on g = log alpha, one decay per head), "
                 "B8 H12 T1568 D64 bf16"),
}
LAYER_DECAY = {"cfg2-layerdecay", "ssv2-d96-layerdecay"}
SCALAR_DECAY = {"gdn-cfg2"}


def op_counts(B, T, H, D, backward):
    """Algorithmic FLOPs and HBM bytes of the whole op (bf16 inputs, fp32 states):
    FLOPs per token-head 10CD + 6D^2 + (2/3)C^2 forward, x3 for fwd+bwd; bytes =
    inputs once, outputs once, states at fp32, nothing stored between passes."""
    n = B * T * H
    f_fwd = 10 * C * D + 6 * D * D + (2.0 / 3.0) * C * C
    flops = n * f_fwd * (3 if backward else 1)
    es = 2
    states = B * H * D * D * 4
    fwd_bytes = n * (4 * D + 1) * es + n * D * es + states
    if not backward:
        return flops, fwd_bytes
    bwd_bytes = n * (5 * D + 1) * es + n * (4 * D + 1) * es + states
    return flops, fwd_bytes + bwd_bytes


def seg_plan(BH, nc):
    """Segments of the bf16 D = 128 forward (kda_seg.hip seg_plan): about 256
    workgroups, at least 4 chunks per segment; (nseg, chunks per segment)."""
    ns = max(1, min(256 // max(BH, 1), nc // 4))
    length = -(-nc // ns)
    return -(-nc // length), length


def kernel_counts(B, T, H, D, es=2):
    """kernel_counts_at for the kernels' head dimension: D = 96 runs the D = 128
    kernels with channels 96..127 zero, so its FLOPs and workspace bytes are
    those of D = 128 (an upper bound for the prep and the local kernel, which
    read and write 96-channel rows of the op's tensors) while its op bytes are
    D = 96's."""
    if D == 96:
        fl, _, ws = kernel_counts_at(B, T, H, 128, es)
        _, alg, _ = kernel_counts_at(B, T, H, 96, es)
        return fl, alg, ws
    return kernel_counts_at(B, T, H, D, es)


def kernel_counts_at(B, T, H, D, es=2):
    """Per-launch figures of each library kernel (ids as in kda_profile_name):
    (flops, alg_bytes, ws_bytes).

    flops: the dense products the kernel owns, full rectangles, 2 per MAC, per
    padded token-head.

    alg_bytes: the op's minimum HBM traffic (the forward reads q, k,
    v, g, beta once and writes o; the backward reads q, k, v, g, beta, dO once
    and writes dq, dk, dv, dg, dbeta; states fp32, read or written once),
    attributed to the kernel that moves it -- prep the forward's inputs, the
    forward recurrence o and the states, the reverse carry dS_T / dS_0, the
    local-adjoint kernel the whole backward I/O.  Per valid token-head at D = 64
    bf16: 514 B (prep), 128 B (recur fwd), 1,156 B (local).  The state
    recompute moves no op-level bytes at all.

    ws_bytes: every input and output tensor of the kernel touched once,
    workspace slabs included (the inter-kernel traffic of this design) -- (B, T,
    H, *) tensors over the T valid tokens, workspace slabs over every chunk --
    with the library's storage types: operands and the W/U/Qp/Kb/V'/dV'/A/h/dh
    workspace in the input dtype (``es`` bytes), Akk, the diagonal-block
    inverses, e^G and the states in fp32.  With bf16 inputs the local-adjoint
    kernel recomputes Akk, the inverses and V', so no kernel moves them."""
    nc = -(-T // C)
    N = B * H * nc              # chunks
    n = N * C                   # padded token-heads
    nt = B * T * H              # valid token-heads
    f4 = 4
    CD, CC, DD, TII = C * D, C * C, D * D, 4 * 16 * 16
    state = B * H * DD * f4
    x = 0 if es == 2 else 1     # Akk, inverses and V' exist in the workspace (fp32 only)
    tr = es == 2 and D == 64    # bf16 D = 64: no transposed slabs
    fl = {
        0: n * (8 * C * D + (2.0 / 3.0) * C * C),       # Akk, Aqk, W, U, solve
        1: n * (6 * D * D + 2 * C * D),                 # W S, Qp S, Kb^T V', Aqk V'
        2: n * (8 * C * D + (2.0 / 3.0) * C * C),
        3: n * (4 * D * D),                             # W S, Kb^T V'
        4: n * (2 * C * D + 6 * D * D),                 # Aqk^T dO, Kb dS, Qp^T dO, W^T dV'
        # dQp, dKb, dW (6D^2); dAqk 2CD; transposed solve on [dW|dU] 4CD; dL 4CD;
        # the four decay-masked K K^T / Q K^T adjoint products 8CD
        # bf16 also recomputes V' = U - W h (2D^2) and the lower half of Akk (CD)
        5: n * (6 * D * D + 18 * C * D) + (1 - x) * n * (2 * D * D + C * D),
        6: n * (8 * C * D + (2.0 / 3.0) * C * C),
    }
    # the segmented forward (bf16 D = 128): maps of segments 0 .. nseg-2 (the
    # chunk loop on 2D columns, no O), nseg-1 start-state steps, the forward
    nseg, seg_len = seg_plan(B * H, nc) if (es == 2 and D == 128) else (1, nc)
    nmap = B * H * max(0, min(nc, (nseg - 1) * seg_len))      # chunks covered by pass A
    fl[11] = nmap * C * 8 * D * D                       # W Sigma, Kb^T V' on D + D columns
    fl[12] = B * H * (nseg - 1) * 2 * D * D * D         # M Sigma per segment boundary
    fl[13] = fl[1]
    io_in = nt * (4 * D + 1) * es                       # q, k, v, g, beta
    alg = {
        11: 0, 12: 0, 13: nt * D * es + state,          # o, S_final (and S_0)
        0: io_in, 2: io_in, 6: io_in,                   # the forward's inputs
        1: nt * D * es + state,                         # o, S_final (S_0 with an initial state)
        3: 0,
        4: 2 * state,                                   # dS_T in, dS_0 out (bounded above by these)
        5: nt * (5 * D + 1) * es + nt * (4 * D + 1) * es,   # q k v g beta dO in; dq dk dv dg dbeta out
    }
    segmap = B * H * nseg * DD * f4                     # one [D][D] fp32 per (b, h, segment)
    ws = {
        11: nmap * (3 * CD * es + D * f4) + 2 * segmap,                                      # W U KbT eG -> X, M
        12: 3 * segmap,                                                                      # M X -> Sigma_in
        13: N * (4 * CD * es + CC * es + D * f4) + segmap + nt * D * es + state,            # slabs, Sigma_in -> o
        0: io_in + N * (4 * CD * es + CC * es + D * f4),                                   # -> W U Qp Kb(T) Aqk eG
        1: N * (4 * CD * es + CC * es + D * f4) + nt * D * es + state,                      # -> o, S_final
        # -> W U Qp Kb Aqk eG (bf16 D = 64) | W U KbT WT QpT Kb AqkT [Akk Tii] eG
        2: io_in + (N * (4 * CD * es + CC * es + D * f4) if tr else
                    N * (6 * CD * es + CC * es + x * (CC + TII) * f4 + D * f4)),
        3: N * (3 * CD * es + D * f4 + DD * es + x * CD * es),                              # -> h [V']
        4: N * (CC * es + 3 * CD * es + D * f4 + DD * es + CD * es) + nt * D * es + state,  # Aqk(T) Kb Qp(T) W(T) -> dh, dV', dS0
        5: io_in + nt * D * es + N * ((3 + x) * CD * es + 2 * DD * es + x * (CC + TII) * f4)
           + nt * (4 * D + 1) * es,                                                         # -> dq dk dv dg dbeta
        6: io_in + (N * (4 * CD * es + CC * es + D * f4) if tr else                      # -> both sets
                    N * (7 * CD * es + 2 * CC * es + x * (CC + TII) * f4 + D * f4)),
    }
    # the state recompute and the reverse carry in one launch (bf16 D = 128)
    fl[14], alg[14], ws[14] = fl[3] + fl[4], alg[3] + alg[4], ws[3] + ws[4]
    return fl, alg, ws


def make_inputs_gpu(B, T, H, D, with_state, seed=0, layer_decay=False, scalar_decay=False):
    """Synthetic inputs with the configs' distributions, drawn on the GPU.  With
    ``layer_decay`` g follows the reference layer at initialisation instead:
    -A_h softplus(N(0, 0.5^2)) with A_h ~ U[1, 16] per head.  With
    ``scalar_decay`` the returned g is alpha = e^{-softplus(N(0, 1)) * 0.1} of
    shape (B, T, H), the scalar-alpha GDN's decay."""
    import torch
    gen = torch.Generator(device="cuda").manual_seed(seed)
    shp = (B, T, H, D)

    def l2n(x):
        return x / torch.clamp(torch.linalg.vector_norm(x, dim=-1, keepdim=True), min=1e-12)
    q = l2n(torch.randn(shp, generator=gen, device="cuda"))
    k = l2n(torch.randn(shp, generator=gen, device="cuda"))
    v = torch.randn(shp, generator=gen, device="cuda")
    beta = torch.sigmoid(torch.randn((B, T, H), generator=gen, device="cuda"))
    if layer_decay:
        A = torch.empty(H, device="cuda").uniform_(1.0, 16.0, generator=gen)
        g = -A[None, None, :, None] * torch.nn.functional.softplus(
            0.5 * torch.randn(shp, generator=gen, device="cuda"))
    elif scalar_decay:
        g = torch.exp(-torch.nn.functional.softplus(torch.randn((B, T, H), generator=gen, device="cuda")) * 0.1)
    else:
        g = -torch.nn.functional.softplus(torch.randn(shp, generator=gen, device="cuda")) * 0.1
    s0 = torch.randn((B, H, D, D), generator=gen, device="cuda") * 0.02 if with_state else None
    do = torch.randn(shp, generator=gen, device="cuda")
    bf = torch.bfloat16
    return q.to(bf), k.to(bf), v.to(bf), g.to(bf), beta.to(bf), s0, do.to(bf)


def load_traffic(kernel_name):
    """HBM bytes per dispatch of a kernel from the committed rocprofv3 PMC
    summary (profiles/traffic.json), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(kernel_name)
        return None if rec is None else float(rec["bytes_per_dispatch"])
    except (OSError, ValueError, KeyError):
        return None


# ---------------------------------------------------------------------------
# HBM traffic from rocprofv3 PMC counters
# ---------------------------------------------------------------------------
PROFILE_ROLES = {
    # rocprof kernel symbol fragment -> profile names in dispatch order within a
    # fwd+bwd step (the training pair: one prep launch, in its training mode)
    "kda_prep_kernel": ["kda_prep_kernel(train)"],
    "kda_recur": ["kda_recur_kernel(fwd)", "kda_recur_kernel(states)"],
    "kda_dh": ["kda_dh_kernel"],
    "kda_bwd_local": ["kda_bwd_local_kernel"],
}
CALIB_FRAGMENT = "neg_kernel"


def copy_calibration(mb):
    """One plain streaming kernel of known size for scaling the PMC byte
    counters: y = -x over ``mb`` MiB of fp32 reads and as many writes."""
    import torch
    x = torch.ones((mb << 20) // 4, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    torch.neg(x, out=y)
    torch.cuda.synchronize()
    return x.numel() * 4


def _pmc_rows(root, counter):
    """(dispatch id, kernel name, value) per dispatch of ``counter`` from every
    counter_collection.csv under ``root``."""
    import csv
    vals = {}
    for dirpath, _, files in os.walk(root):
        for fn in files:
            if not fn.endswith("counter_collection.csv"):
                continue
            with open(os.path.join(dirpath, fn), newline="") as f:
                for row in csv.DictReader(f):
                    if row.get("Counter_Name") != counter:
                        continue
                    key = (int(row.get("Process_Id", 0) or 0), int(row["Dispatch_Id"]))
                    name, v = vals.get(key, (row["Kernel_Name"], 0.0))
                    vals[key] = (name, v + float(row["Counter_Value"]))
    return [(k[1], n, v) for k, (n, v) in sorted(vals.items())]


def pmc_summary(fetch_dir, write_dir, calib_mb):
    """Per-dispatch HBM bytes of each library kernel: FETCH_SIZE and WRITE_SIZE
    (KiB per dispatch) averaged over dispatches, each scaled by the ratio of
    the calibration kernel's known bytes to what the same counter read for it."""
    calib_bytes = (calib_mb << 20) // 4 * 4
    out = {"calibration": {"kernel": CALIB_FRAGMENT, "bytes_read": calib_bytes, "bytes_written": calib_bytes}}
    per = {}
    for counter, root, key in (("FETCH_SIZE", fetch_dir, "fetch"), ("WRITE_SIZE", write_dir, "write")):
        rows = _pmc_rows(root, counter)
        cal = [v for _, n, v in rows if CALIB_FRAGMENT in n]
        if not cal:
            raise SystemExit(f"no {CALIB_FRAGMENT} dispatch with {counter} under {root}")
        factor = calib_bytes / (max(cal) * 1024.0)
        out["calibration"][f"{key}_kib"] = max(cal)
        out["calibration"][f"{key}_factor"] = round(factor, 5)
        seen = {}
        for _, name, v in rows:
            for frag, roles in PROFILE_ROLES.items():
                if frag in name:
                    i = seen.get(frag, 0)
                    seen[frag] = i + 1
                    rec = per.setdefault(roles[i % len(roles)], {})
                    rec.setdefault(key, []).append(v)
    for name, rec in per.items():
        r = {"dispatches": len(rec.get("fetch", []))}
        total = 0.0
        for key in ("fetch", "write"):
            kib = sum(rec[key]) / len(rec[key])
            r[f"{key}_kib"] = round(kib, 1)
            b = kib * 1024.0 * out["calibration"][f"{key}_factor"]
            r[f"{key}_bytes"] = round(b)
            total += b
        r["bytes_per_dispatch"] = round(total)
        out[name] = r
    return out


# waves per SIMD of each library kernel at config 2 (occupancy set by its
# workgroup size and LDS): the prep runs two 8-wave workgroups per CU
SIMD_WAVES = {"kda_prep_kernel(train)": 4}
SQ_CYCLE_COUNTERS = ("SQ_WAVE_CYCLES", "SQ_WAIT_INST_ANY", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_VALU",
                     "SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_ANY", "SQ_WAIT_ANY")


def pmc_sq_summary(*dirs):
    """Per-wave SQ counters of each library kernel from rocprofv3 --pmc runs,
    averaged over dispatches and divided by SQ_WAVES; the cycle counters count
    in units of 4 cycles and are scaled by 4.  bank_conflict_share =
    SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE; valu_busy_simd = waves per SIMD x
    VALU active cycles / wave cycles."""
    names = set()
    for root in dirs:
        for dirpath, _, files in os.walk(root):
            for fn in files:
                if fn.endswith("counter_collection.csv"):
                    import csv
                    with open(os.path.join(dirpath, fn), newline="") as f:
                        names.update(r["Counter_Name"] for r in csv.DictReader(f))
    per = {}
    for counter in sorted(names):
        for root in dirs:
            seen = {}
            for _, name, v in _pmc_rows(root, counter):
                for frag, roles in PROFILE_ROLES.items():
                    if frag in name:
                        i = seen.get(frag, 0)
                        seen[frag] = i + 1
                        per.setdefault(roles[i % len(roles)], {}).setdefault(counter, []).append(v)
    out = {"source": "rocprofv3 --pmc (SQ counters, per wave)"}
    for kname, rec in per.items():
        avg = {c: sum(v) / len(v) for c, v in rec.items()}
        waves = avg.get("SQ_WAVES", 0.0)
        if not waves:
            continue
        r = {"waves": round(waves)}
        for c, v in avg.items():
            if c == "SQ_WAVES":
                continue
            r[c.lower() + "_per_wave"] = round(v * (4 if c in SQ_CYCLE_COUNTERS else 1) / waves, 1)
        if avg.get("SQ_LDS_IDX_ACTIVE"):
            r["bank_conflict_share"] = round(avg.get("SQ_LDS_BANK_CONFLICT", 0.0) / avg["SQ_LDS_IDX_ACTIVE"], 4)
        if avg.get("SQ_WAVE_CYCLES"):
            r["valu_busy_simd"] = round(SIMD_WAVES.get(kname, 2) * avg.get("SQ_ACTIVE_INST_VALU", 0.0)
                                        / avg["SQ_WAVE_CYCLES"], 4)
        out[kname] = r
    return out


def layer_decay_g(B, T, H, D, seed):
    """g of the reference layer at initialisation, drawn on the CPU:
    -A_h softplus(N(0, 0.5^2)) with A_h ~ U[1, 16] per head (the distribution
    make_inputs_gpu draws for the layer-decay workloads)."""
    import torch
    gen = torch.Generator(device="cpu").manual_seed(seed + 1000)
    A = torch.empty(H).uniform_(1.0, 16.0, generator=gen)
    return -A[None, None, :, None] * torch.nn.functional.softplus(0.5 * torch.randn((B, T, H, D), generator=gen))


def pmc_mfma_summary(util_dir, raw_dir=None):
    """Per-kernel MFMA use from rocprofv3 PMC runs, averaged over dispatches:
    ``mfma_busy`` = rocprofv3's derived MfmaUtil / 100 (SQ_VALU_MFMA_BUSY_CYCLES
    summed over the SIMDs / (GRBM_GUI_ACTIVE x SIMD count)), and the MFMA
    FLOPs the hardware issued per dispatch (SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512,
    rocprofv3's MfmaFlopsBF16) -- the split-bf16 products of the fp32-accurate
    solves included.  With ``raw_dir`` (a second run of SQ_VALU_MFMA_BUSY_CYCLES
    and GRBM_GUI_ACTIVE) the raw counters are reported beside them."""
    out = {"source": "rocprofv3 --pmc MfmaUtil SQ_INSTS_VALU_MFMA_MOPS_BF16"}
    per = {}
    counters = [("MfmaUtil", util_dir, "util_pct"), ("SQ_INSTS_VALU_MFMA_MOPS_BF16", util_dir, "mops_bf16")]
    if raw_dir:
        counters += [("SQ_VALU_MFMA_BUSY_CYCLES", raw_dir, "mfma_busy_cycles"), ("GRBM_GUI_ACTIVE", raw_dir, "gui_active")]
    for counter, root, key in counters:
        seen = {}
        for _, name, v in _pmc_rows(root, counter):
            for frag, roles in PROFILE_ROLES.items():
                if frag in name:
                    i = seen.get(frag, 0)
                    seen[frag] = i + 1
                    per.setdefault(roles[i % len(roles)], {}).setdefault(key, []).append(v)
    for name, rec in per.items():
        r = {k: round(sum(v) / len(v), 3) for k, v in rec.items()}
        r["dispatches"] = len(rec.get("util_pct", []))
        if "util_pct" in r:
            r["mfma_busy"] = round(r["util_pct"] / 100.0, 5)
        if "mops_bf16" in r:
            r["mfma_flops_bf16"] = round(r.pop("mops_bf16") * 512)
        out[name] = r
    return out


def load_mfma(kernel_name):
    """Counter-derived MFMA use of a kernel from the committed summary
    (profiles/mfma.json): (busy fraction, MFMA FLOPs per dispatch) or Nones."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "mfma.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(kernel_name)
        if rec is None:
            return None, None
        return rec.get("mfma_busy"), rec.get("mfma_flops_bf16")
    except (OSError, ValueError, KeyError):
        return None, None


def cpu_baseline_leg(B, T, H, D, backward, with_state, hip_out, sample_tokens, seed=0, layer_decay=False,
                     scalar_decay=False):
    """Time the torch fp32 restatement of the reference 'compiled' path on the
    host cores (bounded sample: the same B, H, D over `sample_tokens` steps),
    and measure rel-L2 of the HIP results against the fp64 C oracle on the
    same seeded inputs at the full workload size (drawn on the CPU so the
    oracle can regenerate them), through the same entry points as the timed
    step (kda_fwd_train + kda_bwd_train for a fwd+bwd workload).  With
    ``layer_decay`` the parity inputs carry the layer-init decay the timed
    workload uses (layer_decay_g), not make_inputs' default; with
    ``scalar_decay`` one decay per (b, t, h), alpha = e^{-softplus(N(0, 1)) *
    0.1}: the HIP side gets g = log(alpha) once per head as chunk_gdn passes
    it, the oracle the same g broadcast over D; dg is compared as the sum over
    the channels, and d alpha = dg / alpha is checked too."""
    import torch
    from oracle import cref
    from oracle import kda_reference as R
    import mlx_vit_amd as kda

    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    # --- timing sample
    Ts = min(T, sample_tokens)
    xs = R.make_inputs(B, Ts, H, D, dtype=torch.float32, seed=seed, with_state=with_state, with_grad=True)

    def run():
        leaves = [xs[nm].clone().requires_grad_(backward) for nm in ("q", "k", "v", "g", "beta")]
        o, sf = R.loop_compiled_kda(*leaves, xs["s0"], compute_dtype=torch.float32)
        if backward:
            torch.sum(o * xs["do"]).backward()
    run()                                  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t_med = sorted(times)[1]
    cpu_tps = B * Ts / t_med
    # --- parity at the full workload size
    x = R.make_inputs(B, T, H, D, dtype=torch.bfloat16, seed=seed, with_state=with_state, with_grad=backward)
    if layer_decay:
        x["g"] = layer_decay_g(B, T, H, D, seed).to(torch.bfloat16)
    alpha = None
    dev = lambda t: None if t is None else t.to("cuda")
    q, k, v, g, beta, s0 = (dev(x[nm]) for nm in ("q", "k", "v", "g", "beta", "s0"))
    if scalar_decay:
        from mlx_vit_amd.kda import GDN_LOG_ALPHA_MIN
        gen = torch.Generator(device="cpu").manual_seed(seed + 2000)
        alpha = torch.exp(-torch.nn.functional.softplus(torch.randn((B, T, H), generator=gen)) * 0.1)
        gh = torch.clamp(torch.log(alpha), min=GDN_LOG_ALPHA_MIN)
        x["g"] = gh[..., None].expand(B, T, H, D).contiguous()
        g = dev(gh)
    # through the entry points the timed step calls: the training pair for a
    # fwd+bwd workload, the plain forward otherwise
    if backward:
        o, sf, ws = kda.kda_forward_train(q, k, v, g, beta, s0)
    else:
        o, sf = kda.kda_forward(q, k, v, g, beta, s0)
    ref = cref.forward(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"])
    errs = {"o": R.rel_l2(o.cpu(), ref["o"]), "s_final": R.rel_l2(sf.cpu(), ref["s_final"])}
    if backward:
        grads = kda.kda_backward_train(q, k, v, g, beta, s0, dev(x["do"]), None, ws)
        rb = cref.backward(x["q"], x["k"], x["v"], x["g"], x["beta"], x["s0"], x["do"])
        for nm, gr in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), grads):
            want = rb[nm].double().sum(-1) if (alpha is not None and nm == "dg") else rb[nm]
            errs[nm] = R.rel_l2(gr.cpu(), want)
        if alpha is not None:
            errs["dalpha"] = R.rel_l2(grads[3].double().cpu() / alpha.double(),
                                      rb["dg"].double().sum(-1) / alpha.double())
    baseline = {
        "value": round(cpu_tps, 2), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
        "sample": (f"torch fp32 restatement of _loop_compiled_kda (D x D x D step matmul, autograd VJP) "
                   f"at B={B} H={H} D={D} over T={Ts} tokens, median of 3 after 1 warm-up, "
                   f"{t_med:.2f} s per {'fwd+bwd' if backward else 'fwd'}"),
    }
    return baseline, {n: float(f"{e:.3e}") for n, e in errs.items()}


LAYER_METRIC = "GatedDeltaLayer fwd+bwd tokens/sec @B8 L1568 hidden768 H12 D64 bf16"
LAYER_KERNELS = {7: "producer_fwd", 8: "producer_bwd", 9: "rmsnorm_fwd", 10: "rmsnorm_bwd"}


def layer_kernel_bytes(B, T, H, D, es=2):
    """Algorithmic HBM bytes of the layer's element-wise kernels per call (bf16
    activations, fp32 g / dg): each input read once, each output written once."""
    N, HD = B * T, H * D
    return {
        7: N * ((3 * HD + HD + H) * es + 3 * HD * es + HD * 4 + H * es),
        8: N * ((3 * HD + HD + H) * es + 3 * HD * es + HD * 4 + H * es + (3 * HD + HD + H) * es),
        9: N * (2 * HD * es + HD * es),
        10: N * (3 * HD * es + 2 * HD * es),
    }


def layer_bench(args):
    """One GatedDeltaLayer (nope_gdn_mlx.py:653-885) forward + backward in bf16
    (A_log / dt_bias fp32) on x (8, 1568, 768): projections as torch GEMMs, the
    producer, recurrence and gated-RMSNorm kernels of this library."""
    import ctypes
    import torch
    import mlx_vit_amd as kda
    from mlx_vit_amd import _lib

    B, T, hidden, H, D = 8, 1568, 768, 12, 64
    torch.cuda.set_device(0)
    torch.manual_seed(0)
    layer = kda.GatedDeltaLayer(hidden, H, D).to(torch.bfloat16)
    layer.A_log.data = layer.A_log.data.float()
    layer.dt_bias.data = layer.dt_bias.data.float()
    layer = layer.cuda()
    layer.fused_output_norm = args.fused_norm
    gen = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(B, T, hidden, device="cuda", generator=gen).to(torch.bfloat16).requires_grad_()
    cot = torch.randn(B, T, hidden, device="cuda", generator=gen).to(torch.bfloat16)

    def step():
        out, _ = layer(x)
        out.backward(cot)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed / args.steps * 1e3

    lib = _lib.load()
    lib.kda_profile_enable(1)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    prof_ms = (time.perf_counter() - t1) / args.steps * 1e3
    lib.kda_profile_enable(0)
    lb = layer_kernel_bytes(B, T, H, D)
    kernels, kda_ms, ew_ms = [], 0.0, 0.0
    for kid in range(_lib.PROF_NKERNELS):
        tot, cnt = ctypes.c_double(), ctypes.c_int()
        _lib.check(lib.kda_profile_read(kid, ctypes.byref(tot), ctypes.byref(cnt)), "kda_profile_read")
        if cnt.value == 0:
            continue
        avg_s = tot.value / cnt.value * 1e-3
        row = {"name": lib.kda_profile_name(kid).decode(), "launches": cnt.value, "avg_us": round(avg_s * 1e6, 2)}
        if kid in LAYER_KERNELS:   # the recurrence kernels' rates are reported by the cfg2 workload
            by = lb[kid]
            row.update(gbs=round(by / avg_s / 1e9, 1), hbm_frac=round(by / avg_s / PEAK_HBM, 4), alg_bytes=by)
        kernels.append(row)
        per_step_ms = tot.value / args.steps
        if kid in LAYER_KERNELS:
            ew_ms += per_step_ms
        else:
            kda_ms += per_step_ms
    out = {
        "metric": LAYER_METRIC, "value": round(B * T * args.steps / elapsed, 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) x, random-init layer of the reference's architecture)",
        "config": {"workload": "GatedDeltaLayer fwd+bwd, x (8, 1568, 768), H12 D64, bf16 (A_log, dt_bias fp32)",
                   "B": B, "T": T, "hidden": hidden, "H": H, "D": D, "fused_output_norm": args.fused_norm},
        "profiled_ms_per_step": round(prof_ms, 4),
        "kda_ms_per_step": round(kda_ms, 4), "elementwise_ms_per_step": round(ew_ms, 4),
        "kda_share": round(kda_ms / prof_ms, 4), "elementwise_share": round(ew_ms / prof_ms, 4),
        "kernels": kernels,
    }
    print(json.dumps(out), flush=True)


MODEL_METRIC = "NoPE-GDN ViT-B train step (config 4) clips/sec @B8 16x224x224, 12 GDN blocks, bf16"


def model_bench(args):
    """Config 4: one AdamW training step (forward, label-smoothed loss,
    backward, global clip, update; train_mlx_k400.py:379-408) of the NoPE-GDN
    classifier with 12 GDN blocks of width 768 on 8 clips of 16 x 224 x 224,
    bf16 weights with A_log / dt_bias in fp32, random init, synthetic clips."""
    import ctypes
    import torch
    import mlx_vit_amd as kda
    from mlx_vit_amd import _lib
    from mlx_vit_amd import model as M
    from mlx_vit_amd import train as TR

    B = 8
    torch.cuda.set_device(0)
    torch.manual_seed(0)
    model = M.to_bf16(M.config4()).cuda()
    for mod in model.modules():
        if isinstance(mod, kda.GatedDeltaLayer):
            mod.fused_output_norm = args.fused_norm
    step = TR.TrainStep(model)
    gen = torch.Generator(device="cuda").manual_seed(0)
    video = torch.randn(B, 16, 224, 224, 3, device="cuda", generator=gen).to(torch.bfloat16)
    target = torch.randint(0, 400, (B,), device="cuda", generator=gen)
    for _ in range(args.warmup):
        step(video, target)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        loss = step(video, target)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed / args.steps * 1e3
    lib = _lib.load()
    lib.kda_profile_enable(1)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step(video, target)
    torch.cuda.synchronize()
    prof_ms = (time.perf_counter() - t1) / args.steps * 1e3
    lib.kda_profile_enable(0)
    kernels, kda_ms, ew_ms = [], 0.0, 0.0
    for kid in range(_lib.PROF_NKERNELS):
        tot, cnt = ctypes.c_double(), ctypes.c_int()
        _lib.check(lib.kda_profile_read(kid, ctypes.byref(tot), ctypes.byref(cnt)), "kda_profile_read")
        if cnt.value == 0:
            continue
        kernels.append({"name": lib.kda_profile_name(kid).decode(), "launches": cnt.value,
                        "avg_us": round(tot.value / cnt.value * 1e3, 2)})
        if kid in LAYER_KERNELS:
            ew_ms += tot.value / args.steps
        else:
            kda_ms += tot.value / args.steps
    tokens = B * 1568
    out = {
        "metric": MODEL_METRIC, "value": round(B * args.steps / elapsed, 3), "unit": "clips/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) clips, random labels; random-init weights of the reference's architecture)",
        "config": {"workload": "NoPEGDNClassifier(encoder_depth=0, processor_depth=12, gdn_ratio=12, "
                               "processor_dim=768, processor_heads=12, num_frames=16, num_classes=400), "
                               "AdamW step", "global_batch": B, "tokens_per_clip": 1568},
        "tokens_per_s": round(tokens * args.steps / elapsed, 1), "loss": round(float(loss), 4),
        "profiled_ms_per_step": round(prof_ms, 3), "kda_ms_per_step": round(kda_ms, 3),
        "layer_elementwise_ms_per_step": round(ew_ms, 3), "kda_share": round(kda_ms / prof_ms, 4),
        "layer_elementwise_share": round(ew_ms / prof_ms, 4), "kernels": kernels,
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(WORKLOADS) + ["layer", "model"], default="cfg2")
    ap.add_argument("--cpu-sample-tokens", type=int, default=392)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--fused-norm", action="store_true",
                    help="layer / model workloads: fuse the output norm into the forward recurrence's store "
                         "(kda_fwd_gated) instead of the layer's default standalone norm kernel")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="run one plain fp32 streaming kernel of this many MiB first (PMC byte-counter scale)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE output directories and exit")
    ap.add_argument("--pmc-sq", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 --pmc SQ counter output directories (per wave, per kernel) and exit")
    ap.add_argument("--pmc-mfma", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 --pmc MfmaUtil SQ_INSTS_VALU_MFMA_MOPS_BF16 output (and optionally a "
                         "second directory of SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE) and exit")
    args = ap.parse_args()
    if args.pmc_summary:
        print(json.dumps(pmc_summary(*args.pmc_summary, args.copy_calibration_mb or 512), indent=1))
        return
    if args.pmc_sq:
        print(json.dumps(pmc_sq_summary(*args.pmc_sq), indent=1))
        return
    if args.pmc_mfma:
        print(json.dumps(pmc_mfma_summary(*args.pmc_mfma[:2]), indent=1))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build runs the op on a "
              "single MI355X and reports that GPU's throughput.", file=sys.stderr)
        sys.exit(2)

    if args.workload == "layer":
        layer_bench(args)
        return
    if args.workload == "model":
        model_bench(args)
        return

    import torch
    import mlx_vit_amd as kda
    from mlx_vit_amd import _lib

    B, T, H, D, backward, with_state, desc = WORKLOADS[args.workload]
    torch.cuda.set_device(0)
    if args.copy_calibration_mb:
        copy_calibration(args.copy_calibration_mb)
    scalar = args.workload in SCALAR_DECAY
    q, k, v, g, beta, s0, do = make_inputs_gpu(B, T, H, D, with_state, layer_decay=args.workload in LAYER_DECAY,
                                               scalar_decay=scalar)
    ws = torch.empty(kda.workspace_bytes(2 if backward else 0, B, T, H, D), dtype=torch.uint8, device="cuda")

    def step():
        # a training step runs the training pair; a forward-only workload the plain forward
        if scalar:
            # chunk_gdn's path: g = log(alpha), one decay per (b, t, h), the KDA
            # pair, d alpha = dg / alpha (g is alpha here)
            from mlx_vit_amd.kda import GDN_LOG_ALPHA_MIN
            gh = torch.clamp(torch.log(g.float()), min=GDN_LOG_ALPHA_MIN)
            o, sf, _ = kda.kda_forward_train(q, k, v, gh, beta, s0, workspace=ws)
            grads = kda.kda_backward_train(q, k, v, gh, beta, s0, do, None, ws)
            grads[3].div_(g.float())
            return o
        if backward:
            o, sf, _ = kda.kda_forward_train(q, k, v, g, beta, s0, workspace=ws)
            kda.kda_backward_train(q, k, v, g, beta, s0, do, None, ws)
        else:
            o, sf = kda.kda_forward(q, k, v, g, beta, s0, workspace=ws)
        return o

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed / args.steps * 1e3
    tokens_per_s = B * T * args.steps / elapsed

    # second pass with per-kernel events
    lib = _lib.load()
    lib.kda_profile_enable(1)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    prof_ms_per_step = (time.perf_counter() - t1) / args.steps * 1e3
    lib.kda_profile_enable(0)
    import ctypes
    fl, alg, wsb = kernel_counts(B, T, H, D)
    kernels = []
    for kid in range(_lib.PROF_NKERNELS):
        tot, cnt = ctypes.c_double(), ctypes.c_int()
        _lib.check(lib.kda_profile_read(kid, ctypes.byref(tot), ctypes.byref(cnt)), "kda_profile_read")
        if cnt.value == 0:
            continue
        avg_s = tot.value / cnt.value * 1e-3
        name = lib.kda_profile_name(kid).decode()
        traffic = load_traffic(name)
        mfma_busy, mfma_hw_flops = load_mfma(name)
        kernels.append({
            "name": name, "launches": cnt.value, "avg_us": round(avg_s * 1e6, 2),
            "tflops": round(fl[kid] / avg_s / 1e12, 2), "mfma_frac": round(fl[kid] / avg_s / PEAK_BF16, 4),
            "alg_bytes": alg[kid], "alg_gbs": round(alg[kid] / avg_s / 1e9, 1),
            "hbm_frac": round(alg[kid] / avg_s / PEAK_HBM, 4),
            "ws_bytes": wsb[kid], "ws_gbs": round(wsb[kid] / avg_s / 1e9, 1),
            "pmc_bytes": traffic, "pmc_over_alg": (round(traffic / alg[kid], 3) if traffic and alg[kid] else None),
            "alg_flops": fl[kid], "_avg_s": avg_s,
            # from the committed rocprofv3 counter summary (profiles/mfma.json): the
            # MFMA pipe's busy share, and the MFMA FLOPs the hardware issued per
            # dispatch over this run's duration, as a fraction of bf16 dense peak
            "mfma_busy": mfma_busy,
            "mfma_hw_frac": (round(mfma_hw_flops / avg_s / PEAK_BF16, 4) if mfma_hw_flops else None),
        })
    # the dominant kernel (most time per step) and its roofline on the op's own bytes
    dom = max(kernels, key=lambda r: r["avg_us"] * r["launches"])
    t_mfma, t_hbm = dom["alg_flops"] / PEAK_BF16, dom["alg_bytes"] / PEAK_HBM
    if t_mfma >= t_hbm:
        rl = {"bound": "mfma", "achieved": round(dom["alg_flops"] / dom["_avg_s"] / 1e12, 3),
              "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s"}
    else:
        rl = {"bound": "hbm", "achieved": round(dom["alg_bytes"] / dom["_avg_s"] / 1e9, 2),
              "peak": PEAK_HBM / 1e9, "unit": "GB/s"}
    rl["frac"] = round(rl["achieved"] / rl["peak"], 5)
    rl["traffic"] = dom["pmc_bytes"]
    rl["kernel"] = dom["name"]
    rl["avg_us"] = dom["avg_us"]
    rl["alg_bytes"] = dom["alg_bytes"]
    rl["ws_bytes"] = dom["ws_bytes"]
    rl["traffic_over_alg"] = dom["pmc_over_alg"]
    rl["mfma_busy"] = dom["mfma_busy"]
    for r in kernels:
        r.pop("_avg_s")

    op_flops, op_bytes = op_counts(B, T, H, D, backward)
    step_s = ms_per_step * 1e-3
    out = {
        "metric": METRIC, "value": round(tokens_per_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)-derived inputs of the config's distributions, resident in HBM)",
        "config": {"workload": desc, "B": B, "T": T, "H": H, "D": D, "chunk": C,
                   "backward": backward, "initial_state": with_state, "state_dtype": "fp32"},
        "mfma_frac_op": round(op_flops / step_s / PEAK_BF16, 5),
        "hbm_frac_op": round(op_bytes / step_s / PEAK_HBM, 5),
        "roofline": rl,
        "kernels": kernels,
        "profiled_ms_per_step": round(prof_ms_per_step, 4),
    }
    if not args.no_cpu_baseline:
        cb, errs = cpu_baseline_leg(B, T, H, D, backward, with_state, None, args.cpu_sample_tokens,
                                    layer_decay=args.workload in LAYER_DECAY, scalar_decay=scalar)
        out["cpu_baseline"] = cb
        out["rel_l2"] = errs
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
