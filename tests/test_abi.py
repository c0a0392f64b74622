"""C-ABI checks that need no GPU: the library loads, exports every function the
header declares, and rejects bad arguments before any device work."""
import ctypes
import os
import re

import pytest

from mlx_vit_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kda_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kda_\w+)\s*\(", text)))


def test_header_declares_the_abi():
    names = _declared_functions()
    for n in ("kda_fwd", "kda_bwd", "kda_workspace_size", "kda_last_error", "kda_solve_unit_triangular"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} declared in kda_hip.h but not exported"
    assert set(_declared_functions()) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_abi_version():
    assert _lib.load().kda_abi_version() == _lib.ABI_VERSION == 4


def test_workspace_sizes():
    lib = _lib.load()
    fwd = lib.kda_workspace_size(0, 8, 1568, 12, 64, 64, 1)
    bwd = lib.kda_workspace_size(1, 8, 1568, 12, 64, 64, 1)
    N = 8 * 12 * 25
    # forward: W, U, Qp, Kb (bf16; fp32: KbT) (C*D) + Aqk (C*C) in the input dtype, eG (D) in fp32
    assert fwd == 2 * (4 * N * 64 * 64 + N * 64 * 64) + 4 * N * 64
    assert lib.kda_workspace_size(0, 8, 1568, 12, 64, 64, 0) == 4 * (4 * N * 64 * 64 + N * 64 * 64) + 4 * N * 64
    # backward, bf16: W, U, Qp, Kb, dVp (C*D), h, dh (D*D), Aqk (C*C) in bf16 and
    # eG (D) in fp32; no transposed slab (the recurrences read Kb, Qp, W and Aqk
    # with transposing LDS reads)
    assert bwd == 2 * (5 * N * 64 * 64 + 2 * N * 64 * 64 + N * 64 * 64) + 4 * N * 64
    assert bwd > fwd
    # backward, fp32: also V' (C*D), Akk (C*C) and the diagonal-block inverses (4*16*16)
    bwd32 = lib.kda_workspace_size(1, 8, 1568, 12, 64, 64, 0)
    assert bwd32 == 4 * (8 * N * 64 * 64 + 2 * N * 64 * 64 + N * 64 * 64) + 4 * (N * 64 * 64 + N * 1024 + N * 64)
    # the training pair's workspace holds both passes' regions (at bf16 the
    # forward's regions are a subset of the backward's)
    train = lib.kda_workspace_size(2, 8, 1568, 12, 64, 64, 1)
    assert train == bwd
    fwd32 = lib.kda_workspace_size(0, 8, 1568, 12, 64, 64, 0)
    train32 = lib.kda_workspace_size(2, 8, 1568, 12, 64, 64, 0)
    assert train32 == fwd32 + bwd32 - 4 * (3 * N * 64 * 64) - 4 * N * 64
    assert lib.kda_workspace_size(0, 1, 0, 1, 64, 64, 1) == 0 or lib.kda_workspace_size(0, 1, 0, 1, 64, 64, 1) >= 0


def test_reference_chunk_sizes():
    """chunk is the reference's chunk_size: 8, 16, 32 and 64 are accepted and
    give the same workspace (the kernels block at 64); others are rejected."""
    lib = _lib.load()
    sizes = {c: lib.kda_workspace_size(2, 2, 300, 3, 64, c, 1) for c in (8, 16, 32, 64)}
    assert len(set(sizes.values())) == 1 and sizes[64] > 0
    assert lib.kda_workspace_size(2, 2, 300, 3, 64, 48, 1) == 0
    assert "chunk" in _lib.last_error()


@pytest.mark.parametrize("B,T,H,D", [(8, 1568, 12, 64), (1, 1, 3, 64), (2, 300, 4, 64), (1, 70, 16, 128),
                                     (4, 65, 12, 64)])
def test_layer_workspace_sizes(B, T, H, D):
    """The backward workspaces hold one partial-sum row per workgroup (32 tokens
    of one batch row for the producer, 8 rows for the norm), the summed row,
    and 1 to 64 rows of slice sums; every row is H*D values per parameter
    gradient (17 for the producer), fp32."""
    lib = _lib.load()
    HD = H * D
    for which, rows, vals in ((_lib.KDA_LAYER_PRODUCER, B * -(-T // 32), 17),
                              (_lib.KDA_LAYER_RMSNORM, -(-(B * T) // 8), 1)):
        got = lib.kda_layer_workspace_size(which, B, T, H, D)
        row = 4 * vals * HD
        assert got % row == 0
        assert (rows + 2) * row <= got <= (rows + 1 + 64) * row, (which, got, rows)
    assert lib.kda_layer_workspace_size(7, B, T, H, D) == 0


def test_workspace_offsets_disjoint():
    lib = _lib.load()
    for pass_, shape in ((0, (2, 300, 3, 64)), (1, (2, 300, 3, 64)), (2, (2, 300, 3, 64)),
                         (0, (1, 2000, 2, 128)), (0, (1, 32768, 16, 128)), (0, (2, 1568, 8, 96)),
                         (1, (2, 1568, 8, 96)), (2, (1, 70, 3, 96))):
        arr = (ctypes.c_int64 * len(_lib.WS_REGIONS))()
        assert lib.kda_workspace_offsets(pass_, *shape, 64, 1, arr) == 0
        offs = sorted(o for o in arr if o >= 0)
        assert offs[0] == 0 and all(b - a >= 256 and b % 256 == 0 for a, b in zip(offs, offs[1:]))
        total = lib.kda_workspace_size(pass_, *shape, 64, 1)
        assert offs[-1] < total


def _offsets(lib, pass_, B, T, H, D, dtype):
    arr = (ctypes.c_int64 * len(_lib.WS_REGIONS))()
    assert lib.kda_workspace_offsets(pass_, B, T, H, D, 64, dtype, arr) == 0
    return dict(zip(_lib.WS_REGIONS, arr))


BACKWARD_REGIONS = ("h", "dh", "Vp", "dVp", "SegX", "SegM", "SegS", "PadB")


@pytest.mark.parametrize("pass_,dtype", [(0, 0), (0, 1), (1, 0), (1, 1), (2, 0), (2, 1)])
def test_d96_workspace_is_d128_plus_pad(pass_, dtype):
    """D = 96 runs the D = 128 kernels (the prep and the local adjoints read and
    write 96-channel rows themselves): its regions are those of D = 128 plus
    PAD (the padded s0 and the forward's padded o and s_final) and PADB (the
    backward's padded dout, ds_final and ds0).  Passes 0 and 1: the D = 128
    regions at their offsets, then PAD, then PADB.  Pass 2: the kept regions at
    their D = 128 offsets and PAD after them; the backward's regions follow,
    shifted by PAD, and PADB last."""
    lib = _lib.load()
    B, T, H = 2, 300, 3
    o96, o128 = _offsets(lib, pass_, B, T, H, 96, dtype), _offsets(lib, pass_, B, T, H, 128, dtype)
    assert o128["Pad"] == -1 and o128["PadB"] == -1
    s128 = lib.kda_workspace_size(pass_, B, T, H, 128, 64, dtype)
    tok, es, st = B * T * H * 128, 2 if dtype else 4, B * H * 128 * 128 * 4
    # PAD: s0, and o (es), s_final for the forward passes; PADB: dout (es),
    # ds_final, ds0 for the backward ones
    pad = st + ((tok * es + st) if pass_ != 1 else 0)
    padb = (tok * es + 2 * st) if pass_ != 0 else 0
    assert lib.kda_workspace_size(pass_, B, T, H, 96, 64, dtype) - s128 == pad + padb
    kernel_regions = [r for r in _lib.WS_REGIONS if r not in ("Pad", "PadB")]
    if pass_ != 2:
        assert all(o96[r] == o128[r] for r in kernel_regions)
        assert o96["Pad"] == s128
        assert o96["PadB"] == (s128 + pad if pass_ == 1 else -1)
        return
    kept128 = lib.kda_train_kept_size(B, T, H, 128, 64, dtype)
    assert lib.kda_train_kept_size(B, T, H, 96, 64, dtype) == kept128 + pad
    assert o96["Pad"] == kept128
    for r in kernel_regions:
        assert o96[r] == (o128[r] + pad if r in BACKWARD_REGIONS and o128[r] >= 0 else o128[r]), r
    assert o96["PadB"] == s128 + pad


@pytest.mark.parametrize("B,T,H,D,dtype", [(2, 300, 3, 64, 1), (2, 300, 3, 64, 0), (1, 200, 2, 128, 1),
                                           (1, 200, 2, 128, 0), (2, 70, 3, 96, 1), (1, 65, 2, 32, 0)])
def test_train_workspace_kept_part_first(B, T, H, D, dtype):
    """The training pair's workspace: the regions the forward writes and the
    backward reads come first (kda_train_kept_size bytes), the backward's own
    regions (h, dh, V', dV', the padded gradients) after them."""
    lib = _lib.load()
    off = _offsets(lib, 2, B, T, H, D, dtype)
    kept = lib.kda_train_kept_size(B, T, H, D, 64, dtype)
    total = lib.kda_workspace_size(2, B, T, H, D, 64, dtype)
    assert 0 < kept < total and kept % 256 == 0
    for r, o in off.items():
        if o < 0:
            continue
        assert (o >= kept) == (r in BACKWARD_REGIONS), (r, o, kept)
    assert all(off[r] >= 0 for r in ("W", "U", "eG", "h", "dh", "dVp"))
    # the forward passes' layouts are unchanged by the split
    assert lib.kda_train_kept_size(B, T, H, 48, 64, dtype) == 0 and b"D=48" in lib.kda_last_error()


@pytest.mark.parametrize("B,T,H,D,dtype,nseg", [
    (1, 32768, 16, 128, 1, 16),   # config 3: 16 (b, h) x 16 segments of 32 chunks
    (1, 2000, 2, 128, 1, 8),      # 32 chunks: segments of at least 4 chunks
    (2, 600, 3, 128, 1, 1),       # 2 segments of 5 chunks: one chain per (b, h)
    (2, 2500, 3, 128, 1, 10),
    (5, 12288, 8, 128, 1, 6),     # 6 segments of 32 chunks: the forward only
    (1, 129, 2, 128, 1, 1),       # 3 chunks: one segment, the unsegmented kernel
    (16, 1024, 16, 128, 1, 1),    # 256 (b, h) fill the GPU by themselves
    (1, 32768, 16, 128, 0, 1),    # fp32 inputs: not segmented
    (1, 32768, 16, 64, 1, 1),     # D = 64: not segmented
])
def test_segment_plan_regions(B, T, H, D, dtype, nseg):
    """The bf16 forward at D = 128 is split into segments when the plan (about
    256 workgroups, >= 4 chunks per segment) gives at least 8 segments or
    segments of at least 32 chunks; the three segment regions are then
    B*H*nseg*D*D fp32 each.  The backward's state
    recompute follows the same plan where it gives at least 8 segments: passes
    1 and 2 then hold the same three regions (in pass 2 among the backward's
    own, after the kept part)."""
    lib = _lib.load()
    seg = ("SegX", "SegM", "SegS")
    per = B * H * nseg * D * D * 4
    for pass_ in (0, 1, 2):
        off = _offsets(lib, pass_, B, T, H, D, dtype)
        if nseg == 1 or (pass_ != 0 and nseg < 8):   # the backward: from 8 segments
            assert all(off[r] == -1 for r in seg), pass_
            continue
        for a, b in zip(seg, seg[1:]):
            assert off[b] - off[a] == per, pass_
        if pass_ == 0:
            assert lib.kda_workspace_size(0, B, T, H, D, 64, dtype) - off["SegS"] == per
        if pass_ == 2:
            assert off["SegX"] >= lib.kda_train_kept_size(B, T, H, D, 64, dtype)


@pytest.mark.parametrize("B,T,H,D,chunk,dtype,gdt,code", [
    (1, 64, 1, 64, 48, 1, 1, _lib.KDA_E_UNSUPPORTED),    # chunk
    (1, 64, 1, 48, 64, 1, 1, _lib.KDA_E_UNSUPPORTED),    # head dim
    (1, 64, 1, 64, 64, 2, 1, _lib.KDA_E_UNSUPPORTED),    # dtype
    (1, 64, 1, 64, 64, 1, 5, _lib.KDA_E_UNSUPPORTED),    # g dtype
    (1, 64, 1, 64, 64, 0, 2, _lib.KDA_E_UNSUPPORTED),    # one decay per head: bf16 operands only
    (1, 64, 1, 128, 64, 1, 2, _lib.KDA_E_UNSUPPORTED),   # ... and D in {32, 64}
    (1, 64, 1, 96, 64, 1, 2, _lib.KDA_E_UNSUPPORTED),
    (-1, 64, 1, 64, 64, 1, 1, _lib.KDA_E_INVALID),       # negative size
])
def test_fwd_argument_errors(B, T, H, D, chunk, dtype, gdt, code):
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    rc = lib.kda_fwd(fake, fake, fake, fake, fake, None, fake, None, B, T, H, D, chunk, dtype, gdt,
                     fake, 1 << 40, None)
    assert rc == code
    assert _lib.last_error()


def test_null_and_workspace_errors():
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    rc = lib.kda_fwd(None, fake, fake, fake, fake, None, fake, None, 1, 64, 1, 64, 64, 1, 1, fake, 1 << 40, None)
    assert rc == _lib.KDA_E_INVALID and "q" in _lib.last_error()
    rc = lib.kda_fwd(fake, fake, fake, fake, fake, None, fake, None, 1, 64, 1, 64, 64, 1, 1, fake, 16, None)
    assert rc == _lib.KDA_E_WORKSPACE
    misaligned = ctypes.c_void_p((1 << 20) + 4)
    rc = lib.kda_fwd(misaligned, fake, fake, fake, fake, None, fake, None, 1, 64, 1, 64, 64, 1, 1, fake,
                     1 << 40, None)
    assert rc == _lib.KDA_E_INVALID
    # the backward supports D in {32, 64, 96, 128}
    rc = lib.kda_bwd(*([fake] * 14), 1, 64, 1, 80, 64, 1, 1, fake, 1 << 40, None)
    assert rc == _lib.KDA_E_UNSUPPORTED and "backward" in _lib.last_error()


def test_training_pair_argument_errors():
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    # training needs a backward-capable head dim and dtype, and the pass-2 workspace
    rc = lib.kda_fwd_train(fake, fake, fake, fake, fake, None, fake, None, 1, 64, 1, 80, 64, 0, 0,
                           fake, 1 << 40, None)
    assert rc == _lib.KDA_E_UNSUPPORTED
    need = lib.kda_workspace_size(2, 1, 64, 1, 64, 64, 1)
    kept = lib.kda_train_kept_size(1, 64, 1, 64, 64, 1)
    assert need > kept >= lib.kda_workspace_size(0, 1, 64, 1, 64, 64, 1)
    # the forward needs the kept part, the single-buffer backward all of it
    rc = lib.kda_fwd_train(fake, fake, fake, fake, fake, None, fake, None, 1, 64, 1, 64, 64, 1, 1,
                           fake, kept - 1, None)
    assert rc == _lib.KDA_E_WORKSPACE
    rc = lib.kda_bwd_train(*([fake] * 14), 1, 64, 1, 64, 64, 1, 1, fake, need - 1, None)
    assert rc == _lib.KDA_E_WORKSPACE
    # the split backward: the kept part and a scratch buffer of the rest
    rc = lib.kda_bwd_train_split(*([fake] * 14), 1, 64, 1, 64, 64, 1, 1, fake, kept - 1, fake, need - kept, None)
    assert rc == _lib.KDA_E_WORKSPACE and "workspace" in _lib.last_error()
    rc = lib.kda_bwd_train_split(*([fake] * 14), 1, 64, 1, 64, 64, 1, 1, fake, kept, fake, need - kept - 1, None)
    assert rc == _lib.KDA_E_WORKSPACE and "scratch" in _lib.last_error()
    rc = lib.kda_bwd_train_split(*([fake] * 14), 1, 64, 1, 64, 64, 1, 1, fake, kept, None, need - kept, None)
    assert rc == _lib.KDA_E_WORKSPACE and "scratch" in _lib.last_error()
    misaligned = ctypes.c_void_p((1 << 20) + 16)
    rc = lib.kda_bwd_train_split(*([fake] * 14), 1, 64, 1, 64, 64, 1, 1, fake, kept, misaligned, need, None)
    assert rc == _lib.KDA_E_INVALID and "scratch" in _lib.last_error()
    assert lib.kda_workspace_size(3, 1, 64, 1, 64, 64, 1) == 0


def test_solve_argument_errors():
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    assert lib.kda_solve_unit_triangular(fake, fake, fake, 1, 65, 4, 0, None) == _lib.KDA_E_UNSUPPORTED
    assert lib.kda_solve_unit_triangular(None, fake, fake, 1, 8, 4, 0, None) == _lib.KDA_E_INVALID


def test_error_mapping():
    with pytest.raises(ValueError):
        _lib.check(_lib.KDA_E_UNSUPPORTED, "x")
    with pytest.raises(_lib.KDAError):
        _lib.check(_lib.KDA_E_HIP, "x")
    _lib.check(_lib.KDA_OK, "x")


def test_profile_names():
    lib = _lib.load()
    names = [lib.kda_profile_name(i).decode() for i in range(_lib.PROF_NKERNELS)]
    assert all(names) and len(set(names)) == len(names)
    assert lib.kda_profile_name(99).decode() == ""
