"""Host-side behaviour of the torch front end (no GPU needed): path validation
and dispatch mirroring the reference's compute_path checks, argument errors,
and the rule that the product never routes through the oracle."""
import os
import re

import pytest
import torch

import mlx_vit_amd as kda

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_default_path_is_hip():
    rec = kda.KDARecurrence(num_heads=12, head_dim=64)
    assert rec.compute_path == "hip_chunkwise_kda"


@pytest.mark.parametrize("kwargs,msg", [
    (dict(compute_path="metal_sg"), "Unknown compute_path"),
    (dict(chunk_size=48), "chunk_size"),
    (dict(channel_wise_decay=False, compute_path="hip_chunkwise_kda"), "channel-wise"),
    (dict(channel_wise_decay=True, compute_path="hip_chunkwise_gdn"), "scalar-alpha"),
    (dict(head_dim=80), "head_dim"),
    (dict(head_dim=48, requires_grad=False), "head_dim"),
])
def test_construction_errors(kwargs, msg):
    args = dict(num_heads=2, head_dim=64)
    args.update(kwargs)
    with pytest.raises(ValueError, match=msg):
        kda.KDARecurrence(**args)


@pytest.mark.parametrize("c", [8, 16, 32, 64])
def test_reference_chunk_sizes_accepted(c):
    # the reference's chunk sizes; the result does not depend on the blocking
    assert kda.KDARecurrence(num_heads=2, head_dim=64, chunk_size=c).chunk_size == c


@pytest.mark.parametrize("D", [96, 128])
def test_head_dims_96_and_128_for_inference_and_training(D):
    assert kda.KDARecurrence(num_heads=16, head_dim=D, requires_grad=False).head_dim == D
    assert kda.KDARecurrence(num_heads=16, head_dim=D).head_dim == D


def test_ssv2_layer_constructs():
    """The reference's SSv2 layer (train_mlx_ssv2.py:71-80): 8 heads of 96."""
    from mlx_vit_amd import GatedDeltaLayer
    layer = GatedDeltaLayer(768, 8, 96)
    assert layer.head_dim == 96 and layer.total_dim == 768 and layer.recurrence.requires_grad


def test_layer_rejects_too_many_norm_lanes():
    """The output norm gives a head of 96 channels 32 lanes: 17 such heads
    would need more than the kernel's 8 waves."""
    from mlx_vit_amd import GatedDeltaLayer
    with pytest.raises(ValueError, match="output norm"):
        GatedDeltaLayer(17 * 96, 17, 96)


def test_unknown_path_at_call():
    rec = kda.KDARecurrence(num_heads=1, head_dim=64)
    x = torch.zeros(1, 4, 1, 64)
    with pytest.raises(ValueError, match="Unknown compute_path"):
        rec(x, x, x, x, torch.zeros(1, 4, 1), compute_path="compiled")


def test_cpu_tensors_are_rejected_not_computed():
    """No CPU fallback: the op refuses host tensors."""
    x = torch.zeros(1, 8, 1, 64)
    with pytest.raises(ValueError, match="ROCm device"):
        kda.kda_forward(x, x, x, x, torch.zeros(1, 8, 1))


@pytest.mark.parametrize("bad", ["k", "beta", "state"])
def test_shape_errors(bad):
    x = torch.zeros(1, 8, 2, 64)
    k = torch.zeros(1, 8, 2, 32) if bad == "k" else x
    beta = torch.zeros(1, 8, 3) if bad == "beta" else torch.zeros(1, 8, 2)
    st = torch.zeros(1, 2, 64, 32) if bad == "state" else None
    with pytest.raises(ValueError):
        kda.kda_forward(x, k, x, x, beta, st)


def test_unsupported_dtype():
    x = torch.zeros(1, 8, 1, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="dtype"):
        kda.kda_forward(x, x, x, x, torch.zeros(1, 8, 1, dtype=torch.float16))


def test_product_never_imports_the_oracle():
    pkg = os.path.join(ROOT, "mlx_vit_amd")
    for dirpath, _, files in os.walk(pkg):
        for fn in files:
            if fn.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, fn)).read()
                assert not re.search(r"\boracle\b", text), f"{fn} references the oracle"
