"""CPU checks of the checkpoint format and converters (mlx_vit_amd/checkpoint.py)."""
import json

import pytest
import torch
from safetensors.torch import load_file

from mlx_vit_amd import checkpoint as CK
from mlx_vit_amd import model as M


def _small(seed=0, **kw):
    torch.manual_seed(seed)
    args = dict(img_size=32, num_frames=4, encoder_dim=32, encoder_depth=1, encoder_heads=2, processor_dim=64,
                processor_depth=4, processor_heads=2, gdn_ratio=3, num_classes=5)
    args.update(kw)
    return M.NoPEGDNClassifier(**args)


def test_key_maps():
    assert CK.to_mlx_key("backbone.processor_blocks.0.mlp.3.weight") == \
        "backbone.processor_blocks.0.mlp.layers.3.weight"
    assert CK.from_mlx_key("backbone.encoder.blocks.0.mlp.layers.0.bias") == "backbone.encoder.blocks.0.mlp.0.bias"
    assert CK.pt_key("backbone.processor_blocks.1.layer.f_proj.1.weight") == \
        "backbone.processor_blocks.1.layer.f_proj_2.weight"
    assert CK.pt_key("backbone.processor_blocks.1.layer.g_proj.0.weight") == \
        "backbone.processor_blocks.1.layer.g_proj_1.weight"


def test_save_load_round_trip(tmp_path):
    a = M.to_bf16(_small(0))
    ema = CK.ModelEMA(a, decay=0.9)
    with torch.no_grad():
        for p in a.parameters():
            p.add_(0.5)
    ema.update(a)
    path = tmp_path / "ck" / "model.safetensors"
    n = CK.save_checkpoint(path, a, ema, epoch=3, best_acc=0.42)
    raw = load_file(str(path))
    assert n == len(raw)
    assert "backbone.processor_blocks.0.mlp.layers.0.weight" in raw          # MLX paths in the file
    assert any(k.startswith("__ema__backbone.") for k in raw)
    assert raw["backbone.processor_blocks.0.layer.A_log"].dtype == torch.float32
    assert raw["backbone.processor_blocks.0.layer.q_proj.weight"].dtype == torch.bfloat16
    meta = json.load(open(tmp_path / "ck" / "model.meta.json"))
    assert meta == {"epoch": 3, "best_acc": 0.42, "ema_decay": 0.9}
    b = M.to_bf16(_small(1))
    ema_b = CK.ModelEMA(b, decay=0.5)
    rep = CK.load_checkpoint(path, b, ema_b)
    assert rep["missing"] == [] and rep["unexpected"] == [] and rep["ema_loaded"] == len(ema.shadow)
    for (n1, p1), (n2, p2) in zip(a.named_parameters(), b.named_parameters()):
        assert n1 == n2 and torch.equal(p1, p2), n1
    for k in ema.shadow:
        assert torch.equal(ema.shadow[k], ema_b.shadow[k]), k
    # the EMA moved a tenth of the way towards the shifted weights
    k = "backbone.processor_blocks.0.layer.dt_bias"
    torch.testing.assert_close(ema.shadow[k], a.state_dict()[CK.from_mlx_key(k)] - 0.45)


def test_load_warns_on_missing(tmp_path):
    a = _small(0)
    path = tmp_path / "m.safetensors"
    CK.save_checkpoint(path, a)
    c = _small(0, processor_depth=5)         # one more block -> its keys are missing
    with pytest.warns(UserWarning, match="missing"):
        rep = CK.load_checkpoint(path, c)
    assert any(k.startswith("backbone.processor_blocks.4.") for k in rep["missing"])


def test_pytorch_state_dict_conversion():
    """A PyTorch-era state dict (f_proj.N / g_proj.N Sequentials, channels-first
    Conv3d, (C, 1, K) Conv1d) loads into the same weights."""
    src = _small(2)
    pt = {}
    for n, p in src.state_dict().items():
        k = n
        for a_, b_ in (("f_proj_1", "f_proj.0"), ("f_proj_2", "f_proj.1"), ("g_proj_1", "g_proj.0"),
                       ("g_proj_2", "g_proj.1")):
            k = k.replace("." + a_ + ".", "." + b_ + ".")
        t = p.clone()
        if n.endswith("tubelet_embed.projection.weight"):
            t = t.permute(0, 4, 1, 2, 3).contiguous()
        elif n.endswith(("q_conv1d.weight", "k_conv1d.weight", "v_conv1d.weight")):
            t = t.permute(0, 2, 1).contiguous()
        pt[k] = t
    dst = _small(3)
    rep = CK.load_pytorch_state_dict(dst, pt, strict=True)
    assert len(rep["loaded"]) == len(pt) and not rep["unused"]
    for (n1, p1), (n2, p2) in zip(src.named_parameters(), dst.named_parameters()):
        assert torch.equal(p1, p2), n1
    pt["backbone.processor_blocks.0.layer.q_proj.weight"] = torch.zeros(3, 3)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        CK.load_pytorch_state_dict(_small(4), pt, strict=True)
    rep = CK.load_pytorch_state_dict(_small(4), dict(pt, extra=torch.zeros(1)), strict=False)
    assert "extra" in rep["no_target"] and rep["shape_mismatch"]
