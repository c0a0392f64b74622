"""CPU checks of the model and training-step host code: structure of the
config-4 model, the tubelet embedding against torch's Conv3d, the NoPE-only
path end to end, and the loss / clip / AdamW / schedule against library
routines and closed forms."""
import math

import pytest
import torch
import torch.nn.functional as F

from mlx_vit_amd import model as M
from mlx_vit_amd import train as TR


def test_config4_structure():
    m = M.config4()
    bb = m.backbone
    assert bb.get_block_types() == ["gdn"] * 12
    assert bb.encoder.depth == 0 and bb.encoder.get_grid_dims() == {"T": 8, "H": 14, "W": 14, "total": 1568}
    layer = bb.processor_blocks[0].layer
    assert (layer.num_heads, layer.head_dim, layer.hidden_size) == (12, 64, 768)
    assert isinstance(m.head, M.TemporalPoolingHead) and m.head.fc.out_features == 400
    names = dict(m.named_parameters())
    # reference parameter names (nope_gdn_mlx.py:736-772, 4009-4342)
    for n in ("backbone.processor_blocks.0.layer.q_conv1d.weight", "backbone.processor_blocks.11.layer.A_log",
              "backbone.processor_blocks.3.layer.o_norm.weight", "backbone.encoder.tubelet_embed.projection.weight",
              "backbone.dim_proj.weight", "head.temporal_query", "head.t_proj_k.weight", "head.fc.bias"):
        assert n in names, n
    assert names["backbone.encoder.tubelet_embed.projection.weight"].shape == (384, 2, 16, 16, 3)
    M.to_bf16(m)
    for n, p in m.named_parameters():
        keep = n.endswith("A_log") or n.endswith("dt_bias")
        assert p.dtype == (torch.float32 if keep else torch.bfloat16), n


def test_tubelet_embedding_matches_conv3d():
    torch.manual_seed(0)
    emb = M.TubeletEmbedding3D(img_size=32, num_frames=4, tubelet_size=(2, 16, 16), in_channels=3, embed_dim=8)
    video = torch.randn(2, 4, 32, 32, 3)
    w = emb.projection.weight.permute(0, 4, 1, 2, 3)          # (D, C, kt, kh, kw)
    ref = F.conv3d(video.permute(0, 4, 1, 2, 3), w, emb.projection.bias, stride=(2, 16, 16))
    ref = ref.permute(0, 2, 3, 4, 1).reshape(2, -1, 8)        # (B, T'*H'*W', D), T' major
    torch.testing.assert_close(emb(video), ref, rtol=1e-5, atol=1e-5)


def test_nope_only_classifier_runs_on_cpu():
    torch.manual_seed(1)
    m = M.NoPEGDNClassifier(img_size=32, num_frames=4, encoder_dim=16, encoder_depth=1, encoder_heads=2,
                            processor_dim=32, processor_depth=2, processor_heads=4, gdn_ratio=0, num_classes=5,
                            head_type="mean")
    assert m.backbone.get_block_types() == ["nope", "nope"]
    out = m(torch.randn(3, 4, 32, 32, 3))
    assert out.shape == (3, 5) and torch.isfinite(out).all()
    m2 = M.NoPEGDNClassifier(img_size=32, num_frames=4, encoder_dim=16, encoder_depth=0, processor_dim=16,
                             processor_depth=1, processor_heads=2, gdn_ratio=0, num_classes=3)
    assert m2(torch.randn(2, 4, 32, 32, 3)).shape == (2, 3)


def test_hybrid_block_ratio():
    bb = M.NoPEGDNVideoBackbone(img_size=32, num_frames=4, encoder_dim=64, encoder_depth=0, processor_dim=64,
                                processor_depth=8, processor_heads=2, gdn_ratio=3)
    assert bb.get_block_types() == ["gdn", "gdn", "gdn", "nope"] * 2
    with pytest.raises(ValueError):
        M.HybridBlock(64, 2, block_type="mamba")


def test_cosine_warmup_lr():
    assert TR.cosine_warmup_lr(0, 100, 10, 1.0) == 0.0
    assert TR.cosine_warmup_lr(5, 100, 10, 1.0) == pytest.approx(0.5)
    assert TR.cosine_warmup_lr(10, 100, 10, 1.0) == pytest.approx(1.0)
    assert TR.cosine_warmup_lr(55, 100, 10, 1.0) == pytest.approx(0.5)
    assert TR.cosine_warmup_lr(100, 100, 10, 1.0) == pytest.approx(0.0, abs=1e-12)


def test_loss_matches_library():
    g = torch.Generator().manual_seed(2)
    logits = torch.randn(6, 11, generator=g)
    target = torch.randint(0, 11, (6,), generator=g)
    for ls in (0.0, 0.1):
        torch.testing.assert_close(TR.loss_fn(logits, target, ls),
                                   F.cross_entropy(logits, target, label_smoothing=ls))


def test_clip_matches_library():
    g = torch.Generator().manual_seed(3)
    ps = [torch.nn.Parameter(torch.randn(5, 4, generator=g)) for _ in range(3)]
    qs = [torch.nn.Parameter(p.detach().clone()) for p in ps]
    for p, q in zip(ps, qs):
        p.grad = torch.randn(p.shape, generator=g) * 3
        q.grad = p.grad.clone()
    tot = TR.clip_grads_by_norm(ps, 1.0)
    ref = torch.nn.utils.clip_grad_norm_(qs, 1.0)
    torch.testing.assert_close(tot, ref)
    for p, q in zip(ps, qs):
        torch.testing.assert_close(p.grad, q.grad)


def test_adamw_closed_form_first_step():
    """From zero moments: m = (1-b1) g, v = (1-b2) g^2 and no bias correction."""
    g = torch.Generator().manual_seed(4)
    p = torch.nn.Parameter(torch.randn(7, generator=g))
    p0 = p.detach().clone()
    grad = torch.randn(7, generator=g)
    p.grad = grad.clone()
    opt = TR.AdamW([p], lr=0.01, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.05)
    opt.step()
    expect = p0 * (1 - 0.01 * 0.05) - 0.01 * (0.1 * grad) / (math.sqrt(0.05) * grad.abs() + 1e-8)
    torch.testing.assert_close(p.detach(), expect)


def test_train_step_schedule_and_ema():
    """TrainStep sets the learning rate from cosine_warmup_lr at each global
    step before the update and moves the EMA shadow after it
    (train_mlx_k400.py:427-441).  Checked on a linear model with one fixed
    batch against a hand-run copy of the same sequence."""
    from mlx_vit_amd.checkpoint import ModelEMA, to_mlx_key
    torch.manual_seed(5)
    model = torch.nn.Linear(6, 4)
    ref = torch.nn.Linear(6, 4)
    ref.load_state_dict(model.state_dict())
    ema = ModelEMA(model, decay=0.5)
    step = TR.TrainStep(model, lr=0.1, grad_clip=0.0, label_smoothing=0.0, total_steps=8, warmup_steps=2, ema=ema,
                        step_offset=1)
    ropt = TR.AdamW(ref.parameters(), lr=0.1)
    shadow = {n: p.detach().clone() for n, p in ref.named_parameters()}
    x = torch.randn(3, 6)
    y = torch.tensor([0, 2, 3])
    for k in range(1, 5):
        step(x, y)
        ropt.lr = TR.cosine_warmup_lr(k, 8, 2, 0.1)
        ropt.zero_grad()
        TR.loss_fn(ref(x), y).backward()
        ropt.step()
        for n, p in ref.named_parameters():
            shadow[n] = 0.5 * shadow[n] + 0.5 * p.detach()
        assert step.opt.lr == pytest.approx(ropt.lr)
    assert step.global_step == 5
    for n, p in model.named_parameters():
        torch.testing.assert_close(p.detach(), dict(ref.named_parameters())[n].detach())
        torch.testing.assert_close(ema.shadow[to_mlx_key(n)], shadow[n])
    # warm-up from step 0: the first update has learning rate 0 (weights unchanged but for no decay)
    m2 = torch.nn.Linear(6, 4)
    w0 = m2.weight.detach().clone()
    TR.TrainStep(m2, lr=0.1, grad_clip=0.0, total_steps=8, warmup_steps=2)(x, y)
    torch.testing.assert_close(m2.weight.detach(), w0)
