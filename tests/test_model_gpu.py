"""GPU checks of the NoPE + GDN classifier and its training step.

Parity: a small hybrid classifier (encoder block, three GDN blocks, one NoPE
block, temporal head) in fp32 on the GPU against an fp64 CPU copy whose GDN
layers run the CPU restatement of the layer (oracle/layer_reference.py): loss
and every parameter gradient within rel-L2 1e-4.  The layer's own decay
initialisation (A = e^{A_log} in [1, 16]) puts heads at -2 to -10 per step,
where the decay-gate gradients (A_log, dt_bias, f_proj) are the most
ill-conditioned sums in the model.  Training: the config-4 model (batch 8 of
16x224x224 clips) in bf16 takes optimisation steps with finite losses,
changing weights, the cosine schedule and the EMA, and a small model overfits
one batch."""
import copy
import types

import pytest
import torch

from oracle import kda_reference as R
from oracle import layer_reference as LR

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _oracle_gdn(model):
    """Route every GatedDeltaLayer of a CPU model copy through the restatement."""
    from mlx_vit_amd.layer import GatedDeltaLayer

    def fwd(self, x, state=None, compute_path=None):
        params = dict(self.named_parameters())
        return LR.layer_forward(params, x, self.num_heads, self.head_dim, state,
                                allow_neg_eigval=self.allow_neg_eigval, eps=self.o_norm.eps)

    for mod in model.modules():
        if isinstance(mod, GatedDeltaLayer):
            mod.forward = types.MethodType(fwd, mod)
    return model


def _small(num_classes=7):
    from mlx_vit_amd import model as M
    return M.NoPEGDNClassifier(img_size=64, num_frames=10, encoder_dim=32, encoder_depth=1, encoder_heads=2,
                               processor_dim=64, processor_depth=4, processor_heads=2, gdn_ratio=3,
                               num_classes=num_classes)


def test_classifier_parity_fp32():
    from mlx_vit_amd import train as TR
    torch.manual_seed(0)
    model = _small()
    print("classifier parity: blocks", model.backbone.get_block_types(), flush=True)
    ref = _oracle_gdn(copy.deepcopy(model).double())
    model = model.to(DEV)
    g = torch.Generator().manual_seed(1)
    video = torch.randn(2, 10, 64, 64, 3, generator=g)
    target = torch.tensor([3, 5])
    loss = TR.loss_fn(model(video.to(DEV)), target.to(DEV), 0.1)
    loss.backward()
    rloss = TR.loss_fn(ref(video.double()), target, 0.1)
    rloss.backward()
    errs = {"loss": abs(loss.item() - rloss.item()) / abs(rloss.item())}
    rp = dict(ref.named_parameters())
    for n, p in model.named_parameters():
        errs[n] = R.rel_l2(p.grad.cpu().double(), rp[n].grad)
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:6]
    print("classifier parity worst", {k: f"{v:.2e}" for k, v in worst}, flush=True)
    bad = {k: v for k, v in errs.items() if not (v <= 1e-4)}
    assert not bad, bad


def test_small_model_overfits_one_batch():
    from mlx_vit_amd import model as M
    from mlx_vit_amd import train as TR
    torch.manual_seed(2)
    model = M.to_bf16(_small(num_classes=4)).to(DEV)
    step = TR.TrainStep(model, lr=2e-3, grad_clip=1.0, label_smoothing=0.1)
    g = torch.Generator(device=DEV).manual_seed(3)
    video = torch.randn(4, 10, 64, 64, 3, device=DEV, generator=g).to(torch.bfloat16)
    target = torch.tensor([0, 1, 2, 3], device=DEV)
    losses = [step(video, target).item() for _ in range(12)]
    print("overfit losses", [f"{x:.3f}" for x in losses], flush=True)
    assert all(torch.isfinite(torch.tensor(losses)))
    assert losses[-1] < 0.7 * losses[0]


def test_config4_train_steps_bf16():
    """The config-4 model (12 GDN blocks, 768 wide, 1568 tokens per clip) in bf16
    with A_log / dt_bias in fp32: two optimisation steps on a batch of 8 clips
    (the stated configuration), with the warm-up schedule and the EMA."""
    from mlx_vit_amd import checkpoint as CK
    from mlx_vit_amd import model as M
    from mlx_vit_amd import train as TR
    torch.manual_seed(4)
    model = M.to_bf16(M.config4()).to(DEV)
    blk = model.backbone.processor_blocks[5].layer
    before = blk.q_proj.weight.detach().clone()
    a_before = blk.A_log.detach().clone()
    ema = CK.ModelEMA(model, decay=0.9)
    step = TR.TrainStep(model, lr=3e-4, total_steps=100, warmup_steps=5, ema=ema, step_offset=1)
    g = torch.Generator(device=DEV).manual_seed(5)
    video = torch.randn(8, 16, 224, 224, 3, device=DEV, generator=g).to(torch.bfloat16)
    target = torch.randint(0, 400, (8,), device=DEV, generator=g)
    losses = [step(video, target).item() for _ in range(2)]
    print("config4 B=8 losses", losses, "lr", step.opt.lr, flush=True)
    assert all(torch.isfinite(torch.tensor(losses)))
    assert abs(losses[0] - torch.log(torch.tensor(400.0)).item()) < 1.0
    assert step.opt.lr == TR.cosine_warmup_lr(2, 100, 5, 3e-4)
    assert not torch.equal(blk.q_proj.weight, before)
    assert blk.A_log.dtype == torch.float32 and not torch.equal(blk.A_log, a_before)
    key = CK.to_mlx_key("backbone.processor_blocks.5.layer.A_log")
    # after two updates the shadow sits strictly between the start and the weights
    assert not torch.equal(ema.shadow[key], a_before) and not torch.equal(ema.shadow[key], blk.A_log.detach())
    for n, p in model.named_parameters():
        assert torch.isfinite(p).all(), n
