"""GPU checks of the NoPE + GDN classifier and its training step.

Parity: a small hybrid classifier (encoder block, three GDN blocks, one NoPE
block, temporal head) in fp32 on the GPU against an fp64 CPU copy whose GDN
layers run the CPU restatement of the layer (oracle/layer_reference.py): loss
and every parameter gradient within rel-L2 1e-4, except the decay-gate
parameters (2e-3, for the reason given at ``DECAY_GATE``).  Training: the config-4 model
in bf16 takes optimisation steps with finite losses and changing weights, and
a small model overfits one batch."""
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
    bad = {k: v for k, v in errs.items() if not (v <= _tol(k))}
    assert not bad, bad


# The gradients of the decay-gate parameters are sums over every token of dg
# (times g or sigmoid terms).  Heads whose per-step decay exceeds the anchored
# path's span guard (here A = e^{A_log} of 9 to 14, g of -6 to -10 per step)
# take the pairwise path, where the in-chunk cumulative log-decay reaches ~600
# and exp(gamma_t - gamma_s) formed from two fp32 cumsums carries a relative
# error of about |gamma| 2^-24 ~ 4e-5 that is coherent across a chunk.  The op's
# own dg stays <= 1.4e-5 at such decays (test_bwd_dg_pairwise_strong_decay);
# summed over 160 tokens these four gradients reach ~7e-4.
DECAY_GATE = ("A_log", "dt_bias", "f_proj_1", "f_proj_2")


def _tol(name):
    return 2e-3 if any(s in name for s in DECAY_GATE) else 1e-4


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
    with A_log / dt_bias in fp32: two optimisation steps on a batch of 2 clips."""
    from mlx_vit_amd import model as M
    from mlx_vit_amd import train as TR
    torch.manual_seed(4)
    model = M.to_bf16(M.config4()).to(DEV)
    before = model.backbone.processor_blocks[5].layer.q_proj.weight.detach().clone()
    a_before = model.backbone.processor_blocks[5].layer.A_log.detach().clone()
    step = TR.TrainStep(model)
    g = torch.Generator(device=DEV).manual_seed(5)
    video = torch.randn(2, 16, 224, 224, 3, device=DEV, generator=g).to(torch.bfloat16)
    target = torch.tensor([7, 123], device=DEV)
    losses = [step(video, target).item() for _ in range(2)]
    print("config4 losses", losses, flush=True)
    assert all(torch.isfinite(torch.tensor(losses)))
    assert abs(losses[0] - torch.log(torch.tensor(400.0)).item()) < 1.0
    blk = model.backbone.processor_blocks[5].layer
    assert not torch.equal(blk.q_proj.weight, before)
    assert blk.A_log.dtype == torch.float32 and not torch.equal(blk.A_log, a_before)
    for n, p in model.named_parameters():
        assert torch.isfinite(p).all(), n
