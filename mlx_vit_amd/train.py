"""Training step of the reference trainer (train_mlx_k400.py) in torch.

* ``cosine_warmup_lr`` -- linear warm-up then cosine decay (train_mlx_k400.py:229-234);
* ``loss_fn`` -- cross entropy on fp32 logits with label smoothing
  (train_mlx_k400.py:255-266): (1 - ls) * nll + ls * mean(-log_softmax);
* ``clip_grads_by_norm`` -- global-norm clipping, scale = min(max_norm /
  (||g|| + 1e-6), 1) (train_mlx_k400.py:241-252);
* ``AdamW`` -- MLX's AdamW update, which has no bias correction by default:
  p <- p (1 - lr wd); m <- b1 m + (1 - b1) g; v <- b2 v + (1 - b2) g^2;
  p <- p - lr m / (sqrt(v) + eps), with the moments in the parameter's dtype
  (train_mlx_k400.py:548-549: betas (0.9, 0.95), weight decay 0.05);
* ``TrainStep`` -- the per-step body of the reference's epoch loop
  (train_mlx_k400.py:379-408, 417-441): learning rate from
  ``cosine_warmup_lr`` at the global step (when a schedule is given), forward,
  loss, backward, clip, update, then the EMA update (when an EMA is given).
"""
from __future__ import annotations

import math
from typing import Iterable, List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F


def cosine_warmup_lr(step: int, total_steps: int, warmup_steps: int, base_lr: float) -> float:
    if step < warmup_steps:
        return base_lr * step / max(1, warmup_steps)
    progress = (step - warmup_steps) / max(1, total_steps - warmup_steps)
    return 0.5 * base_lr * (1 + math.cos(math.pi * progress))


def loss_fn(logits: torch.Tensor, target: torch.Tensor, label_smoothing: float = 0.0) -> torch.Tensor:
    logits = logits.float()
    if label_smoothing > 0:
        logp = F.log_softmax(logits, dim=-1)
        nll = -logp.gather(-1, target[:, None]).squeeze(-1)
        smooth = -logp.mean(dim=-1)
        return ((1 - label_smoothing) * nll + label_smoothing * smooth).mean()
    return F.cross_entropy(logits, target)


@torch.no_grad()
def clip_grads_by_norm(params: Iterable[torch.Tensor], max_norm: float) -> torch.Tensor:
    """Scale every gradient by min(max_norm / (total_norm + 1e-6), 1); returns
    the total norm (fp32)."""
    grads = [p.grad for p in params if p.grad is not None]
    if not grads:
        return torch.zeros(())
    by_dtype = {}
    for g in grads:
        by_dtype.setdefault(g.dtype, []).append(g)
    # per-tensor norms accumulated in fp32 straight from each dtype group (no
    # fp32 copy of every gradient: one cast launch per parameter was 3% of the
    # config-4 step)
    norms = [n for gs in by_dtype.values() for n in torch._foreach_norm(gs, 2, dtype=torch.float32)]
    total = torch.linalg.vector_norm(torch.stack(norms))
    scale = torch.clamp(max_norm / (total + 1e-6), max=1.0)
    for dt, gs in by_dtype.items():
        torch._foreach_mul_(gs, scale.to(dt))
    return total


class AdamW:
    """MLX's AdamW (no bias correction), moments in the parameter dtype."""

    def __init__(self, params: Iterable[nn.Parameter], lr: float = 3e-4, betas=(0.9, 0.95), eps: float = 1e-8,
                 weight_decay: float = 0.05):
        self.params: List[nn.Parameter] = [p for p in params if p.requires_grad]
        self.lr, self.betas, self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self.m = [torch.zeros_like(p) for p in self.params]
        self.v = [torch.zeros_like(p) for p in self.params]

    @torch.no_grad()
    def step(self) -> None:
        """One update over every parameter with a gradient, as multi-tensor
        (``torch._foreach_*``) ops grouped by dtype: a handful of launches per
        step instead of several per parameter."""
        b1, b2 = self.betas
        lr, wd = self.lr, self.weight_decay
        groups = {}
        for p, m, v in zip(self.params, self.m, self.v):
            if p.grad is not None:
                groups.setdefault((p.dtype, p.device), []).append((p, m, v))
        for items in groups.values():
            ps, ms, vs = (list(t) for t in zip(*items))
            gs = [p.grad for p in ps]
            torch._foreach_mul_(ps, 1 - lr * wd)
            torch._foreach_mul_(ms, b1)
            torch._foreach_add_(ms, gs, alpha=1 - b1)
            torch._foreach_mul_(vs, b2)
            torch._foreach_addcmul_(vs, gs, gs, value=1 - b2)
            denom = torch._foreach_sqrt(vs)
            torch._foreach_add_(denom, self.eps)
            torch._foreach_addcdiv_(ps, ms, denom, value=-lr)

    def zero_grad(self) -> None:
        for p in self.params:
            p.grad = None


class TrainStep:
    """One optimisation step: learning rate, forward, label-smoothed loss,
    backward, global clip, AdamW update, EMA update.  Returns the loss (a 0-d
    fp32 tensor).

    With ``total_steps`` set, the learning rate of step ``global_step`` is
    ``cosine_warmup_lr(global_step, total_steps, warmup_steps, lr)`` (the
    reference sets it before each step, train_mlx_k400.py:427-429); without it
    the rate stays ``lr``.  ``ema`` (a ``checkpoint.ModelEMA``) is updated after
    every optimiser step (train_mlx_k400.py:440-441).  ``global_step`` starts at
    ``step_offset`` and advances by one per call."""

    def __init__(self, model: nn.Module, lr: float = 3e-4, weight_decay: float = 0.05, betas=(0.9, 0.95),
                 grad_clip: float = 1.0, label_smoothing: float = 0.1, total_steps: Optional[int] = None,
                 warmup_steps: int = 0, ema=None, step_offset: int = 0):
        self.model = model
        self.opt = AdamW(model.parameters(), lr=lr, betas=betas, weight_decay=weight_decay)
        self.base_lr = lr
        self.grad_clip = grad_clip
        self.label_smoothing = label_smoothing
        self.total_steps, self.warmup_steps = total_steps, warmup_steps
        self.ema = ema
        self.global_step = step_offset

    def __call__(self, video: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
        if self.total_steps is not None:
            self.opt.lr = cosine_warmup_lr(self.global_step, self.total_steps, self.warmup_steps, self.base_lr)
        self.opt.zero_grad()
        loss = loss_fn(self.model(video), target, self.label_smoothing)
        loss.backward()
        if self.grad_clip > 0:
            clip_grads_by_norm(self.opt.params, self.grad_clip)
        self.opt.step()
        if self.ema is not None:
            self.ema.update(self.model)
        self.global_step += 1
        return loss.detach()
