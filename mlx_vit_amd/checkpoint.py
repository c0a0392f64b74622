"""Checkpoint wire format and weight converters of the reference, for the torch model.

* ``save_checkpoint`` / ``load_checkpoint`` -- one safetensors file with the
  model's parameters under their MLX parameter-tree paths, the EMA shadow under
  the ``__ema__`` prefix, and ``<name>.meta.json`` with epoch, best accuracy
  and EMA decay (train_mlx_k400.py:273-321).  Files written by the reference
  load here and the other way round: the only path difference between the two
  module trees is ``mlp.layers.N`` (MLX Sequential) versus ``mlp.N`` (torch).
* ``ModelEMA`` -- exponential moving average of the trainable parameters,
  ``shadow = d shadow + (1 - d) p`` (train_mlx_k400.py:181-221).
* ``load_pytorch_state_dict`` -- the PyTorch-era NoPE+GDN checkpoint
  (nope_gdn_mlx.py:4349-4494): ``f_proj.{0,1}`` / ``g_proj.{0,1}`` become
  ``f_proj_{1,2}`` / ``g_proj_{1,2}``, the Conv3d weight goes from (oC, iC, T,
  H, W) to channels-last (oC, T, H, W, iC) and the depthwise Conv1d weights
  from (C, 1, K) to (C, K, 1); a report lists loaded keys, shape mismatches,
  keys without a target and parameters not covered.
"""
from __future__ import annotations

import json
import re
import warnings
from pathlib import Path
from typing import Dict, Optional

import torch
import torch.nn as nn

EMA_PREFIX = "__ema__"
_MLP_TORCH = re.compile(r"\.mlp\.(\d+)\.")
_MLP_MLX = re.compile(r"\.mlp\.layers\.(\d+)\.")


def to_mlx_key(name: str) -> str:
    """torch parameter name -> MLX parameter-tree path."""
    return _MLP_TORCH.sub(r".mlp.layers.\1.", name)


def from_mlx_key(key: str) -> str:
    """MLX parameter-tree path -> torch parameter name."""
    return _MLP_MLX.sub(r".mlp.\1.", key)


class ModelEMA:
    """EMA shadow of the trainable parameters, keyed by MLX paths."""

    def __init__(self, model: nn.Module, decay: float = 0.9999):
        self.decay = decay
        self.shadow: Dict[str, torch.Tensor] = {
            to_mlx_key(n): p.detach().clone() for n, p in model.named_parameters() if p.requires_grad}

    @torch.no_grad()
    def update(self, model: nn.Module) -> None:
        pairs = [(self.shadow[to_mlx_key(n)], p.detach()) for n, p in model.named_parameters()
                 if p.requires_grad and to_mlx_key(n) in self.shadow]
        groups: Dict[tuple, list] = {}
        for s, p in pairs:
            groups.setdefault((s.dtype, s.device), []).append((s, p))
        for items in groups.values():
            ss, ps = [s for s, _ in items], [p.to(s.dtype) for s, p in items]
            torch._foreach_lerp_(ss, ps, 1.0 - self.decay)

    def state_dict(self):
        return {"decay": self.decay, "shadow": dict(self.shadow)}

    def load_state_dict(self, sd) -> None:
        self.decay = sd["decay"]
        self.shadow = sd["shadow"]


def _meta_path(path: Path) -> Path:
    return path.with_suffix(".meta.json")


def save_checkpoint(path, model: nn.Module, ema: Optional[ModelEMA] = None, epoch: int = 0,
                    best_acc: float = 0.0) -> int:
    """Write ``path`` (safetensors) and ``path.with_suffix('.meta.json')``;
    returns the number of tensors written."""
    from safetensors.torch import save_file
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    weights = {to_mlx_key(n): p.detach().cpu().contiguous() for n, p in model.named_parameters()}
    if ema is not None:
        for k, v in ema.shadow.items():
            weights[EMA_PREFIX + k] = v.detach().cpu().contiguous()
    save_file(weights, str(path))
    with open(_meta_path(path), "w") as f:
        json.dump({"epoch": epoch, "best_acc": best_acc, "ema_decay": ema.decay if ema else None}, f)
    return len(weights)


def load_checkpoint(path, model: nn.Module, ema: Optional[ModelEMA] = None) -> Dict[str, list]:
    """Load a checkpoint written by ``save_checkpoint`` (or by the reference)
    into ``model`` (and the EMA shadow).  Parameters keep their dtype and device.
    Returns {"missing": [...], "unexpected": [...], "ema_loaded": n}; missing
    and unexpected keys warn, as the reference prints them."""
    from safetensors.torch import load_file
    weights = load_file(str(path))
    model_w = {k: v for k, v in weights.items() if not k.startswith(EMA_PREFIX)}
    ema_w = {k[len(EMA_PREFIX):]: v for k, v in weights.items() if k.startswith(EMA_PREFIX)}
    params = {to_mlx_key(n): p for n, p in model.named_parameters()}
    missing = sorted(params.keys() - model_w.keys())
    unexpected = sorted(model_w.keys() - params.keys())
    if missing:
        warnings.warn(f"{len(missing)} model keys missing from checkpoint (first 3): {missing[:3]}")
    if unexpected:
        warnings.warn(f"{len(unexpected)} unexpected keys in checkpoint (first 3): {unexpected[:3]}")
    with torch.no_grad():
        for k, v in model_w.items():
            if k in params:
                params[k].copy_(v.to(params[k].dtype))
    n_ema = 0
    if ema is not None:
        for k, v in ema_w.items():
            if k in ema.shadow:
                ema.shadow[k] = v.to(ema.shadow[k].device, ema.shadow[k].dtype)
                n_ema += 1
    return {"missing": missing, "unexpected": unexpected, "ema_loaded": n_ema}


def read_meta(path) -> dict:
    with open(_meta_path(Path(path))) as f:
        return json.load(f)


def pt_key(key: str) -> str:
    """PyTorch-era key -> this model's parameter name (nope_gdn_mlx.py:4349-4375:
    the low-rank ``f_proj`` / ``g_proj`` Sequentials; ``mlp.N`` is already the
    torch form)."""
    for a, b in ((".f_proj.0.", ".f_proj_1."), (".f_proj.1.", ".f_proj_2."),
                 (".g_proj.0.", ".g_proj_1."), (".g_proj.1.", ".g_proj_2.")):
        key = key.replace(a, b)
    return key


def load_pytorch_state_dict(model: nn.Module, pt_state_dict: Dict[str, torch.Tensor], strict: bool = True
                            ) -> Dict[str, list]:
    """Load a PyTorch-era NoPE+GDN state dict (nope_gdn_mlx.py:4378-4494).
    Returns {"loaded", "shape_mismatch", "no_target", "unused"}; with
    ``strict`` a shape mismatch, an unmapped key or an uncovered parameter
    raises ``RuntimeError``."""
    params = dict(model.named_parameters())
    remaining = set(params)
    report = {"loaded": [], "shape_mismatch": [], "no_target": [], "unused": []}
    staged = {}
    for k, t in pt_state_dict.items():
        name = pt_key(k)
        if name not in params:
            report["no_target"].append(k)
            continue
        arr = t.detach()
        if name.endswith("tubelet_embed.projection.weight") and arr.dim() == 5:
            arr = arr.permute(0, 2, 3, 4, 1)          # (oC, iC, T, H, W) -> (oC, T, H, W, iC)
        elif name.endswith(("q_conv1d.weight", "k_conv1d.weight", "v_conv1d.weight")) and arr.dim() == 3:
            arr = arr.permute(0, 2, 1)                # (C, 1, K) -> (C, K, 1)
        if tuple(arr.shape) != tuple(params[name].shape):
            report["shape_mismatch"].append((k, name, tuple(arr.shape), tuple(params[name].shape)))
            continue
        staged[name] = arr
        report["loaded"].append((k, name))
        remaining.discard(name)
    report["unused"] = sorted(remaining)
    if strict:
        if report["shape_mismatch"]:
            raise RuntimeError(f"{len(report['shape_mismatch'])} shape mismatches; first: "
                               f"{report['shape_mismatch'][0]}")
        if report["no_target"] or report["unused"]:
            raise RuntimeError(f"{len(report['no_target'])} PT keys without a target, "
                               f"{len(report['unused'])} parameters not covered")
    with torch.no_grad():
        for name, arr in staged.items():
            params[name].copy_(arr.to(params[name].dtype))
    return report
