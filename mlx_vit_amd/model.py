"""NoPE + GDN video classifier (the reference's model family) around the HIP
GatedDeltaLayer.

Module structure, parameter names and defaults follow nope_gdn_mlx.py:
TubeletEmbedding3D (98-150), NoPEMultiheadAttention (157-194), DropPath and
NoPEViTBlock (200-262), NoPEVideoEncoder (269-333), HybridBlock (4009-4091),
NoPEGDNVideoBackbone (4097-4209), TemporalPoolingHead (4215-4264),
VideoClassificationHead (4267-4282) and NoPEGDNClassifier (4285-4342).
Video input is channels-last (B, T, H, W, C) as in the reference.

Differences of form, not of function:
* the tubelet embedding is the equivalent patch reshape + one GEMM (the
  reference's Conv3d has kernel = stride, so every output reads a disjoint
  patch); its weight keeps the MLX Conv3d layout (D, kt, kh, kw, C);
* attention runs in fp32 (torch SDPA) whatever the activation dtype, and its
  result is cast back;
* ``to_bf16`` keeps ``A_log`` and ``dt_bias`` in fp32, as the reference's
  bf16 policy does (nope_gdn_mlx.py:4959-5008).
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .layer import GatedDeltaLayer

BF16_KEEP_FP32 = ("A_log", "dt_bias")


class TubeletEmbedding3D(nn.Module):
    """Non-overlapping 3D patches -> (B, T'*H'*W', D) (nope_gdn_mlx.py:98-150)."""

    def __init__(self, img_size: int = 224, num_frames: int = 32, tubelet_size=(2, 16, 16),
                 in_channels: int = 3, embed_dim: int = 384):
        super().__init__()
        self.tubelet_size = tuple(tubelet_size)
        self.img_size = img_size
        self.num_frames = num_frames
        self.embed_dim = embed_dim
        t, h, w = self.tubelet_size
        self.projection = _PatchProjection(embed_dim, t, h, w, in_channels)
        self.num_temporal_patches = num_frames // t
        self.num_spatial_patches_h = img_size // h
        self.num_spatial_patches_w = img_size // w
        self.num_patches = self.num_temporal_patches * self.num_spatial_patches_h * self.num_spatial_patches_w

    def forward(self, video: torch.Tensor) -> torch.Tensor:
        B, T, H, W, C = video.shape
        t, h, w = self.tubelet_size
        x = video.reshape(B, T // t, t, H // h, h, W // w, w, C)
        x = x.permute(0, 1, 3, 5, 2, 4, 6, 7).reshape(B, -1, t * h * w * C)
        return self.projection(x)

    def get_grid_dims(self):
        return {"T": self.num_temporal_patches, "H": self.num_spatial_patches_h,
                "W": self.num_spatial_patches_w, "total": self.num_patches}


class _PatchProjection(nn.Module):
    """The Conv3d(kernel = stride) of the tubelet embedding as a GEMM; weight in
    the MLX Conv3d layout (out, kt, kh, kw, in), PyTorch's default Conv3d init."""

    def __init__(self, out: int, kt: int, kh: int, kw: int, cin: int):
        super().__init__()
        fan_in = kt * kh * kw * cin
        bound = 1.0 / fan_in ** 0.5
        self.weight = nn.Parameter(torch.empty(out, kt, kh, kw, cin).uniform_(-bound, bound))
        self.bias = nn.Parameter(torch.empty(out).uniform_(-bound, bound))

    def forward(self, patches: torch.Tensor) -> torch.Tensor:
        return F.linear(patches, self.weight.reshape(self.weight.shape[0], -1), self.bias)


def _attention(q, k, v, scale):
    dt = q.dtype
    out = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), scale=scale)
    return out.to(dt)


class NoPEMultiheadAttention(nn.Module):
    """Self-attention without positional encoding (nope_gdn_mlx.py:157-194)."""

    def __init__(self, embed_dim: int, num_heads: int, dropout: float = 0.0, bias: bool = False):
        super().__init__()
        if embed_dim % num_heads:
            raise ValueError("embed_dim must be divisible by num_heads")
        self.embed_dim, self.num_heads = embed_dim, num_heads
        self.head_dim = embed_dim // num_heads
        self.scale = self.head_dim ** -0.5
        self.qkv_proj = nn.Linear(embed_dim, embed_dim * 3, bias=bias)
        self.out_proj = nn.Linear(embed_dim, embed_dim, bias=bias)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if mask is not None:
            raise ValueError("attention masks are not supported on this path")
        B, N, D = x.shape
        H, d = self.num_heads, self.head_dim
        qkv = self.qkv_proj(x).reshape(B, N, 3, H, d).permute(2, 0, 3, 1, 4)
        out = _attention(qkv[0], qkv[1], qkv[2], self.scale)
        return self.out_proj(out.transpose(1, 2).reshape(B, N, D))


class DropPath(nn.Module):
    """Stochastic depth, per sample (nope_gdn_mlx.py:200-213)."""

    def __init__(self, drop_prob: float = 0.0):
        super().__init__()
        self.drop_prob = drop_prob

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.drop_prob == 0.0 or not self.training:
            return x
        keep = 1.0 - self.drop_prob
        mask = torch.empty((x.shape[0],) + (1,) * (x.dim() - 1), device=x.device).bernoulli_(keep).to(x.dtype)
        return x * mask / keep


def _mlp(dim: int, ratio: float, dropout: float) -> nn.Sequential:
    h = int(dim * ratio)
    return nn.Sequential(nn.Linear(dim, h), nn.GELU(), nn.Dropout(dropout), nn.Linear(h, dim), nn.Dropout(dropout))


class NoPEViTBlock(nn.Module):
    """Pre-norm ViT block, optional spatial-only attention (nope_gdn_mlx.py:216-262)."""

    def __init__(self, embed_dim: int, num_heads: int, mlp_ratio: float = 4.0, dropout: float = 0.0,
                 spatial_tokens: Optional[int] = None, drop_path: float = 0.0):
        super().__init__()
        self.spatial_tokens = spatial_tokens
        self.norm1 = nn.LayerNorm(embed_dim, eps=1e-6)
        self.attn = NoPEMultiheadAttention(embed_dim, num_heads, dropout)
        self.drop_path = DropPath(drop_path) if drop_path > 0 else nn.Identity()
        self.norm2 = nn.LayerNorm(embed_dim, eps=1e-6)
        self.mlp = _mlp(embed_dim, mlp_ratio, dropout)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, N, D = x.shape
        normed = self.norm1(x)
        if self.spatial_tokens is not None:
            S = self.spatial_tokens
            a = self.attn(normed.reshape(B * (N // S), S, D)).reshape(B, N, D)
        else:
            a = self.attn(normed, mask=mask)
        x = x + self.drop_path(a)
        return x + self.drop_path(self.mlp(self.norm2(x)))


class NoPEVideoEncoder(nn.Module):
    """Tubelet embedding + NoPE ViT blocks (nope_gdn_mlx.py:269-333)."""

    def __init__(self, img_size: int = 224, num_frames: int = 32, tubelet_size=(2, 16, 16), in_channels: int = 3,
                 embed_dim: int = 384, depth: int = 12, num_heads: int = 6, mlp_ratio: float = 4.0,
                 dropout: float = 0.0, factorized_attention: bool = True, drop_path_rate: float = 0.0):
        super().__init__()
        self.tubelet_embed = TubeletEmbedding3D(img_size, num_frames, tubelet_size, in_channels, embed_dim)
        grid = self.tubelet_embed.get_grid_dims()
        spatial = grid["H"] * grid["W"] if factorized_attention else None
        dpr = [drop_path_rate * i / (depth - 1) for i in range(depth)] if drop_path_rate > 0 and depth > 1 \
            else [0.0] * depth
        self.blocks = nn.ModuleList([NoPEViTBlock(embed_dim, num_heads, mlp_ratio, dropout, spatial, dpr[i])
                                     for i in range(depth)])
        self.norm = nn.LayerNorm(embed_dim, eps=1e-6)
        self.embed_dim, self.depth = embed_dim, depth
        self.factorized_attention = factorized_attention

    def forward(self, video: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        x = self.tubelet_embed(video)
        for blk in self.blocks:
            x = blk(x, mask=mask)
        return self.norm(x)

    def get_grid_dims(self):
        return self.tubelet_embed.get_grid_dims()


class HybridBlock(nn.Module):
    """One processor block, GDN or NoPE attention (nope_gdn_mlx.py:4009-4091)."""

    def __init__(self, dim: int, num_heads: int, block_type: str = "gdn", head_dim: Optional[int] = None,
                 chunk_size: int = 64, mlp_ratio: float = 4.0, dropout: float = 0.0,
                 channel_wise_decay: bool = True, allow_neg_eigval: bool = False,
                 spatial_tokens: Optional[int] = None, drop_path: float = 0.0, gdn_temporal_only: bool = False):
        super().__init__()
        if block_type not in ("gdn", "nope"):
            raise ValueError(f"block_type must be 'gdn' or 'nope'; got {block_type!r}")
        self.block_type = block_type
        self.spatial_tokens = spatial_tokens
        self.gdn_temporal_only = gdn_temporal_only
        self.norm1 = nn.LayerNorm(dim, eps=1e-6)
        self.drop_path = DropPath(drop_path) if drop_path > 0 else nn.Identity()
        if block_type == "gdn":
            self.layer = GatedDeltaLayer(dim, num_heads, head_dim or dim // num_heads, chunk_size,
                                         channel_wise_decay=channel_wise_decay, allow_neg_eigval=allow_neg_eigval)
        else:
            self.layer = NoPEMultiheadAttention(dim, num_heads, dropout)
        self.norm2 = nn.LayerNorm(dim, eps=1e-6)
        self.mlp = _mlp(dim, mlp_ratio, dropout)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None,
                state: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        B, N, D = x.shape
        normed = self.norm1(x)
        if self.block_type == "gdn":
            if self.gdn_temporal_only and self.spatial_tokens is not None:
                # time-only scan: one recurrence per spatial location over T'
                S = self.spatial_tokens
                T = N // S
                xt = normed.reshape(B, T, S, D).transpose(1, 2).reshape(B * S, T, D)
                out_t, _ = self.layer(xt, None)
                out = out_t.reshape(B, S, T, D).transpose(1, 2).reshape(B, N, D)
                new_state = state
            else:
                out, new_state = self.layer(normed, state)
        elif self.spatial_tokens is not None:
            S = self.spatial_tokens
            out = self.layer(normed.reshape(B * (N // S), S, D)).reshape(B, N, D)
            new_state = state
        else:
            out = self.layer(normed, mask=mask)
            new_state = state
        x = x + self.drop_path(out)
        x = x + self.drop_path(self.mlp(self.norm2(x)))
        return x, new_state


class NoPEGDNVideoBackbone(nn.Module):
    """NoPE encoder + GDN:NoPE hybrid processor (nope_gdn_mlx.py:4097-4209)."""

    def __init__(self, img_size: int = 224, num_frames: int = 32, tubelet_size=(2, 16, 16), in_channels: int = 3,
                 encoder_dim: int = 384, encoder_depth: int = 12, encoder_heads: int = 6,
                 processor_dim: int = 384, processor_depth: int = 4, processor_heads: int = 6,
                 gdn_ratio: int = 3, chunk_size: int = 64, channel_wise_decay: bool = True,
                 allow_neg_eigval: bool = False, factorized_attention: bool = True,
                 gdn_temporal_only: bool = False, mlp_ratio: float = 4.0, dropout: float = 0.0,
                 drop_path_rate: float = 0.0):
        super().__init__()
        total = encoder_depth + processor_depth
        dpr = [drop_path_rate * i / (total - 1) for i in range(total)] if drop_path_rate > 0 and total > 1 \
            else [0.0] * total
        enc_rate = drop_path_rate * encoder_depth / total if total > 0 else 0.0
        self.encoder = NoPEVideoEncoder(img_size, num_frames, tubelet_size, in_channels, encoder_dim,
                                        encoder_depth, encoder_heads, mlp_ratio, dropout, factorized_attention,
                                        enc_rate)
        grid = self.encoder.get_grid_dims()
        spatial = grid["H"] * grid["W"] if factorized_attention else None
        self.dim_proj = nn.Linear(encoder_dim, processor_dim) if encoder_dim != processor_dim else nn.Identity()
        period = gdn_ratio + 1
        blocks = []
        for i in range(processor_depth):
            bt = "nope" if (i + 1) % period == 0 else "gdn"
            blocks.append(HybridBlock(processor_dim, processor_heads, bt, processor_dim // processor_heads,
                                      chunk_size, mlp_ratio, dropout, channel_wise_decay, allow_neg_eigval,
                                      spatial if (bt == "nope" or gdn_temporal_only) else None,
                                      dpr[encoder_depth + i], gdn_temporal_only))
        self.processor_blocks = nn.ModuleList(blocks)
        self.processor_norm = nn.LayerNorm(processor_dim, eps=1e-6)
        self.encoder_dim, self.processor_dim = encoder_dim, processor_dim
        self.spatial_tokens = spatial
        self.factorized_attention = factorized_attention

    def forward(self, video: torch.Tensor, processor_mask: Optional[torch.Tensor] = None,
                return_encoder_features: bool = False):
        enc = self.encoder(video)
        x = self.dim_proj(enc)
        states: List[Optional[torch.Tensor]] = [None] * len(self.processor_blocks)
        for i, blk in enumerate(self.processor_blocks):
            x, states[i] = blk(x, mask=processor_mask, state=states[i])
        x = self.processor_norm(x)
        return (x, enc) if return_encoder_features else x

    def get_block_types(self) -> List[str]:
        return [b.block_type for b in self.processor_blocks]


class TemporalPoolingHead(nn.Module):
    """Spatial mean per frame, single-query temporal attention, linear classifier
    (nope_gdn_mlx.py:4215-4264)."""

    def __init__(self, embed_dim: int, num_classes: int, num_heads: int = 8, dropout: float = 0.0):
        super().__init__()
        self.embed_dim, self.num_heads = embed_dim, num_heads
        self.head_dim = embed_dim // num_heads
        self.temporal_query = nn.Parameter(torch.randn(1, 1, embed_dim) * 0.02)
        self.t_proj_k = nn.Linear(embed_dim, embed_dim, bias=False)
        self.t_proj_v = nn.Linear(embed_dim, embed_dim, bias=False)
        self.t_proj_out = nn.Linear(embed_dim, embed_dim, bias=False)
        self.t_norm = nn.LayerNorm(embed_dim, eps=1e-6)
        self.dropout = nn.Dropout(dropout)
        self.fc = nn.Linear(embed_dim, num_classes)

    def forward(self, x: torch.Tensor, S: int = 196) -> torch.Tensor:
        B, N, D = x.shape
        T = N // S
        H, d = self.num_heads, self.head_dim
        x_frame = x.reshape(B, T, S, D).mean(dim=2)
        q = self.temporal_query.expand(B, 1, D).reshape(B, 1, H, d).transpose(1, 2)
        k = self.t_proj_k(x_frame).reshape(B, T, H, d).transpose(1, 2)
        v = self.t_proj_v(x_frame).reshape(B, T, H, d).transpose(1, 2)
        out = _attention(q, k, v, d ** -0.5).transpose(1, 2).reshape(B, D)
        out = self.t_proj_out(out) + x_frame.mean(dim=1)
        return self.fc(self.dropout(self.t_norm(out)))


class VideoClassificationHead(nn.Module):
    """LayerNorm, mean over tokens, linear classifier (nope_gdn_mlx.py:4267-4282)."""

    def __init__(self, embed_dim: int, num_classes: int, dropout: float = 0.0):
        super().__init__()
        self.norm = nn.LayerNorm(embed_dim, eps=1e-6)
        self.dropout = nn.Dropout(dropout)
        self.fc = nn.Linear(embed_dim, num_classes)

    def forward(self, x: torch.Tensor, S: Optional[int] = None) -> torch.Tensor:
        return self.fc(self.dropout(self.norm(x).mean(dim=1)))


class NoPEGDNClassifier(nn.Module):
    """End-to-end NoPE + GDN video classifier (nope_gdn_mlx.py:4285-4342)."""

    def __init__(self, img_size: int = 224, num_frames: int = 32, tubelet_size=(2, 16, 16), in_channels: int = 3,
                 encoder_dim: int = 384, encoder_depth: int = 12, encoder_heads: int = 6,
                 processor_dim: int = 384, processor_depth: int = 4, processor_heads: int = 6,
                 gdn_ratio: int = 3, chunk_size: int = 64, channel_wise_decay: bool = True,
                 allow_neg_eigval: bool = False, factorized_attention: bool = True,
                 gdn_temporal_only: bool = False, head_type: str = "temporal", num_classes: int = 174,
                 mlp_ratio: float = 4.0, dropout: float = 0.0, head_dropout: float = 0.0,
                 drop_path_rate: float = 0.0):
        super().__init__()
        self.backbone = NoPEGDNVideoBackbone(
            img_size, num_frames, tubelet_size, in_channels, encoder_dim, encoder_depth, encoder_heads,
            processor_dim, processor_depth, processor_heads, gdn_ratio, chunk_size, channel_wise_decay,
            allow_neg_eigval, factorized_attention, gdn_temporal_only, mlp_ratio, dropout, drop_path_rate)
        self.spatial_tokens = (img_size // tubelet_size[1]) * (img_size // tubelet_size[2])
        if head_type == "mean":
            self.head = VideoClassificationHead(processor_dim, num_classes, dropout=head_dropout)
        else:
            self.head = TemporalPoolingHead(processor_dim, num_classes, num_heads=processor_heads,
                                            dropout=head_dropout)

    def forward(self, video: torch.Tensor) -> torch.Tensor:
        return self.head(self.backbone(video), S=self.spatial_tokens)


def to_bf16(model: nn.Module, keep_fp32: Tuple[str, ...] = BF16_KEEP_FP32) -> nn.Module:
    """Cast every fp32 parameter to bf16 except those whose name contains one of
    ``keep_fp32`` (nope_gdn_mlx.py:4959-5008).  In place; returns the model."""
    for name, p in model.named_parameters():
        if p.dtype == torch.float32 and not any(s in name for s in keep_fp32):
            p.data = p.data.to(torch.bfloat16)
    return model


def config4(num_classes: int = 400) -> NoPEGDNClassifier:
    """The NoPE-GDN ViT-B step's model: 12 GDN processor blocks of width 768
    with 12 heads of 64, no encoder blocks, 16 frames of 224 x 224 (1568 tokens)."""
    return NoPEGDNClassifier(num_frames=16, encoder_depth=0, processor_depth=12, gdn_ratio=12,
                             processor_dim=768, processor_heads=12, num_classes=num_classes)
