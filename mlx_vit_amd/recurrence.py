"""The recurrence half of the reference's GatedDeltaLayer: path validation and
string dispatch, with ``gdn_path='hip_chunkwise_kda'`` as the MI355X path
(and ``'hip_chunkwise_gdn'`` for scalar-alpha decay, where ``g`` is alpha).

The reference selects a KDA compute path by name at construction and per call
(``compute_path``, nope_gdn_mlx.py:693-735 and 823-878); every path is a method
with the signature ``(q, k, v, g, beta, state) -> (output, new_state)``
(nope_gdn_mlx.py:3056-3068).  ``KDARecurrence`` keeps that contract:

* construction validates the path and raises ``ValueError`` for combinations
  the kernels cannot run (as nope_gdn_mlx.py:696-734 does for its Metal
  budgets);
* ``__call__(q, k, v, g, beta, state=None, compute_path=None)`` dispatches by
  name and raises ``ValueError(f"Unknown compute_path: {path}")`` otherwise
  (nope_gdn_mlx.py:877-878).

There is no silent fallback to another path: the reference falls back from
Metal to 'compiled' on failure (nope_gdn_mlx.py:852-866); here a failure
raises, so a result always comes from the HIP kernels.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from .kda import BWD_HEAD_DIMS, CHUNK, CHUNK_SIZES, FWD_HEAD_DIMS, chunk_gdn, chunk_kda

HIP_PATH = "hip_chunkwise_kda"
GDN_HIP_PATH = "hip_chunkwise_gdn"   # scalar-alpha GDN on the same kernels
KDA_PATHS = (HIP_PATH, GDN_HIP_PATH)


class KDARecurrence:
    """KDA recurrence dispatcher for ``head_dim``-wide heads."""

    def __init__(self, num_heads: int, head_dim: int = 64, chunk_size: int = CHUNK,
                 channel_wise_decay: bool = True, compute_path: Optional[str] = None,
                 requires_grad: bool = True):
        if compute_path is None:
            compute_path = HIP_PATH if channel_wise_decay else GDN_HIP_PATH
        # the reference's pairing of paths and decay kinds (nope_gdn_mlx.py:696-705)
        if compute_path == HIP_PATH and not channel_wise_decay:
            raise ValueError(f"{HIP_PATH} is only valid for channel-wise KDA (channel_wise_decay=True). "
                             f"For scalar-alpha use '{GDN_HIP_PATH}'.")
        if compute_path == GDN_HIP_PATH and channel_wise_decay:
            raise ValueError(f"{GDN_HIP_PATH} is only valid for scalar-alpha GDN (channel_wise_decay=False). "
                             f"For channel-wise KDA use '{HIP_PATH}'.")
        self._validate(compute_path, head_dim, chunk_size, requires_grad)
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.chunk_size = chunk_size
        self.channel_wise_decay = channel_wise_decay
        self.compute_path = compute_path
        self.requires_grad = requires_grad

    @staticmethod
    def _validate(path: str, head_dim: int, chunk_size: int, requires_grad: bool) -> None:
        if path not in KDA_PATHS:
            raise ValueError(f"Unknown compute_path: {path}")
        if chunk_size not in CHUNK_SIZES:
            raise ValueError(f"compute_path='{path}' requires chunk_size in {CHUNK_SIZES}; got {chunk_size}")
        dims = BWD_HEAD_DIMS if requires_grad else FWD_HEAD_DIMS
        if head_dim not in dims:
            raise ValueError(
                f"compute_path='{path}' supports head_dim in {dims} "
                f"({'training' if requires_grad else 'inference'}); got head_dim={head_dim}")

    def __call__(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                 beta: torch.Tensor, state: Optional[torch.Tensor] = None,
                 compute_path: Optional[str] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        path = compute_path or self.compute_path
        if path == HIP_PATH and self.channel_wise_decay:
            return self._hip_chunkwise_kda(q, k, v, g, beta, state)
        if path == GDN_HIP_PATH and not self.channel_wise_decay:
            return chunk_gdn(q, k, v, g, beta, state, self.chunk_size)
        if path in KDA_PATHS:
            raise ValueError(f"compute_path='{path}' does not match channel_wise_decay={self.channel_wise_decay}")
        raise ValueError(f"Unknown compute_path: {path}")

    def _hip_chunkwise_kda(self, q, k, v, g, beta, state):
        """(B, L, H, D) q/k/v/g, (B, L, H) beta, (B, H, D, D) state or None ->
        (output in q.dtype, new_state fp32)."""
        B, L, H, D = q.shape
        if D != self.head_dim:
            raise ValueError(f"{HIP_PATH} D mismatch: got {D}, expected {self.head_dim}")
        return chunk_kda(q, k, v, g, beta, state, self.chunk_size)
