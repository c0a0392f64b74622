"""MI355X-native KDA (Kimi Delta Attention / gated delta rule) chunkwise recurrence.

Hand-written gfx950 HIP kernels behind a C ABI (``include/kda_hip.h``,
``libkda_hip.so``), driven from torch through ctypes.
"""
from .kda import (ChunkKDAFunction, chunk_gdn, chunk_kda, gated_supported, kda_backward, kda_backward_train,
                  kda_forward, kda_forward_gated, kda_forward_train, solve_unit_triangular, train_kept_bytes,
                  workspace_bytes, workspace_offsets)
from .layer import (ChunkKDAGatedFunction, GatedDeltaLayer, GatedRMSNormFunction, ProducerFunction, RMSNormGated,
                    ShortCausalConv1d, gated_rmsnorm_backward, gated_rmsnorm_forward, producer_backward,
                    producer_forward)
from .recurrence import GDN_HIP_PATH, HIP_PATH, KDA_PATHS, KDARecurrence

__all__ = [
    "ChunkKDAFunction", "chunk_kda", "chunk_gdn", "kda_forward", "kda_backward", "kda_forward_train",
    "kda_backward_train", "kda_forward_gated", "gated_supported", "solve_unit_triangular",
    "workspace_bytes", "workspace_offsets", "train_kept_bytes", "KDARecurrence", "HIP_PATH", "GDN_HIP_PATH", "KDA_PATHS",
    "GatedDeltaLayer", "ShortCausalConv1d", "RMSNormGated", "ProducerFunction", "GatedRMSNormFunction",
    "ChunkKDAGatedFunction",
    "producer_forward", "producer_backward", "gated_rmsnorm_forward", "gated_rmsnorm_backward",
]
