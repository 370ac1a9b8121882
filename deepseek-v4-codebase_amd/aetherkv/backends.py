"""Attention backend with the reference's protocol (aether_pipeline/serving.py:71-83, :146-172).

``HipSparseAttentionBackend`` replaces ``CudaSparseAttentionBackend``: ``name()``,
``available()``, ``availability_error()`` and ``sparse_attention(q, kv, topk_indices, sink,
softmax_scale)``.  ``CudaSparseAttentionBackend`` is an alias so engine code that constructs the
reference class name picks up the HIP backend unchanged.
"""
from __future__ import annotations

from typing import Optional

import torch

from .loader import cuda_extension_unavailable_reason
from .sparse_attention import sparse_sink_attention


class HipSparseAttentionBackend:
    """libaetherkv backend for sparse compressed-KV attention on MI355X."""

    def name(self) -> str:
        return "hip_extension"

    def available(self) -> bool:
        return cuda_extension_unavailable_reason(require_device=True) is None

    def availability_error(self) -> Optional[str]:
        return cuda_extension_unavailable_reason(require_device=True)

    def sparse_attention(self, q: torch.Tensor, kv: torch.Tensor, topk_indices: torch.Tensor, sink: torch.Tensor,
                         softmax_scale: float) -> torch.Tensor:
        return sparse_sink_attention(q.contiguous(), kv.contiguous(), topk_indices.contiguous(), sink.contiguous(),
                                     softmax_scale)


CudaSparseAttentionBackend = HipSparseAttentionBackend
