"""Fused matching kernel of the sparse-convex planners (API of the reference's Triton module).

`streaming_top4(query, basis_t)` keeps the signature and contract of
vggt_omega/models/sparse_convex_kernels.py:309-329: memory-bounded bf16 top-4
retrieval, scores rounded once to bf16 before ranking, ties keep the earlier
basis id.  It runs `vgo_similarity_topk` (csrc/similarity.hip).
"""
from __future__ import annotations

import torch

from . import _kernels, _lib


def triton_acceleration_available() -> bool:
    """Name kept for callers of the reference API: True when the HIP library loads."""
    try:
        _lib.load()
    except _lib.ExtensionUnavailable:
        return False
    return True


def streaming_top4(query: torch.Tensor, basis_t: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Memory-bounded BF16 Top-4 without materializing ``query @ basis``."""
    if not triton_acceleration_available() or not query.is_cuda:
        raise RuntimeError("streaming_top4 requires the vgo HIP library and GPU tensors")
    if query.ndim != 2 or basis_t.ndim != 2 or query.shape[1] != basis_t.shape[0]:
        raise ValueError("query [M,D] and transposed basis [D,N] are required")
    if basis_t.shape[1] < 4:
        raise ValueError("streaming Top-4 requires at least four bases")
    query = query.contiguous().to(torch.bfloat16)
    basis = basis_t.to(torch.bfloat16).T.contiguous()
    values, index = _kernels.similarity_topk(query, basis, 4, index_dtype=torch.int64)
    return values, index
