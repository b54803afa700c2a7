"""Fused kernels of the sparse-convex planners (API of the reference's Triton module).

* `streaming_top4(query, basis_t)` keeps the signature and contract of
  vggt_omega/models/sparse_convex_kernels.py:309-329: memory-bounded bf16 top-4
  retrieval, scores rounded once to bf16 before ranking, ties keep the earlier
  basis id.  It runs `vgo_similarity_topk` (csrc/similarity.hip).
* `four_support_active_set(gram, rhs, ridge=1e-4)` (:332-353) and
  `four_support_projected_gradient(gram, rhs, steps=32)` (:283-296): the two
  four-variable simplex least-squares solvers on [N,4,4] Gram / [N,4] rhs
  inputs, one lane per row (`vgo_four_support_active_set`,
  `vgo_four_support_projected_gradient`, csrc/simplex.hip).
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


def _solver_inputs(gram: torch.Tensor, rhs: torch.Tensor, message: str) -> tuple[torch.Tensor, torch.Tensor]:
    if gram.ndim != 3 or gram.shape[1:] != (4, 4) or rhs.shape != (len(gram), 4):
        raise ValueError(message)
    return gram.contiguous().float(), rhs.contiguous().float()


def four_support_projected_gradient(
    gram: torch.Tensor, rhs: torch.Tensor, *, steps: int = 32,
) -> torch.Tensor:
    """Run the four-way simplex projected-gradient iterations in one kernel."""
    if not triton_acceleration_available():
        raise RuntimeError("the fused convex solver requires the vgo HIP library")
    gram, rhs = _solver_inputs(gram, rhs, "the fused convex solver requires [N,4,4] Gram and [N,4] rhs")
    _lib.require_gpu(gram, rhs)
    output = torch.empty_like(rhs)
    status = _lib.load().vgo_four_support_projected_gradient(
        gram.data_ptr(), rhs.data_ptr(), len(gram), int(steps), output.data_ptr(), _lib.stream_of(gram))
    _lib.check(status)
    return output


def four_support_active_set(gram: torch.Tensor, rhs: torch.Tensor, *, ridge: float = 1e-4) -> torch.Tensor:
    """Exact 15-active-set simplex least-squares solve in one kernel."""
    if not triton_acceleration_available() or not gram.is_cuda:
        raise RuntimeError("four_support_active_set requires the vgo HIP library and GPU tensors")
    gram, rhs = _solver_inputs(gram, rhs, "active-set solver requires [N,4,4] Gram and [N,4] rhs")
    _lib.require_gpu(gram, rhs)
    output = torch.empty_like(rhs)
    status = _lib.load().vgo_four_support_active_set(
        gram.data_ptr(), rhs.data_ptr(), len(gram), float(ridge), output.data_ptr(), _lib.stream_of(gram))
    _lib.check(status)
    return output
