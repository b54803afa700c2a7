"""Top-4 convex projection (unmerge) on gfx950.

`top4_project(table, index, weight)` returns out[i] = sum_c weight[i,c] *
table[index[i,c]] with the reference's rounding: weights rounded to the value
dtype, each product rounded to the value dtype, fp32 sum, result in the value
dtype (reference vggt_omega/models/token_merging.py:408-413).  It is the kernel
behind every plan `restore`.
"""
from __future__ import annotations

import torch

from . import _kernels, _lib


def top4_project(table: torch.Tensor, index: torch.Tensor, weight: torch.Tensor, *,
                 out: torch.Tensor | None = None, order: torch.Tensor | None = None) -> torch.Tensor:
    """Gather four rows of `table` [M, D] per output row and take their weighted sum
    (torch.ops.vgo.top4_project, or top4_project_into with `out`); see
    `_top4_project_impl`.  `order` (int32 [N], e.g. from `locality_order`) only sets
    the order the rows are computed in; the result is the same."""
    _lib.require_gpu(table, index, weight, out, order)
    if order is not None:
        if out is None:
            out = torch.empty((index.shape[0], table.shape[1]), device=table.device, dtype=table.dtype)
        torch.ops.vgo.top4_project_ordered_into(table, index, weight, order, out)
        return out
    if out is None:
        return torch.ops.vgo.top4_project(table, index, weight)
    torch.ops.vgo.top4_project_into(table, index, weight, out)
    return out


def locality_order(index: torch.Tensor, table_rows: int) -> torch.Tensor:
    """Output rows grouped by their first parent (stable, int32 [N]): computed in this
    order, the rows that share a parent run together and that parent's repeated
    gathers hit the L2 cache.  Reusable for every restore with the same index."""
    _lib.require_gpu(index)
    if index.ndim != 2 or index.shape[1] != 4 or index.dtype != torch.int32:
        raise ValueError("locality_order requires int32 index [N, 4]")
    order, _ = _kernels.csr_build(index[:, 0].contiguous(), int(table_rows))
    return order.view(torch.int32)


def gather_probe(table: torch.Tensor, index: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """The projection's gathers and arithmetic without its row writes: each output row's
    values summed in fp32 (float32 [N]).  A measurement probe (vgo_top4_gather_probe):
    its time is what the memory fabric gives `top4_project`'s random-row reads."""
    lib = _lib.load()
    _lib.require_gpu(table, index, weight)
    if table.ndim != 2 or index.shape != weight.shape or index.ndim != 2 or index.shape[1] != 4:
        raise ValueError("gather_probe requires table [M,D], index [N,4] and weight [N,4]")
    if index.dtype != torch.int32 or weight.dtype != torch.float32 or table.stride(-1) != 1:
        raise ValueError("gather_probe requires int32 indices, float32 weights and unit-stride rows")
    index, weight = index.contiguous(), weight.contiguous()
    sums = torch.empty(index.shape[0], device=table.device, dtype=torch.float32)
    _lib.check(lib.vgo_top4_gather_probe(
        table.data_ptr(), table.stride(0), index.data_ptr(), weight.data_ptr(), sums.data_ptr(),
        index.shape[0], table.shape[0], table.shape[1], _lib.dtype_code(table.dtype), _lib.stream_of(table)))
    return sums


def _top4_project_impl(table: torch.Tensor, index: torch.Tensor, weight: torch.Tensor, *,
                       out: torch.Tensor | None = None,
                       order: torch.Tensor | None = None) -> torch.Tensor:
    """Gather four rows of `table` [M, D] per output row and take their weighted sum.

    index: [N, 4] int32, weight: [N, 4] float32 (both contiguous).  Zero weights
    skip their gather; an out-of-range index with a non-zero weight yields a NaN
    row (the kernel never reads outside the table).
    """
    lib = _lib.load()
    _lib.require_gpu(table, index, weight, out)
    if table.ndim != 2 or index.ndim != 2 or index.shape[1] != 4 or weight.shape != index.shape:
        raise ValueError("top4_project requires table [M,D], index [N,4] and weight [N,4]")
    if index.dtype != torch.int32 or weight.dtype != torch.float32:
        raise ValueError("top4_project requires int32 indices and float32 weights")
    index = index.contiguous()
    weight = weight.contiguous()
    if table.stride(-1) != 1:
        table = table.contiguous()
    n_rows, dim = index.shape[0], table.shape[1]
    if out is None:
        out = torch.empty((n_rows, dim), device=table.device, dtype=table.dtype)
    elif out.shape != (n_rows, dim) or out.dtype != table.dtype or out.stride(-1) != 1:
        raise ValueError("top4_project output must be [N, D] of the table dtype")
    if order is not None:
        if order.shape != (n_rows,) or order.dtype != torch.int32:
            raise ValueError("top4_project order must be int32 [N]")
        order = order.contiguous()
        status = lib.vgo_top4_project_ordered(
            table.data_ptr(), table.stride(0), index.data_ptr(), weight.data_ptr(), order.data_ptr(),
            out.data_ptr(), out.stride(0), n_rows, table.shape[0], dim, _lib.dtype_code(table.dtype),
            _lib.stream_of(table))
    else:
        status = lib.vgo_top4_project(
            table.data_ptr(), table.stride(0), index.data_ptr(), weight.data_ptr(), out.data_ptr(),
            out.stride(0), n_rows, table.shape[0], dim, _lib.dtype_code(table.dtype),
            _lib.stream_of(table),
        )
    _lib.check(status)
    return out
