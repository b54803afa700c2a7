"""Oracle: top-4 convex projection / plan restore (test infrastructure only).

Restates the restore arithmetic of vggt_omega/models/token_merging.py:405-413:
  parent   = value[:, parent_compact]                      -> [M, 4, C]
  restored = (parent * w.to(value.dtype)[..., None]).sum(2) -> products rounded
             to the value dtype, summed in fp32 (autocast runs `sum` in fp32),
             result cast back to the value dtype (:413).
Zero weights contribute nothing (for finite tables identical to multiplying by
zero); an out-of-range index with a non-zero weight makes the row NaN, which is
the HIP kernel's documented error signal.
"""
from __future__ import annotations

import torch


def top4_project(table: torch.Tensor, index: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """table [M,D], index [N,4] int, weight [N,4] float32 -> [N,D] in table.dtype."""
    dtype = table.dtype
    n_rows = index.shape[0]
    index = index.long()
    valid = (index >= 0) & (index < table.shape[0])
    safe = torch.where(valid, index, torch.zeros_like(index))
    acc = torch.zeros((n_rows, table.shape[1]), dtype=torch.float32)
    w_value = weight if dtype == torch.float32 else weight.to(dtype)
    bad = torch.zeros(n_rows, dtype=torch.bool)
    for corner in range(4):
        use = weight[:, corner] != 0
        bad |= use & ~valid[:, corner]
        rows = table.index_select(0, safe[:, corner])
        product = (rows * w_value[:, corner, None]).to(torch.float32)
        acc = torch.where((use & valid[:, corner])[:, None], acc + product, acc)
    acc[bad] = float("nan")
    return acc.to(dtype)


def top4_project_fp64(table: torch.Tensor, index: torch.Tensor,
                      weight: torch.Tensor) -> torch.Tensor:
    """Closed form in float64 with no intermediate rounding (pins the above)."""
    rows = table.double()[index.long()]
    return (rows * weight.double()[..., None]).sum(dim=1)
