"""Pins the top-4 projection oracle (CPU only)."""
from __future__ import annotations

import pytest
import torch

from oracle import projection as oracle
from tests._tol import rel_error


def _case(seed, n=97, m=31, d=40, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    table = torch.randn(m, d, generator=g).to(dtype)
    index = torch.stack([torch.randperm(m, generator=g)[:4] for _ in range(n)]).int()
    e = -torch.rand(n, 4, generator=g, dtype=torch.float64).log()
    weight = (e / e.sum(1, keepdim=True)).float()
    return table, index, weight


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_one_hot_is_gather(dtype):
    table, index, _ = _case(0, dtype=dtype)
    weight = torch.zeros(index.shape)
    weight[:, 2] = 1.0
    out = oracle.top4_project(table, index, weight)
    assert torch.equal(out, table[index[:, 2].long()])


def test_uniform_weights_are_the_mean():
    table, index, _ = _case(1)
    weight = torch.full(index.shape, 0.25)
    out = oracle.top4_project(table, index, weight)
    mean = table.double()[index.long()].mean(1)
    assert rel_error(out, mean) < 1e-6


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-6), (torch.bfloat16, 2e-2),
                                       (torch.float16, 5e-3)])
def test_matches_fp64_closed_form(dtype, tol):
    table, index, weight = _case(2, dtype=dtype)
    out = oracle.top4_project(table, index, weight)
    assert rel_error(out, oracle.top4_project_fp64(table, index, weight)) < tol


def test_bf16_products_are_rounded_before_the_sum():
    # The reference multiplies in the value dtype, so each product is rounded.
    table, index, weight = _case(3, dtype=torch.bfloat16)
    out = oracle.top4_project(table, index, weight)
    w = weight.to(torch.bfloat16)
    rows = table[index.long()]
    manual = (rows * w[..., None]).float()
    manual = ((manual[:, 0] + manual[:, 1]) + manual[:, 2]) + manual[:, 3]
    assert torch.equal(out, manual.to(torch.bfloat16))


def test_bad_index_gives_nan_row():
    table, index, weight = _case(4)
    index[5, 1] = table.shape[0] + 3
    index[7, 0] = -1
    weight[7, 0] = 0.0  # zero weight: the bad index is never read
    out = oracle.top4_project(table, index, weight)
    assert torch.isnan(out[5]).all()
    assert torch.isfinite(out[7]).all()


def test_checks_have_teeth():
    table, index, weight = _case(5)
    exact = oracle.top4_project_fp64(table, index, weight)
    swapped = oracle.top4_project(table, index.flip(1), weight)
    assert rel_error(swapped, exact) > 1e-2
