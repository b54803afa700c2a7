"""Parity of the gfx950 top-4 projection kernel against the CPU oracle.

The kernel and the oracle perform the same IEEE operations in the same order
(weight rounded to the value type, each product rounded, fp32 sum in corner
order), so the comparison is bit-exact.
"""
from __future__ import annotations

import pytest
import torch

from oracle import projection as oracle

pytestmark = pytest.mark.gpu


def _case(seed, n, m, d, dtype):
    g = torch.Generator().manual_seed(seed)
    table = torch.randn(m, d, generator=g).to(dtype)
    keys = torch.rand(n, m, generator=g) if m <= 4096 else None
    if keys is not None:
        index = keys.argsort(dim=1)[:, :4].int()
    else:
        index = torch.randint(0, m, (n, 4), generator=g, dtype=torch.int32)
    e = -torch.rand(n, 4, generator=g, dtype=torch.float64).log()
    weight = (e / e.sum(1, keepdim=True)).float()
    return table, index, weight


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("n,m,d", [(1, 4, 8), (97, 31, 64), (1044, 522, 1024), (333, 50, 1000),
                                   (4099, 700, 2048), (257, 16, 23)])
def test_bit_exact_vs_oracle(vgo, device, dtype, n, m, d):
    print(f"[project] dtype={dtype} n={n} m={m} d={d}", flush=True)
    table, index, weight = _case(n + m + d, n, m, d, dtype)
    out = vgo.top4_project(table.to(device), index.to(device), weight.to(device))
    torch.cuda.synchronize()
    ref = oracle.top4_project(table, index, weight)
    assert torch.equal(out.cpu(), ref)


def test_one_hot_restore_is_exact_copy(vgo, device):
    table, index, _ = _case(3, 500, 200, 1024, torch.bfloat16)
    weight = torch.zeros(index.shape)
    weight[:, 0] = 1.0
    out = vgo.top4_project(table.to(device), index.to(device), weight.to(device))
    assert torch.equal(out.cpu(), table[index[:, 0].long()])


def test_bad_index_poisons_row_without_reading(vgo, device):
    table, index, weight = _case(4, 64, 32, 256, torch.float32)
    index[3, 2] = 1 << 30
    index[9, 1] = -5
    weight[9, 1] = 0.0
    out = vgo.top4_project(table.to(device), index.to(device), weight.to(device)).cpu()
    assert torch.isnan(out[3]).all()
    assert torch.isfinite(out[9]).all()
    ref = oracle.top4_project(table, index, weight)
    assert torch.equal(torch.nan_to_num(out), torch.nan_to_num(ref))


def test_strided_table_and_output(vgo, device):
    table, index, weight = _case(6, 300, 90, 512, torch.bfloat16)
    wide = torch.zeros(90, 1024, dtype=torch.bfloat16)
    wide[:, 256:768] = table
    out = torch.full((300, 1024), 7.0, dtype=torch.bfloat16, device=device)
    view = out[:, 128:640]
    vgo.top4_project(wide.to(device)[:, 256:768], index.to(device), weight.to(device), out=view)
    ref = oracle.top4_project(table, index, weight)
    assert torch.equal(view.cpu(), ref)
    assert (out[:, :128] == 7).all() and (out[:, 640:] == 7).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,m,d", [(4099, 700, 1024), (1044, 522, 1000), (257, 16, 23)])
def test_ordered_projection_equals_plain(dtype, device, n, m, d):
    """Rows computed in the locality order (grouped by first parent) or any other
    order give the plain projection bit for bit; order entries outside [0, N)
    compute nothing."""
    print(f"[project] ordered dtype={dtype} n={n} m={m} d={d}", flush=True)
    from tests.conftest import import_package
    proj = import_package("projection")
    table, index, weight = _case(n * 3 + m + d, n, m, d, dtype)
    table, index, weight = table.to(device), index.to(device), weight.to(device)
    plain = proj.top4_project(table, index, weight)
    order = proj.locality_order(index, m)
    assert order.dtype == torch.int32 and torch.equal(order.sort().values.cpu(), torch.arange(n, dtype=torch.int32))
    first = index[:, 0].long()[order.long()].cpu()
    assert bool((first[1:] >= first[:-1]).all()), "locality order must group rows by first parent"
    assert torch.equal(proj.top4_project(table, index, weight, order=order), plain)
    shuffled = torch.randperm(n, generator=torch.Generator().manual_seed(n)).int().to(device)
    assert torch.equal(proj.top4_project(table, index, weight, order=shuffled), plain)
    partial = shuffled.clone()
    partial[: n // 2] = -1
    out = torch.full_like(plain, 7.0)
    proj.top4_project(table, index, weight, out=out, order=partial)
    done = torch.zeros(n, dtype=torch.bool)
    done[partial[n // 2:].long().cpu()] = True
    assert torch.equal(out[done.to(device)], plain[done.to(device)])
    assert bool((out[~done.to(device)] == 7.0).all())


@pytest.mark.parametrize("dtype,n,m,d,strided", [
    (torch.bfloat16, 40007, 3000, 1024, False), (torch.float32, 33001, 1500, 1024, False),
    (torch.float16, 33000, 2500, 1024, True), (torch.bfloat16, 33000, 2500, 1024, True),
    (torch.bfloat16, 32800, 1100, 2048, False)])
def test_large_tables_bit_exact(vgo, device, dtype, n, m, d, strided):
    """Tables larger than an XCD's L2 (4 MB) with tens of thousands of rows, the C2
    regime at a size the oracle checks whole: bit-exact on a ragged row count, strided
    table and output views, a poisoned row (out-of-range id with a non-zero weight), a
    zero-weight out-of-range id that must not poison, and one-hot rows."""
    print(f"[project] large table dtype={dtype} n={n} m={m} d={d} strided={strided}", flush=True)
    table, index, weight = _case(n + m + d, n, m, d, dtype)
    index[5, 1] = m + 17           # poisons row 5
    index[11, 3] = -2              # zero weight: ignored
    weight[11, 3] = 0.0
    weight[13] = torch.tensor([0.0, 1.0, 0.0, 0.0])   # one-hot row
    assert table.numel() * table.element_size() > 4 << 20
    if strided:
        wide = torch.zeros(m, d + 256, dtype=dtype)
        wide[:, 128:128 + d] = table
        table_d = wide.to(device)[:, 128:128 + d]
        out_full = torch.full((n, d + 64), 3.0, dtype=dtype, device=device)
        out = out_full[:, 64:]
    else:
        table_d = table.to(device)
        out_full = out = torch.empty(n, d, dtype=dtype, device=device)
    vgo.top4_project(table_d, index.to(device), weight.to(device), out=out)
    torch.cuda.synchronize()
    got = out.cpu()
    ref = oracle.top4_project(table, index, weight)
    assert torch.isnan(got[5]).all() and torch.isfinite(got[11]).all()
    assert torch.equal(torch.nan_to_num(got), torch.nan_to_num(ref))
    assert torch.equal(got[13], table[index[13, 1].long()])
    if strided:
        assert bool((out_full[:, :64] == 3.0).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gather_probe_sums_the_projection_rows(vgo, device, dtype):
    """vgo_top4_gather_probe reads what the projection reads and writes each row's sum:
    the sums equal the projection's rows summed (fp32, within summation-order
    rounding), a poisoned row gives NaN in both, and rows of odd width are refused."""
    print(f"[project] gather probe dtype={dtype}", flush=True)
    from tests.conftest import import_package
    proj = import_package("projection")
    table, index, weight = _case(21, 5000, 700, 1024, dtype)
    index[7, 2] = 1 << 20
    td, idd, wd = table.to(device), index.to(device), weight.to(device)
    sums = proj.gather_probe(td, idd, wd)
    rows = proj.top4_project(td, idd, wd).double().sum(1)
    assert torch.isnan(sums[7]) and torch.isnan(rows[7])
    ok = ~torch.isnan(rows)
    assert torch.allclose(sums[ok].double(), rows[ok], rtol=1e-5, atol=1e-3)
    small = table[:, :23].contiguous().to(device)
    with pytest.raises(RuntimeError, match="16-byte"):
        proj.gather_probe(small, idd, wd)
