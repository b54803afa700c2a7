"""GPU parity of the four-support simplex solvers against the CPU oracle.

The kernels compute in fp32 and the oracle in fp64, so weights are compared
to tolerance.  The active-set solver also makes two discrete choices (the
candidate with the lowest objective, and the one-hot override); on rows where
the oracle's choice is decided by less than fp32 rounding, the test requires
only that the kernel's weights be as good (objective within tolerance of the
oracle's) rather than identical.
"""
from __future__ import annotations

import pytest
import torch

from oracle import simplex as oracle
from tests.conftest import import_package
from tests.test_oracle_simplex import _problems

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sck():
    return import_package("sparse_convex_kernels")


def _edge_rows():
    """Degenerate inputs: identical supports, zero problems, scaled problems."""
    ones = torch.ones(4, 4, dtype=torch.float64)
    eye = torch.eye(4, dtype=torch.float64)
    gram = torch.stack([ones, ones, eye, eye * 1e3, torch.zeros(4, 4, dtype=torch.float64), eye])
    rhs = torch.tensor([[0.5, 0.5, 0.5, 0.5], [1.0, 0.2, 0.2, 0.2], [0.9, 0.1, 0.0, -0.3],
                        [10.0, 20.0, -5.0, 0.0], [0.0, 0.0, 0.0, 0.0], [0.3, 0.3, 0.3, 0.3]],
                       dtype=torch.float64)
    return gram, rhs


@pytest.mark.parametrize("steps", [0, 1, 32, 200])
def test_projected_gradient_matches_oracle(sck, device, steps):
    print(f"[simplex] projected gradient steps={steps}", flush=True)
    gram, rhs, _, _ = _problems(50000, 11, correlated=1.0)
    eg, er = _edge_rows()
    gram, rhs = torch.cat([gram, eg]), torch.cat([rhs, er])
    out = sck.four_support_projected_gradient(gram.float().to(device), rhs.float().to(device), steps=steps)
    torch.cuda.synchronize()
    ref = oracle.four_support_projected_gradient(gram.float(), rhs.float(), steps=steps)
    assert out.shape == rhs.shape and out.dtype == torch.float32
    err = (out.cpu().double() - ref).abs().amax().item()
    assert err <= 2e-5, f"projected gradient max abs error {err:.3e}"
    assert torch.allclose(out.cpu().double().sum(-1), torch.ones(len(rhs), dtype=torch.float64), atol=1e-5)


@pytest.mark.parametrize("correlated", [0.0, 2.0])
def test_active_set_matches_oracle(sck, device, correlated):
    print(f"[simplex] active set correlated={correlated}", flush=True)
    gram, rhs, _, _ = _problems(50000, 12, correlated=correlated)
    eg, er = _edge_rows()
    gram, rhs = torch.cat([gram, eg]), torch.cat([rhs, er])
    g32, r32 = gram.float(), rhs.float()
    out = sck.four_support_active_set(g32.to(device), r32.to(device), ridge=1e-4).cpu().double()
    torch.cuda.synchronize()
    cands, objs = oracle.active_set_candidates(g32, r32, 1e-4)
    ref, one_hot = oracle.select_candidate(cands, objs, g32, r32)
    # Rows whose decisions are clear of fp32 rounding must match to tolerance.
    srt, _ = torch.sort(objs, dim=1)
    gap = srt[:, 1] - srt[:, 0]
    fit = cands[torch.arange(len(cands)), torch.argmin(objs, 1)]
    fit = fit / fit.sum(-1, keepdim=True)
    quad = torch.einsum("nij,nj->ni", g32.double(), fit)
    cosine = (fit * r32.double()).sum(-1) / (fit * quad).sum(-1).clamp_min(1e-12).sqrt()
    clear = (gap > 1e-5 * (1.0 + srt[:, 0].abs())) & ((r32[:, 0].double() - cosine).abs() > 1e-5)
    assert clear.float().mean() > 0.95
    err = (out[clear] - ref[clear]).abs().amax().item()
    assert err <= 1e-4, f"active set max abs error {err:.3e} on {int(clear.sum())} clear rows"
    # Elsewhere the kernel's weights must be as good as the oracle's.
    close = ~clear
    if close.any():
        o_k = oracle.objective(g32[close], r32[close], out[close])
        o_r = oracle.objective(g32[close], r32[close], ref[close])
        one = one_hot[close] | (out[close, 0] == 1.0)
        ok = one | (o_k <= o_r + 1e-5 * (1.0 + o_r.abs()))
        assert ok.all()
    assert torch.allclose(out.sum(-1), torch.ones(len(out), dtype=torch.float64), atol=1e-5)
    assert (out >= 0).all()


def test_errors_match_reference(sck, device):
    g = torch.zeros(3, 4, 4, device=device)
    with pytest.raises(ValueError, match=r"\[N,4,4\] Gram and \[N,4\] rhs"):
        sck.four_support_active_set(g, torch.zeros(3, 3, device=device))
    with pytest.raises(ValueError, match=r"\[N,4,4\] Gram and \[N,4\] rhs"):
        sck.four_support_projected_gradient(torch.zeros(3, 4, 3, device=device), torch.zeros(3, 4, device=device))
    with pytest.raises(RuntimeError):
        sck.four_support_active_set(torch.zeros(3, 4, 4), torch.zeros(3, 4))
    with pytest.raises(RuntimeError):
        sck.four_support_projected_gradient(torch.zeros(3, 4, 4), torch.zeros(3, 4))
    # Empty inputs and non-contiguous / non-fp32 inputs follow the reference's casts.
    assert sck.four_support_active_set(torch.zeros(0, 4, 4, device=device), torch.zeros(0, 4, device=device)).shape == (0, 4)
    gram, rhs, _, _ = _problems(64, 13)
    gt = gram.to(device).half().transpose(1, 2)   # symmetric, so the values are unchanged
    out = sck.four_support_projected_gradient(gt, rhs.to(device).half(), steps=32)
    ref = oracle.four_support_projected_gradient(gram.half().float(), rhs.half().float(), steps=32)
    assert (out.cpu().double() - ref).abs().amax() <= 2e-5
