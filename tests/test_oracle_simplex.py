"""Pins the simplex-solver oracle (oracle/simplex.py) with mathematics it does not share.

* The sorting-network projection equals the textbook sort-and-threshold
  Euclidean projection onto the probability simplex.
* The active-set candidate with the lowest objective is the minimiser of the
  simplex-constrained quadratic program: it satisfies the KKT conditions, no
  point of a dense random search of the simplex beats it, and the
  projected-gradient iteration run to convergence reaches the same point.
* The one-hot override follows the cosine of the reconstruction computed from
  the underlying vectors.
"""
from __future__ import annotations

import pytest
import torch

from oracle import simplex as oracle


def _problems(n: int, seed: int, dim: int = 64, correlated: float = 0.0):
    """Gram/rhs of unit supports S [n,4,dim] and a unit source x [n,dim]."""
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(n, 1, dim, generator=g, dtype=torch.float64)
    s = torch.randn(n, 4, dim, generator=g, dtype=torch.float64) + correlated * base
    s = s / s.norm(dim=-1, keepdim=True)
    x = s[:, 0] * 0.6 + 0.4 * torch.randn(n, dim, generator=g, dtype=torch.float64)
    x = x / x.norm(dim=-1, keepdim=True)
    gram = s @ s.transpose(1, 2)
    rhs = (s @ x.unsqueeze(-1)).squeeze(-1)
    return gram, rhs, s, x


def _textbook_projection(p: torch.Tensor) -> torch.Tensor:
    """Sort, find the last k with u_k > (sum_{j<=k} u_j - 1) / k, shift and clip."""
    u, _ = torch.sort(p, dim=-1, descending=True)
    css = u.cumsum(-1)
    k = torch.arange(1, p.shape[-1] + 1, dtype=p.dtype)
    cond = u - (css - 1.0) / k > 0
    kk = (cond * k).amax(-1)                       # largest k meeting the condition
    theta = (css.gather(-1, (kk.long() - 1)[..., None])[..., 0] - 1.0) / kk
    return (p - theta[..., None]).clamp_min(0.0)


def test_projection_is_the_euclidean_simplex_projection():
    g = torch.Generator().manual_seed(1)
    p = torch.randn(20000, 4, generator=g, dtype=torch.float64) * torch.tensor([0.3, 1.0, 3.0, 10.0])[
        torch.randint(0, 4, (20000, 1), generator=g)]
    special = torch.tensor([[0.25, 0.25, 0.25, 0.25], [1.0, 1.0, 1.0, 1.0], [5.0, -5.0, 5.0, -5.0],
                            [0.0, 0.0, 0.0, 0.0], [1.0, 0.0, 0.0, 0.0], [-3.0, -2.0, -1.0, -0.5],
                            [0.7, 0.7, -0.1, 0.3]], dtype=torch.float64)
    p = torch.cat([p, special])
    net = oracle.project_simplex_network(p)
    ref = _textbook_projection(p)
    assert torch.allclose(net, ref, atol=1e-12, rtol=0)
    assert torch.allclose(net.sum(-1), torch.ones(len(p), dtype=torch.float64), atol=1e-12)
    assert (net >= 0).all()
    # A projection is idempotent and no simplex point is closer to p.
    assert torch.allclose(oracle.project_simplex_network(net), net, atol=1e-12)
    w = torch.distributions.Dirichlet(torch.ones(4, dtype=torch.float64)).sample((len(p),))
    assert ((p - net).norm(dim=-1) <= (p - w).norm(dim=-1) + 1e-12).all()


def _best_candidate(cands, objs):
    best = torch.argmin(objs, dim=1)
    alpha = cands[torch.arange(len(cands)), best]
    return alpha / alpha.sum(-1, keepdim=True).clamp_min(1e-12), objs[torch.arange(len(objs)), best]


@pytest.mark.parametrize("correlated", [0.0, 1.5])
def test_active_set_minimises_the_qp(correlated):
    gram, rhs, _, _ = _problems(3000, 2, correlated=correlated)
    ridge = 0.0
    cands, objs = oracle.active_set_candidates(gram, rhs, ridge)
    alpha, best_obj = _best_candidate(cands, objs)
    assert torch.isfinite(best_obj).all()
    # KKT of min a^T G a - 2 r^T a on the simplex: equal gradient on the support,
    # no smaller gradient off it.
    grad = 2.0 * torch.einsum("nij,nj->ni", gram, alpha) - 2.0 * rhs
    support = alpha > 1e-9
    lam = (grad * support).sum(-1) / support.sum(-1)
    spread = ((grad - lam[:, None]).abs() * support).amax(-1)
    assert (spread < 1e-8).all()
    assert ((grad - lam[:, None])[~support] > -1e-8).all()
    # Dense random search of the simplex never beats it.
    w = torch.distributions.Dirichlet(torch.full((4,), 0.5, dtype=torch.float64)).sample((3000, 64))
    vals = torch.einsum("nki,nij,nkj->nk", w, gram, w) - 2.0 * torch.einsum("nki,ni->nk", w, rhs)
    assert (vals.amin(-1) >= best_obj - 1e-10).all()


def test_projected_gradient_converges_to_the_active_set_solution():
    gram, rhs, _, _ = _problems(500, 3)
    cands, objs = oracle.active_set_candidates(gram, rhs, 0.0)
    exact, _ = _best_candidate(cands, objs)
    pg = oracle.four_support_projected_gradient(gram, rhs, steps=20000)
    assert torch.allclose(pg, exact, atol=1e-6, rtol=0)


def test_ridge_moves_the_solution_by_at_most_the_ridge_term():
    gram, rhs, _, _ = _problems(1000, 4, correlated=1.0)
    a0, o0 = _best_candidate(*oracle.active_set_candidates(gram, rhs, 0.0))
    a1, _ = _best_candidate(*oracle.active_set_candidates(gram, rhs, 1e-4))
    # The ridged optimum is within ridge * |a|^2 <= 1e-4 of the exact objective.
    assert (oracle.objective(gram, rhs, a1) - o0 <= 1e-4 + 1e-12).all()


def test_one_hot_override_uses_the_reconstruction_cosine():
    gram, rhs, s, x = _problems(4000, 5, correlated=2.0)
    cands, objs = oracle.active_set_candidates(gram, rhs, 1e-4)
    alpha, one_hot = oracle.select_candidate(cands, objs, gram, rhs)
    fit, _ = _best_candidate(cands, objs)
    recon = torch.einsum("nk,nkd->nd", fit, s)
    cosine = (recon * x).sum(-1) / recon.norm(dim=-1)
    expect = rhs[:, 0] > cosine
    margin = (rhs[:, 0] - cosine).abs() > 1e-12
    assert torch.equal(one_hot[margin], expect[margin])
    assert one_hot.any() and (~one_hot).any()
    e0 = torch.tensor([1.0, 0.0, 0.0, 0.0], dtype=torch.float64)
    assert (alpha[one_hot] == e0).all()
    assert torch.allclose(alpha[~one_hot], fit[~one_hot])


def test_singular_gram_stays_finite():
    # Identical supports: G is all ones; the ridge keeps every reduced system solvable.
    gram = torch.ones(3, 4, 4, dtype=torch.float64)
    rhs = torch.tensor([[0.5, 0.5, 0.5, 0.5], [1.0, 1.0, 1.0, 1.0], [0.0, 0.0, 0.0, 0.0]], dtype=torch.float64)
    alpha = oracle.four_support_active_set(gram, rhs, 1e-4)
    assert torch.isfinite(alpha).all()
    assert torch.allclose(alpha.sum(-1), torch.ones(3, dtype=torch.float64))
    pg = oracle.four_support_projected_gradient(gram, rhs, steps=32)
    assert torch.isfinite(pg).all() and torch.allclose(pg.sum(-1), torch.ones(3, dtype=torch.float64))
