"""Oracle: four-variable simplex least-squares solvers (test infrastructure only).

Restates, vectorised over rows in float64 (or the dtype given):

* `four_support_active_set` -- vggt_omega/models/sparse_convex_kernels.py:
  102-180 (one candidate per active set of the table at :316-323: eliminate the
  last active variable p through sum-to-one, solve the 1x1/2x2/3x3 reduced
  system on G + ridge I by Cramer's rule, |det| <= 1e-12 is unstable, weights
  below -1e-5 infeasible, clamp and renormalise, objective a^T G a - 2 r^T a
  on G without the ridge) and :183-212 (argmin with the first index on ties,
  renormalise, one-hot (1,0,0,0) when r_0 exceeds the fit's cosine); wrapper
  :332-353.
* `four_support_projected_gradient` -- :214-280 (step 0.95 / max(max row L1
  norm, 1e-4), `steps` gradient steps from (1,0,0,0), each followed by the
  simplex projection whose threshold comes from a four-value sorting
  network); wrapper :283-296.

Pinned in tests/test_oracle_simplex.py against mathematics the code does not
share: the textbook sort-and-threshold simplex projection, KKT conditions of
the simplex-constrained quadratic program, a dense random search of the
simplex, and the two solvers against each other.
"""
from __future__ import annotations

import torch

# Active sets in the reference's table order (sparse_convex_kernels.py:316-323).
ACTIVE_IDS = (
    (0, 0, 0, 0), (1, 1, 1, 1), (2, 2, 2, 2), (3, 3, 3, 3),
    (0, 1, 1, 1), (0, 2, 2, 2), (0, 3, 3, 3),
    (1, 2, 2, 2), (1, 3, 3, 3), (2, 3, 3, 3),
    (0, 1, 2, 2), (0, 1, 3, 3), (0, 2, 3, 3), (1, 2, 3, 3),
    (0, 1, 2, 3),
)
ACTIVE_COUNT = (1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 3, 3, 3, 3, 4)


def active_set_candidates(gram: torch.Tensor, rhs: torch.Tensor, ridge: float = 1e-4,
                          dtype: torch.dtype = torch.float64) -> tuple[torch.Tensor, torch.Tensor]:
    """Candidates [N,15,4] and objectives [N,15] (inf where infeasible)."""
    g = gram.to(dtype)
    r = rhs.to(dtype)
    eye = torch.eye(4, dtype=dtype)
    gr = g + ridge * eye

    def ge(a: int, b: int) -> torch.Tensor:
        return gr[:, a, b]

    cands, objs = [], []
    for ids, count in zip(ACTIVE_IDS, ACTIVE_COUNT):
        i0, i1, i2 = ids[0], ids[1], ids[2]
        p = ids[count - 1]
        hp = ge(p, p)
        rp = r[:, p]
        h = [[ge(a, b) - ge(a, p) - ge(p, b) + hp for b in (i0, i1, i2)] for a in (i0, i1, i2)]
        c = [r[:, a] - rp - ge(a, p) + hp for a in (i0, i1, i2)]
        dim = count - 1
        zero = torch.zeros_like(hp)
        b = [zero, zero, zero]
        if dim == 0:
            stable = torch.ones_like(hp, dtype=torch.bool)
        elif dim == 1:
            stable = h[0][0].abs() > 1e-12
            b = [c[0] / torch.where(stable, h[0][0], torch.ones_like(hp)), zero, zero]
        elif dim == 2:
            det = h[0][0] * h[1][1] - h[0][1] * h[1][0]
            stable = det.abs() > 1e-12
            d = torch.where(stable, det, torch.ones_like(hp))
            b = [(c[0] * h[1][1] - h[0][1] * c[1]) / d, (h[0][0] * c[1] - h[1][0] * c[0]) / d, zero]
        else:
            m = torch.stack([torch.stack(row, -1) for row in h], -2)     # [N,3,3]
            det = torch.linalg.det(m) if dtype == torch.float64 else (
                h[0][0] * (h[1][1] * h[2][2] - h[1][2] * h[2][1])
                - h[0][1] * (h[1][0] * h[2][2] - h[1][2] * h[2][0])
                + h[0][2] * (h[1][0] * h[2][1] - h[1][1] * h[2][0]))
            stable = det.abs() > 1e-12
            d = torch.where(stable, det, torch.ones_like(hp))
            cv = torch.stack(c, -1)
            b = []
            for col in range(3):  # Cramer's rule
                mc = m.clone()
                mc[:, :, col] = cv
                b.append(torch.linalg.det(mc) / d)
        ap = 1.0 - b[0] - b[1] - b[2]
        alpha = torch.zeros(len(g), 4, dtype=dtype)
        for var in range(4):
            alpha[:, var] = ((b[0] if i0 == var else 0.0) + (b[1] if i1 == var else 0.0)
                             + (b[2] if i2 == var else 0.0) + (ap if p == var else 0.0))
        feasible = stable & (alpha >= -1e-5).all(-1)
        alpha = alpha.clamp_min(0.0)
        alpha = alpha / alpha.sum(-1, keepdim=True).clamp_min(1e-12)
        obj = torch.einsum("ni,nij,nj->n", alpha, g, alpha) - 2.0 * (alpha * r).sum(-1)
        objs.append(torch.where(feasible, obj, torch.full_like(obj, float("inf"))))
        cands.append(alpha)
    return torch.stack(cands, 1), torch.stack(objs, 1)


def select_candidate(cands: torch.Tensor, objs: torch.Tensor, gram: torch.Tensor,
                     rhs: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Reference :183-212.  Returns alpha [N,4] and the one-hot flag [N]."""
    dtype = cands.dtype
    best = torch.argmin(objs, dim=1)                # first minimal index
    alpha = cands[torch.arange(len(cands)), best]
    alpha = alpha / alpha.sum(-1, keepdim=True).clamp_min(1e-12)
    g = gram.to(dtype)
    r = rhs.to(dtype)
    quadratic = torch.einsum("nij,nj->ni", g, alpha)
    cosine = (alpha * r).sum(-1) / (alpha * quadratic).sum(-1).clamp_min(1e-12).sqrt()
    one_hot = r[:, 0] > cosine
    alpha = torch.where(one_hot[:, None], torch.tensor([1.0, 0.0, 0.0, 0.0], dtype=dtype), alpha)
    return alpha, one_hot


def four_support_active_set(gram: torch.Tensor, rhs: torch.Tensor, ridge: float = 1e-4,
                            dtype: torch.dtype = torch.float64) -> torch.Tensor:
    cands, objs = active_set_candidates(gram, rhs, ridge, dtype)
    return select_candidate(cands, objs, gram, rhs)[0]


def project_simplex_network(p: torch.Tensor) -> torch.Tensor:
    """The projection step of :254-275 (threshold from a sorting network)."""
    p0, p1, p2, p3 = p.unbind(-1)
    s0, s1 = torch.maximum(p0, p1), torch.minimum(p0, p1)
    s2, s3 = torch.maximum(p2, p3), torch.minimum(p2, p3)
    s0, s2 = torch.maximum(s0, s2), torch.minimum(s0, s2)
    s1, s3 = torch.maximum(s1, s3), torch.minimum(s1, s3)
    s1, s2 = torch.maximum(s1, s2), torch.minimum(s1, s2)
    theta = s0 - 1.0
    theta2 = (s0 + s1 - 1.0) * 0.5
    theta = torch.where(s1 > theta2, theta2, theta)
    theta3 = (s0 + s1 + s2 - 1.0) / 3.0
    theta = torch.where(s2 > theta3, theta3, theta)
    theta4 = (s0 + s1 + s2 + s3 - 1.0) * 0.25
    theta = torch.where(s3 > theta4, theta4, theta)
    return (p - theta[..., None]).clamp_min(0.0)


def four_support_projected_gradient(gram: torch.Tensor, rhs: torch.Tensor, steps: int = 32,
                                    dtype: torch.dtype = torch.float64) -> torch.Tensor:
    g = gram.to(dtype)
    r = rhs.to(dtype)
    lipschitz = g.abs().sum(-1).amax(-1)
    step = 0.95 / lipschitz.clamp_min(1e-4)
    alpha = torch.zeros(len(g), 4, dtype=dtype)
    alpha[:, 0] = 1.0
    for _ in range(steps):
        grad = torch.einsum("nij,nj->ni", g, alpha) - r
        alpha = project_simplex_network(alpha - step[:, None] * grad)
    return alpha


def objective(gram: torch.Tensor, rhs: torch.Tensor, alpha: torch.Tensor, ridge: float = 0.0) -> torch.Tensor:
    """a^T (G + ridge I) a - 2 r^T a per row, float64."""
    g = gram.double() + ridge * torch.eye(4, dtype=torch.float64)
    a = alpha.double()
    return torch.einsum("ni,nij,nj->n", a, g, a) - 2.0 * (a * rhs.double()).sum(-1)
