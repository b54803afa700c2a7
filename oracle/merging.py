"""Oracle: merge planners, masses, compaction and restore (test infrastructure only).

CPU restatement, in torch-CPU ops, of:
* build_fastvggt_plan          vggt_omega/models/token_merging.py:1044-1122
* TokenPlan.compact / restore  vggt_omega/models/token_merging.py:176-196
* WeightedBilinearTokenPlan.compact / restore  token_merging.py:323-414
* deterministic_weighted_normalizer            token_merging.py:40-59
* build_sparse_convex_plan + _convex_fit       vggt_omega/models/sparse_convex.py:2260-2481

Two rules are fixed here where the reference leaves them to library internals:
* scores are rounded once to bf16 from the exact dot product of the bf16
  operands (the reference rounds an fp32 accumulation whose order belongs to
  the BLAS in use), and
* top-k ties go to the lower dictionary position (the contract written in
  vggt_omega/models/sparse_convex_kernels.py:51-54, 67-84; torch.topk leaves
  tie order unspecified).
`max` already returns the first maximum and the rank uses a stable sort, as in
the reference.  Pinned by tests/golden fixtures written from the real
reference (tests/golden/make_fixtures.py) and by the invariants in
tests/test_oracle_merging.py.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

ACTIVE_SETS = torch.tensor((
    (1., 1., 1., 1.),
    (1., 1., 1., 0.), (1., 1., 0., 1.), (1., 0., 1., 1.), (0., 1., 1., 1.),
    (1., 1., 0., 0.), (1., 0., 1., 0.), (1., 0., 0., 1.),
    (0., 1., 1., 0.), (0., 1., 0., 1.), (0., 0., 1., 1.),
    (1., 0., 0., 0.), (0., 1., 0., 0.), (0., 0., 1., 0.), (0., 0., 0., 1.),
))  # the reference's active-set table, sparse_convex.py:22-28
RIDGE = 1e-4
EARLY_MARGIN = 1e-2
LOCAL_FRAME_GROUP = 8


# --------------------------------------------------------------- layout ----
def patch_ids(frames: int, tokens_per_frame: int, patch_token_start: int) -> torch.Tensor:
    patches = tokens_per_frame - patch_token_start
    return (torch.arange(frames)[:, None] * tokens_per_frame + patch_token_start
            + torch.arange(patches)[None, :])


def anchor_positions(frames: int, patch_hw: tuple[int, int], seed: int) -> torch.Tensor:
    """sparse_convex.py:2366-2371 / token_merging.py:1072-1082."""
    height, width = patch_hw
    generator = torch.Generator(device="cpu").manual_seed(seed)
    rows, cols = torch.arange(0, height, 2), torch.arange(0, width, 2)
    choice = torch.rand(frames - 1, len(rows), len(cols), 2, generator=generator)
    row = rows[None, :, None] + (choice[..., 0] * (height - rows).clamp(max=2)[None, :, None]).long()
    col = cols[None, None, :] + (choice[..., 1] * (width - cols).clamp(max=2)[None, None, :]).long()
    return (row * width + col).reshape(frames - 1, -1)


def bf16_scores(src_bf16: torch.Tensor, dst_bf16: torch.Tensor) -> torch.Tensor:
    """bf16(exact dot) of bf16 operands, returned as float32 [n_src, n_dst]."""
    exact = src_bf16.double() @ dst_bf16.double().T
    return exact.to(torch.bfloat16).float()


def topk_lowest_index(scores: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    values, index = scores.sort(dim=-1, descending=True, stable=True)
    return values[:, :k], index[:, :k]


# ------------------------------------------------------------ FastVGGT ----
def fastvggt_layout(total, frames, tokens_per_frame, patch_token_start, patch_hw,
                    protect_ratio, seed):
    """token_merging.py:1067-1095: (source ids, destination ids)."""
    ids = patch_ids(frames, tokens_per_frame, patch_token_start)
    destination = torch.zeros(total, dtype=torch.bool)
    destination[ids[0]] = True
    selected = anchor_positions(frames, patch_hw, seed)
    destination[ids[1:].gather(1, selected).flatten()] = True
    protected = torch.ones(total, dtype=torch.bool)
    protected[ids.flatten()] = False
    protected[ids[0]] = True
    count = int(total * protect_ratio)
    if count:
        protected[torch.arange(0, total, max(1, total // count))[:count]] = True
    return (~(destination | protected)).nonzero().flatten(), destination.nonzero().flatten()


def fastvggt_select(best: torch.Tensor, targets: torch.Tensor, sources: torch.Tensor,
                    destinations: torch.Tensor, total: int, removed: int):
    """token_merging.py:1112-1121 for one batch element -> (keep [K], inverse [N])."""
    ranked = best.argsort(descending=True, stable=True)
    removed_source = sources[ranked[:removed]]
    target_original = destinations[targets[ranked[:removed]]]
    kept = torch.ones(total, dtype=torch.bool)
    kept[removed_source] = False
    keep = torch.arange(total)[kept]
    original_to_compact = torch.full((total,), -1, dtype=torch.long)
    original_to_compact[keep] = torch.arange(keep.numel())
    inverse = original_to_compact.clone()
    inverse[removed_source] = original_to_compact[target_original]
    return keep, inverse


def fastvggt_plan(tokens: torch.Tensor, *, frames, tokens_per_frame, patch_token_start, patch_hw,
                  merge_ratio=0.9, protect_ratio=0.10, seed=0, scores=None):
    """token_merging.py:1044-1122 for batch 1 (tokens [1, N, C] CPU).

    Returns dict(keep, inverse, best, targets, sources, destinations, removed).
    `scores` ([n_src, n_dst] float32 of bf16 values) replaces the oracle's own
    score matrix, to check the selection logic on the exact scores a kernel saw.
    """
    total = tokens.shape[1]
    if frames == 1 or merge_ratio == 0:
        ident = torch.arange(total)
        return dict(keep=ident, inverse=ident, removed=0)
    sources, destinations = fastvggt_layout(total, frames, tokens_per_frame, patch_token_start,
                                            patch_hw, protect_ratio, seed)
    removed = min(int(total * merge_ratio), sources.numel())
    if removed == 0:
        ident = torch.arange(total)
        return dict(keep=ident, inverse=ident, removed=0)
    if scores is None:
        src = F.normalize(tokens[0, sources].float(), dim=-1).to(torch.bfloat16)
        dst = F.normalize(tokens[0, destinations].float(), dim=-1).to(torch.bfloat16)
        scores = bf16_scores(src, dst)
    best, targets = scores.max(dim=-1)
    keep, inverse = fastvggt_select(best, targets, sources, destinations, total, removed)
    return dict(keep=keep, inverse=inverse, best=best, targets=targets, sources=sources,
                destinations=destinations, removed=removed, scores=scores)


def token_plan_compact(inverse: torch.Tensor, kept: int, value: torch.Tensor) -> torch.Tensor:
    """TokenPlan.compact (token_merging.py:176-191), sums in ascending token order."""
    acc_dtype = torch.float32 if value.dtype in (torch.float16, torch.bfloat16) else value.dtype
    out = torch.zeros(kept, value.shape[-1], dtype=acc_dtype)
    counts = torch.zeros(kept, dtype=acc_dtype)
    for t in range(inverse.numel()):
        k = int(inverse[t])
        out[k] = out[k] + value[t].to(acc_dtype)
        counts[k] += 1
    return (out / counts[:, None]).to(value.dtype)


def token_plan_restore(inverse: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
    """TokenPlan.restore (token_merging.py:193-196)."""
    return value[inverse]


# ------------------------------------------- weighted bilinear plans ----
def deterministic_weighted_normalizer(parent_compact: torch.Tensor, weights: torch.Tensor,
                                      kept_tokens: int) -> torch.Tensor:
    """token_merging.py:40-59, same op sequence on the CPU."""
    mass = torch.ones((1, kept_tokens, 1), dtype=torch.float32)
    for corner in range(parent_compact.shape[-1]):
        destination = parent_compact[0, :, corner]
        order = destination.argsort(stable=True)
        lengths = torch.bincount(destination, minlength=kept_tokens).view(1, -1)
        ordered_weight = weights[0, :, corner].index_select(0, order).float().view(1, -1, 1)
        mass = mass + torch.segment_reduce(ordered_weight, reduce="sum", lengths=lengths, axis=1)
    return mass


def weighted_compact(keep, source_original, parent_compact, pool_weights, normalizer,
                     value: torch.Tensor) -> torch.Tensor:
    """WeightedBilinearTokenPlan.compact (token_merging.py:343-370), one batch element.

    value [N, C] -> [K, C]; fp32 accumulation for half inputs.
    """
    acc_dtype = torch.float32 if value.dtype in (torch.float16, torch.bfloat16) else value.dtype
    compact = value[keep.reshape(-1)].to(acc_dtype)
    src_ids = source_original.reshape(-1)
    if src_ids.numel() == 0:
        return value[keep.reshape(-1)]
    source = value[src_ids].to(acc_dtype)
    parent = parent_compact.reshape(-1, parent_compact.shape[-1])
    w = pool_weights.reshape(-1, parent.shape[-1])
    kept = compact.shape[0]
    for corner in range(parent.shape[-1]):
        order = parent[:, corner].argsort(stable=True)
        lengths = torch.bincount(parent[:, corner], minlength=kept).view(1, -1)
        ordered = source.index_select(0, order)[None] * w[:, corner].index_select(0, order).view(1, -1, 1).to(acc_dtype)
        compact = compact + torch.segment_reduce(ordered, reduce="sum", lengths=lengths, axis=1)[0]
    return (compact / normalizer.reshape(-1, 1).to(acc_dtype)).to(value.dtype)


def weighted_restore(keep, source_original, parent_compact, restore_weights, total: int,
                     value: torch.Tensor) -> torch.Tensor:
    """WeightedBilinearTokenPlan.restore (token_merging.py:403-414), value [K, C] -> [N, C]."""
    from oracle.projection import top4_project
    out = torch.zeros((total, value.shape[-1]), dtype=value.dtype)
    out[keep.reshape(-1)] = value
    src = source_original.reshape(-1)
    if src.numel():
        out[src] = top4_project(value, parent_compact.reshape(-1, 4).int(),
                                restore_weights.reshape(-1, 4).float())
    return out


# -------------------------------------------------------- sparse convex ----
def convex_fit(source: torch.Tensor, supports: torch.Tensor):
    """_convex_fit (sparse_convex.py:2260-2304), identical op sequence on the CPU."""
    source, supports = source.float(), supports.float()
    count = source.shape[0]
    gram = supports @ supports.transpose(1, 2)
    rhs = torch.bmm(supports, source.unsqueeze(-1)).squeeze(-1)
    active = ACTIVE_SETS
    pair = active[:, :, None] * active[:, None, :]
    inactive_diag = torch.diag_embed(1.0 - active)
    block = 2.0 * gram[:, None] * pair[None]
    block = block * (1.0 - inactive_diag) + inactive_diag + 2.0 * RIDGE * torch.diag_embed(active)
    matrix = torch.zeros(count, 15, 5, 5, dtype=torch.float32)
    matrix[..., :4, :4] = block
    matrix[..., :4, 4] = active
    matrix[..., 4, :4] = 1.0
    target = torch.zeros(count, 15, 5, dtype=torch.float32)
    target[..., :4] = 2.0 * rhs[:, None] * active[None]
    target[..., 4] = 1.0
    solution, info = torch.linalg.solve_ex(matrix, target)
    alpha = solution[..., :4].clamp_min(0.0)
    alpha = alpha / alpha.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    quadratic = torch.matmul(gram[:, None], alpha.unsqueeze(-1)).squeeze(-1)
    objective = (alpha * quadratic).sum(dim=-1) - 2.0 * (alpha * rhs[:, None]).sum(dim=-1)
    feasible = (info == 0) & (solution[..., :4] >= -1e-5).all(dim=-1)
    objective = torch.where(feasible, objective, torch.inf)
    best = objective.argmin(dim=-1)
    alpha = alpha.gather(1, best[:, None, None].expand(-1, 1, 4)).squeeze(1)
    numerator = (alpha * rhs).sum(dim=-1)
    squared_norm = (alpha * torch.bmm(gram, alpha.unsqueeze(-1)).squeeze(-1)).sum(dim=-1)
    cosine = numerator / squared_norm.clamp_min(1e-12).sqrt()
    single = rhs[:, 0]
    one_hot = single > cosine
    if one_hot.any():
        alpha[one_hot] = 0
        alpha[one_hot, 0] = 1
    return torch.maximum(cosine, single), alpha


def sparse_convex_layout(total, frames, tokens_per_frame, patch_token_start, patch_hw):
    height, width = patch_hw
    patches = height * width
    ids = patch_ids(frames, tokens_per_frame, patch_token_start)
    frame0 = ids[0]
    if frames == 1:
        return dict(ids=ids, frame0=frame0, candidate=torch.empty(0, dtype=torch.long),
                    destination=frame0, groups=[], per_frame=0)
    anchor_position = anchor_positions(frames, patch_hw, 0)
    anchor_ids = ids[1:].gather(1, anchor_position)
    mask = torch.ones((frames - 1, patches), dtype=torch.bool)
    mask.scatter_(1, anchor_position, False)
    candidate_position = torch.arange(patches).expand(frames - 1, patches)[mask].reshape(frames - 1, -1)
    candidate = ids[1:].gather(1, candidate_position).flatten()
    destination = torch.cat((frame0, anchor_ids.flatten()))
    groups = []
    for begin in range(1, frames, LOCAL_FRAME_GROUP):
        end = min(begin + LOCAL_FRAME_GROUP, frames)
        anchor_begin = max(begin - 2, 0)
        anchor_end = min(end - 1, frames - 2) + 1
        local = torch.cat((frame0, anchor_ids[anchor_begin:anchor_end].flatten()))
        groups.append((begin, end, local))
    return dict(ids=ids, frame0=frame0, candidate=candidate, destination=destination,
                groups=groups, per_frame=candidate_position.shape[1],
                candidate_position=candidate_position)


def sparse_convex_plan(tokens: torch.Tensor, *, frames, tokens_per_frame, patch_token_start,
                       patch_hw, threshold=0.90):
    """build_sparse_convex_plan (sparse_convex.py:2343-2481) on the CPU, batch 1.

    Returns dict of the plan fields plus intermediates (support, top1, fit, alpha,
    hard, failed).  Mass uses the deterministic normalizer order.
    """
    total = tokens.shape[1]
    lay = sparse_convex_layout(total, frames, tokens_per_frame, patch_token_start, patch_hw)
    candidate, destination = lay["candidate"], lay["destination"]
    normalized = F.normalize(tokens[0].float(), dim=-1, eps=1e-6)
    count = candidate.numel()
    support = torch.empty((count, 4), dtype=torch.long)
    top1 = torch.empty(count, dtype=torch.float32)
    per_frame = lay["per_frame"]
    for begin, end, local in lay["groups"]:
        positions = lay["candidate_position"][begin - 1:end - 1]
        source_ids = lay["ids"][begin:end].gather(1, positions).flatten()
        scores = bf16_scores(normalized[source_ids].to(torch.bfloat16), normalized[local].to(torch.bfloat16))
        value, local_index = topk_lowest_index(scores, 4)
        offset = (begin - 1) * per_frame
        support[offset:offset + source_ids.numel()] = local[local_index]
        top1[offset:offset + source_ids.numel()] = value[:, 0]
    fit = torch.empty(count, dtype=torch.float32)
    alpha = torch.zeros((count, 4), dtype=torch.float32)
    easy = top1 >= threshold + EARLY_MARGIN
    hard = (~easy).nonzero().flatten()
    alpha[easy, 0] = 1.0
    fit[easy] = top1[easy]
    if hard.numel():
        source = F.normalize(normalized[candidate[hard]], dim=-1, eps=1e-6)
        parent_feature = F.normalize(normalized[support[hard]], dim=-1, eps=1e-6)
        fit[hard], alpha[hard] = convex_fit(source, parent_feature)
    failed = hard[fit[hard] < threshold]
    if failed.numel():
        dictionary = normalized[destination].to(torch.bfloat16)
        source = normalized[candidate[failed]]
        scores = bf16_scores(source.to(torch.bfloat16), dictionary)
        _, local = topk_lowest_index(scores, 4)
        support[failed] = destination[local]
        source = F.normalize(source, dim=-1, eps=1e-6)
        parent_feature = F.normalize(normalized[support[failed]], dim=-1, eps=1e-6)
        fit[failed], alpha[failed] = convex_fit(source, parent_feature)
    selected = fit >= threshold
    source_original = candidate[selected]
    source_support = support[selected]
    weights = alpha[selected]
    kept_mask = torch.ones(total, dtype=torch.bool)
    kept_mask[source_original] = False
    keep = torch.arange(total)[kept_mask]
    original_to_compact = torch.full((total,), -1, dtype=torch.long)
    original_to_compact[keep] = torch.arange(keep.numel())
    parent_compact = original_to_compact[source_support]
    assert (parent_compact >= 0).all()
    mass = deterministic_weighted_normalizer(parent_compact[None], weights[None], keep.numel())
    special_original = (torch.arange(frames)[:, None] * tokens_per_frame
                        + torch.arange(patch_token_start)[None, :]).flatten()
    return dict(keep=keep, source_original=source_original, parent_compact=parent_compact,
                weights=weights, mass=mass.reshape(-1), key_log_mass=mass.reshape(-1).log(),
                special_original=special_original,
                special_compact=original_to_compact[special_original],
                original_to_compact=original_to_compact, support=support, top1=top1, fit=fit,
                alpha=alpha, hard=hard, failed=failed, candidate=candidate,
                destination=destination)

