"""Sparse-convex ("fixed_topology") merge planner on gfx950.

Drop-in for `build_sparse_convex_plan` (reference
vggt_omega/models/sparse_convex.py:2343-2481), returning the same
`WeightedBilinearTokenPlan`.  Pipeline, all in the HIP library:

1. `vgo_normalize_rows`   candidates and destinations -> bf16 (eps 1e-6)
2. `vgo_similarity_topk`  local top-4 per 8-frame group against frame-0
                          patches + the anchors of frames [begin-2, end-1)
3. `vgo_convex_fit`       easy accept (top1 >= threshold + 0.01) or the exact
                          15-active-set simplex fit
4. `vgo_failed_rows`      hard rows whose fit is below the threshold
5. `vgo_similarity_topk`  global top-4 of those rows against all destinations
   `vgo_convex_fit`       refit with the new supports (device-side row count)
6. `vgo_sparse_convex_assemble`  selection, keep, compact ids, parents, weights
7. plan CSR + `vgo_segment_mass`  deterministic mass and log-mass

One 16-byte device->host copy (the number of merged sources and three
statistics) sizes the plan; the reference synchronises several times instead.
Ties in the bf16 top-4 go to the lower dictionary position (the contract of the
reference's `_streaming_top4_kernel`); `torch.topk` leaves tie order open.
"""
from __future__ import annotations

import functools

import torch

from . import _kernels, _lib
from .token_merging import (
    FAST_MATCH_SOURCE_CHUNK,
    WeightedBilinearTokenPlan,
    _patch_ids,
    _two_by_two_anchor_positions,
    deterministic_weighted_normalizer,
)

_RIDGE = 1e-4
_EARLY_MARGIN = 1e-2
_LOCAL_FRAME_GROUP = 8
_NORMALIZE_EPS = 1e-6

__all__ = ["build_sparse_convex_plan", "convex_fit", "deterministic_weighted_normalizer"]


@functools.lru_cache(maxsize=64)
def _layout(total: int, frames: int, tokens_per_frame: int, patch_token_start: int,
            patch_hw: tuple[int, int], device: torch.device):
    """Layout-only index lists (reference :2359-2382), built once per shape on the host."""
    height, width = patch_hw
    patches = height * width
    ids = _patch_ids(frames, tokens_per_frame, patch_token_start)
    frame0 = ids[0]
    special = (torch.arange(frames)[:, None] * tokens_per_frame
               + torch.arange(patch_token_start)[None, :]).flatten()
    if frames == 1:
        empty = torch.empty(0, dtype=torch.int64)
        return dict(candidate=empty.to(device), destination=frame0.to(device), groups=(),
                    special=special.to(device), per_frame=0, anchors=0, frame0=patches)
    anchor_position = _two_by_two_anchor_positions(frames, patch_hw, 0)
    anchor_ids = ids[1:].gather(1, anchor_position)
    candidate_mask = torch.ones((frames - 1, patches), dtype=torch.bool)
    candidate_mask.scatter_(1, anchor_position, False)
    candidate_position = torch.arange(patches).expand(frames - 1, patches)[candidate_mask]
    candidate_position = candidate_position.reshape(frames - 1, -1)
    candidate = ids[1:].gather(1, candidate_position).flatten()
    destination = torch.cat((frame0, anchor_ids.flatten()))
    per_frame = candidate_position.shape[1]
    anchors = anchor_ids.shape[1]
    groups = []
    for begin in range(1, frames, _LOCAL_FRAME_GROUP):
        end = min(begin + _LOCAL_FRAME_GROUP, frames)
        anchor_begin = max(begin - 2, 0)
        anchor_end = min(end - 1, frames - 2) + 1
        # Local dictionary = destination[0:patches] + destination[patches + ab*A : patches + ae*A].
        groups.append(((begin - 1) * per_frame, (end - 1) * per_frame,
                       patches + anchor_begin * anchors, (anchor_end - anchor_begin) * anchors))
    return dict(candidate=candidate.to(device), destination=destination.to(device),
                groups=tuple(groups), special=special.to(device), per_frame=per_frame,
                anchors=anchors, frame0=patches)


def convex_fit(tokens: torch.Tensor, rows: torch.Tensor, supports: torch.Tensor, *,
               top1: torch.Tensor | None = None, easy_threshold: float = 2.0,
               row_list: torch.Tensor | None = None, n_list: torch.Tensor | None = None,
               list_supports: torch.Tensor | None = None,
               fit: torch.Tensor | None = None, alpha: torch.Tensor | None = None,
               eps: float = _NORMALIZE_EPS) -> tuple[torch.Tensor, torch.Tensor]:
    """Exact four-support simplex fit of token rows against four support rows.

    Equivalent of `_convex_fit(F.normalize(F.normalize(tokens[rows])),
    F.normalize(F.normalize(tokens[supports])))` (reference :2260-2304,
    :2421-2423) returning (fit [n], alpha [n,4]).  `top1 >= easy_threshold`
    rows keep the one-hot fit; `row_list`/`n_list` restrict the solve to a
    device-side list of rows, writing into the given `fit`/`alpha`; with
    `list_supports` ([n, 4], indexed by list position) those rows are solved
    against, and `supports` updated with, the listed supports.
    """
    lib = _lib.load()
    _lib.require_gpu(tokens, rows, supports, top1, row_list, n_list)
    if tokens.ndim != 2 or tokens.stride(-1) != 1:
        raise ValueError("convex_fit needs a [tokens, dim] matrix with unit channel stride")
    n = rows.numel()
    rows = rows.to(torch.int64).contiguous()
    if supports.dtype != torch.int64 or not supports.is_contiguous():
        raise ValueError("supports must be a contiguous int64 [n, 4] tensor (updated in place)")
    if list_supports is not None:
        list_supports = list_supports.to(torch.int64).contiguous()
    if fit is None:
        fit = torch.empty(n, device=tokens.device, dtype=torch.float32)
    if alpha is None:
        alpha = torch.empty((n, 4), device=tokens.device, dtype=torch.float32)
    status = lib.vgo_convex_fit(
        tokens.data_ptr(), tokens.stride(0), tokens.shape[0], _lib.dtype_code(tokens.dtype),
        rows.data_ptr(), supports.data_ptr(),
        None if list_supports is None else list_supports.data_ptr(),
        None if top1 is None else top1.data_ptr(),
        float(easy_threshold), None if row_list is None else row_list.data_ptr(),
        None if n_list is None else n_list.data_ptr(), n, tokens.shape[1], float(eps),
        float(_RIDGE), fit.data_ptr(), alpha.data_ptr(), _lib.stream_of(tokens))
    _lib.check(status)
    return fit, alpha


class PendingSparseConvexPlan:
    """A sparse-convex plan whose kernels are enqueued and whose size is on its way.

    The plan's shapes depend on how many candidates merged, a count the
    assemble kernel leaves on the device.  It travels to pinned host memory by
    an asynchronous copy; `result()` waits for that copy alone (an event right
    after it), so work enqueued on the stream in between -- the block's qkv
    projection, say -- keeps the GPU busy while the host sizes the plan."""

    def __init__(self, finish, stats_host: torch.Tensor, event: torch.cuda.Event):
        self._finish, self._stats_host, self._event = finish, stats_host, event
        self._plan = None

    def result(self) -> WeightedBilinearTokenPlan:
        if self._plan is None:
            self._event.synchronize()
            self._plan = self._finish(self._stats_host)
        return self._plan


@torch.no_grad()
def build_sparse_convex_plan(
    tokens: torch.Tensor, *, frames: int, tokens_per_frame: int,
    patch_token_start: int, patch_hw: tuple[int, int], threshold: float = .90,
    preserve_queries: bool = False, match_chunk_size: int = FAST_MATCH_SOURCE_CHUNK,
    fit_chunk_size: int = 16384, preserve_destination_keys: bool | None = None,
) -> WeightedBilinearTokenPlan:
    """Fixed-topology sparse-convex plan (reference sparse_convex.py:2343-2481).

    `match_chunk_size` / `fit_chunk_size` are accepted for signature
    compatibility; the HIP kernels stream without chunk loops.
    """
    return start_sparse_convex_plan(
        tokens, frames=frames, tokens_per_frame=tokens_per_frame,
        patch_token_start=patch_token_start, patch_hw=patch_hw, threshold=threshold,
        preserve_queries=preserve_queries, match_chunk_size=match_chunk_size,
        fit_chunk_size=fit_chunk_size, preserve_destination_keys=preserve_destination_keys).result()


@torch.no_grad()
def start_sparse_convex_plan(
    tokens: torch.Tensor, *, frames: int, tokens_per_frame: int,
    patch_token_start: int, patch_hw: tuple[int, int], threshold: float = .90,
    preserve_queries: bool = False, match_chunk_size: int = FAST_MATCH_SOURCE_CHUNK,
    fit_chunk_size: int = 16384, preserve_destination_keys: bool | None = None,
) -> PendingSparseConvexPlan:
    """build_sparse_convex_plan without waiting: enqueues every kernel of the plan and an
    asynchronous copy of its four counts, and returns before the host has them."""
    del match_chunk_size, fit_chunk_size
    if tokens.shape[0] != 1:
        raise ValueError("sparse-convex compaction currently supports batch size one")
    _, total, _ = tokens.shape
    height, width = patch_hw
    patches = height * width
    if total != frames * tokens_per_frame or patch_token_start + patches != tokens_per_frame:
        raise ValueError("invalid frame/token layout for sparse-convex compaction")
    if not tokens.is_cuda:
        raise RuntimeError("vgo kernels run on the GPU only; got a CPU tensor")
    lib = _lib.load()
    device = tokens.device
    stream = _lib.stream_of(tokens)
    lay = _layout(total, frames, tokens_per_frame, patch_token_start, tuple(patch_hw), device)
    x = tokens[0] if tokens[0].stride(-1) == 1 else tokens[0].contiguous()
    candidate, destination = lay["candidate"], lay["destination"]
    n_cand = candidate.numel()
    easy_threshold = threshold + _EARLY_MARGIN

    support = torch.empty((n_cand, 4), device=device, dtype=torch.int64)
    top1 = torch.empty(n_cand, device=device, dtype=torch.float32)
    fit = torch.empty(n_cand, device=device, dtype=torch.float32)
    alpha = torch.empty((n_cand, 4), device=device, dtype=torch.float32)
    failed_list = torch.empty(max(n_cand, 1), device=device, dtype=torch.int32)
    failed_count = torch.zeros(1, device=device, dtype=torch.int32)
    if n_cand:
        cand_bf16 = _kernels.normalize_rows(x, candidate, _NORMALIZE_EPS)
        dest_bf16 = _kernels.normalize_rows(x, destination, _NORMALIZE_EPS)
        for c0, c1, off1, n_anchor in lay["groups"]:
            values, index = _kernels.similarity_topk(
                cand_bf16[c0:c1], dest_bf16, 4,
                dict_ranges=(lay["frame0"], off1, lay["frame0"] + n_anchor), index_map=destination)
            support[c0:c1] = index
            top1[c0:c1] = values[:, 0]
        convex_fit(x, candidate, support, top1=top1, easy_threshold=easy_threshold, fit=fit,
                   alpha=alpha)
        _lib.check(lib.vgo_failed_rows(fit.data_ptr(), top1.data_ptr(), float(easy_threshold),
                                       n_cand, float(threshold), failed_list.data_ptr(),
                                       failed_count.data_ptr(), stream))
        # Global fallback: top-4 of the failed rows against every destination, then refit.
        _, fb_index = _kernels.similarity_topk(
            cand_bf16, dest_bf16, 4, src_rows=failed_list[:n_cand].to(torch.int64),
            n_src_device=failed_count, n_src=n_cand, index_map=destination)
        convex_fit(x, candidate, support, row_list=failed_list, n_list=failed_count,
                   list_supports=fb_index, fit=fit, alpha=alpha)

    keep_buf = torch.empty(total, device=device, dtype=torch.int64)
    o2c = torch.empty(total, device=device, dtype=torch.int64)
    source_buf = torch.empty(max(n_cand, 1), device=device, dtype=torch.int64)
    parent_buf = torch.empty((max(n_cand, 1), 4), device=device, dtype=torch.int64)
    weight_buf = torch.empty((max(n_cand, 1), 4), device=device, dtype=torch.float32)
    stats = torch.zeros(4, device=device, dtype=torch.float32)
    _lib.check(lib.vgo_sparse_convex_assemble(
        fit.data_ptr(), alpha.data_ptr(), support.data_ptr(), candidate.data_ptr(),
        top1.data_ptr(), float(easy_threshold), failed_count.data_ptr(), n_cand, total,
        float(threshold), keep_buf.data_ptr(), o2c.data_ptr(), source_buf.data_ptr(),
        parent_buf.data_ptr(), weight_buf.data_ptr(), stats.data_ptr(), stream))
    stats_host = torch.empty(4, dtype=torch.float32, pin_memory=True)
    stats_host.copy_(stats, non_blocking=True)
    copied = torch.cuda.Event()
    copied.record(torch.cuda.current_stream(device))

    def finish(counts: torch.Tensor) -> WeightedBilinearTokenPlan:
        return _finish_plan(counts, lay, total, keep_buf, o2c, source_buf, parent_buf, weight_buf,
                            threshold, preserve_queries, preserve_destination_keys,
                            (fit, alpha, support, top1, failed_list, failed_count))

    return PendingSparseConvexPlan(finish, stats_host, copied)


def _finish_plan(counts, lay, total, keep_buf, o2c, source_buf, parent_buf, weight_buf, threshold,
                 preserve_queries, preserve_destination_keys, fit_state) -> WeightedBilinearTokenPlan:
    """The plan over the assemble kernel's buffers, sized by its counts (host copy)."""
    merged, hard, fallback, fit_sum = (float(v) for v in counts)
    m = int(merged)
    keep = keep_buf[:total - m].view(1, -1)
    source_original = source_buf[:m].view(1, -1)
    parent_compact = parent_buf[:m].view(1, -1, 4)
    weights = weight_buf[:m].view(1, -1, 4)
    special_original = lay["special"]
    special_compact = o2c.index_select(0, special_original)
    plan = WeightedBilinearTokenPlan(
        keep=keep, source_original=source_original,
        source_parent_compact=parent_compact,
        source_pool_weights=weights, source_restore_weights=weights,
        original_tokens=total, normalizer=torch.empty(0, device=keep_buf.device),
        preserve_queries=preserve_queries,
        preserve_destination_keys=(
            preserve_queries if preserve_destination_keys is None else preserve_destination_keys
        ),
        dense_special_queries=True,
        special_query_original=special_original,
        special_query_compact=special_compact,
        metadata={
            "planner": "fixed_topology_sparse_convex_v1",
            "threshold": float(threshold),
            "merge_ratio": float(m / total),
            "fit_mean": float(fit_sum / m) if m else 0.0,
            "preserve_queries": bool(preserve_queries),
            "search": "local_frame_group_exact_fallback_v1",
            "solver": "simplex_active_set_exact_v1",
            "early_accept_margin": float(_EARLY_MARGIN),
            "hard_candidates": int(hard),
            "fallback_candidates": int(fallback),
        },
    )
    mass, log_mass = plan.plan_mass()
    plan.normalizer = mass.view(1, -1, 1)
    plan.key_log_mass = log_mass.view(1, -1)
    plan._derived["fit"] = fit_state
    return plan

