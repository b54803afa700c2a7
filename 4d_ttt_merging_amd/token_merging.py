"""Merge plans and the FastVGGT bipartite planner on gfx950.

Mirrors the plan API of vggt_omega/models/token_merging.py (the names, fields,
methods and error behaviour that vggt_omega/models/layers/attention.py reads):

* `TokenPlan`                 (reference :143-196)  hard map, mean-pool compact,
                                                   one-hot restore
* `WeightedBilinearTokenPlan` (reference :253-426)  four-support convex pool and
                                                   restore, optional log-mass
* `deterministic_weighted_normalizer` (reference :40-59)
* `build_fastvggt_plan`       (reference :1044-1122)

Every reduction, gather and selection runs in the HIP library: compaction is
`vgo_compact` over a stable CSR of plan members (`vgo_csr_build`), restore is
`vgo_top4_project` over a dense [N,4] map, masses are `vgo_segment_mass`, and
the FastVGGT match/rank is `vgo_normalize_rows` -> `vgo_similarity_topk` ->
`vgo_fastvggt_assemble_ws`.  Only the layout-dependent index lists (which tokens
are destinations, protected or sources) are computed on the host, once per
layout, with torch's CPU generator exactly as the reference draws them.
"""
from __future__ import annotations

import ctypes

import functools
import math
from dataclasses import dataclass, field
from typing import Callable

import torch

from . import _kernels
from .projection import top4_project

FAST_MATCH_SOURCE_CHUNK = 5000

_SUPPORTED_VALUE_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _check_value(value: torch.Tensor) -> None:
    if value.dtype not in _SUPPORTED_VALUE_DTYPES:
        raise ValueError(f"merge plans support float32/bfloat16/float16 values, got {value.dtype}")
    if not value.is_cuda:
        raise RuntimeError("vgo kernels run on the GPU only; got a CPU tensor")


def _as_rows(value: torch.Tensor) -> torch.Tensor:
    """[N, C] view with unit channel stride (copies only if needed)."""
    return value if value.stride(-1) == 1 else value.contiguous()


def _zero_offsets(cache: dict, rows: int, device) -> torch.Tensor:
    """All-empty CSR offsets [rows + 1]: makes vgo_compact a plain row gather."""
    key = ("zero_offsets", rows)
    if key not in cache:
        cache[key] = torch.zeros(rows + 1, device=device, dtype=torch.int32)
    return cache[key]


@dataclass
class _Csr:
    order: torch.Tensor      # int32 item ids grouped by segment (stable)
    offsets: torch.Tensor    # int32 [segments + 1]


# ----------------------------------------------------------------------------
# deterministic mass
# ----------------------------------------------------------------------------
def _corner_csr(parent_compact: torch.Tensor, kept_tokens: int) -> _Csr:
    """Stable CSR of (destination, corner) pairs: item p = i*S + c, key = parent*S + c."""
    corners = parent_compact.shape[-1]
    parent = parent_compact.reshape(-1, corners)
    key = parent * corners + torch.arange(corners, device=parent.device)
    key = torch.where(parent >= 0, key, torch.full_like(key, kept_tokens * corners))
    order, offsets = _kernels.csr_build(key.reshape(-1), kept_tokens * corners)
    return _Csr(order, offsets)


def deterministic_weighted_normalizer(
    parent_compact: torch.Tensor,
    weights: torch.Tensor,
    kept_tokens: int,
) -> torch.Tensor:
    """Return physical-plus-source mass without atomic additions.

    mass[k] = 1 + sum over corners (in corner order) of the sequential sum, in
    source order, of the weights whose parent is k (reference
    token_merging.py:40-59).  [1, M, S] inputs -> [1, K, 1] float32.
    """
    if parent_compact.shape != weights.shape or parent_compact.shape[0] != 1:
        raise ValueError("parent ids and weights must have matching [1,M,S] shapes")
    csr = _corner_csr(parent_compact, kept_tokens)
    mass, _ = _kernels.segment_mass(csr.offsets, parent_compact.shape[-1], csr.order,
                                    weights.reshape(-1), kept_tokens, 1.0, want_log=False)
    return mass.view(1, kept_tokens, 1)


# ----------------------------------------------------------------------------
# TokenPlan
# ----------------------------------------------------------------------------
@dataclass
class TokenPlan:
    """A compact-token map for one attention operation (reference :143-196).

    `compact` mean-pools every cluster (members in ascending token order, fp32
    sum divided by the member count); `restore` broadcasts the compact update
    back through `inverse`.  `key_log_mass` is None for the reference's
    FastVGGT plan; `build_fastvggt_plan(..., mass_bias=True)` fills it with
    log(cluster size) so the bipartite plan can drive mass-bias attention.
    """

    keep: torch.Tensor                 # [B, K], original token indices
    inverse: torch.Tensor              # [B, N], original -> compact index
    original_tokens: int
    pool_sources: bool = True
    pool_mask: torch.Tensor | None = None
    metadata: dict[str, float | int] = field(default_factory=dict)
    precomputed_qkv: torch.Tensor | None = None
    key_log_mass: torch.Tensor | None = None
    _derived: dict = field(default_factory=dict, init=False, repr=False)

    @property
    def kept_tokens(self) -> int:
        return self.keep.shape[1]

    @property
    def keep_ratio(self) -> float:
        return self.kept_tokens / self.original_tokens

    # Derived device structures, built once per batch element on first use.
    def _inverse32(self, b: int) -> torch.Tensor:
        """inverse[b] as int32: the CSR keys and the one-hot restore map."""
        key = ("inverse32", b)
        if key not in self._derived:
            self._derived[key] = self.inverse[b].to(torch.int32).contiguous()
        return self._derived[key]

    def _cluster_csr(self, b: int) -> tuple[_Csr, torch.Tensor]:
        key = ("csr", b)
        if key not in self._derived:
            order, offsets = _kernels.csr_build(self._inverse32(b), self.kept_tokens)
            contribution = None if self.pool_mask is None else self.pool_mask[b].to(torch.float32)
            counts, _ = _kernels.segment_mass(offsets, 1, order, contribution, self.kept_tokens,
                                              0.0, want_log=False)
            self._derived[key] = (_Csr(order, offsets), counts, contribution)
        csr, counts, _ = self._derived[key]
        return csr, counts

    def _contribution(self, b: int) -> torch.Tensor | None:
        self._cluster_csr(b)
        return self._derived[("csr", b)][2]

    def _restore_map(self, b: int) -> tuple[torch.Tensor, torch.Tensor]:
        key = ("restore", b)
        if key not in self._derived:
            self._derived[key] = _kernels.restore_map(
                self.original_tokens, device=self.inverse.device,
                inverse=self.inverse[b].contiguous())
        return self._derived[key]

    def cluster_counts(self, b: int = 0) -> torch.Tensor:
        """Members per compact token (float32 [K]) in batch element b."""
        return self._cluster_csr(b)[1]

    def restore_map_for(self, value: torch.Tensor) -> tuple[torch.Tensor, None] | None:
        """(index [N] int32, None): the one-hot map with which `restore(value)` gathers
        value[0] (row t = value[0, inverse[t]]), for a caller that fuses the restore into
        its next pass; None when restore returns `value` itself or value holds more than
        one batch element."""
        if self.kept_tokens == self.original_tokens or value.shape[0] != 1:
            return None
        _check_value(value)
        return self._inverse32(0), None

    def compact(self, value: torch.Tensor, *, merge: bool = True) -> torch.Tensor:
        if self.kept_tokens == self.original_tokens:
            return value
        _check_value(value)
        out = torch.empty((value.shape[0], self.kept_tokens, value.shape[-1]),
                          device=value.device, dtype=value.dtype)
        for b in range(value.shape[0]):
            self.compact_into(value[b], out[b], b=b, merge=merge)
        return out

    def compact_into(self, x: torch.Tensor, out: torch.Tensor, *, b: int = 0,
                     merge: bool = True, layer_norm=None) -> torch.Tensor:
        """compact() of one batch element between [N,C] / [H,N,64] views.

        `layer_norm` = (weight, bias, eps) applies the per-head LayerNorm(64)
        to every member row before pooling (the q/k norm of the attention)."""
        if not merge and self.pool_mask is None:
            return _kernels.compact_into(x, out, base_rows=self.keep[b].contiguous(),
                                         offsets=_zero_offsets(self._derived, self.kept_tokens, x.device),
                                         segs_per_row=1, items=None, item_shift=0, item_rows=None,
                                         weights=None, normalizer=None, layer_norm=layer_norm)
        csr, counts = self._cluster_csr(b)
        return _kernels.compact_into(x, out, base_rows=None, offsets=csr.offsets, segs_per_row=1,
                                     items=csr.order, item_shift=0, item_rows=None,
                                     weights=self._contribution(b), normalizer=counts,
                                     layer_norm=layer_norm)

    def compact_multi_into(self, x: torch.Tensor, outputs, *, b: int = 0, merge: bool = True) -> None:
        """compact_into of several channel ranges of one [N, W] row table in one launch.

        `outputs` holds (channel offset, out, layer_norm or None) per output, as
        for q, k and v of a packed qkv projection; results equal compact_into's."""
        if not merge and self.pool_mask is None:
            for off, out, ln in outputs:
                self.compact_into(x[:, off:off + (out.shape[1] if out.ndim == 2 else out.shape[0] * 64)],
                                  out, b=b, merge=merge, layer_norm=ln)
            return
        csr, counts = self._cluster_csr(b)
        _kernels.compact_multi_into(x, outputs, base_rows=None, offsets=csr.offsets, segs_per_row=1,
                                    items=csr.order, item_shift=0, item_rows=None,
                                    weights=self._contribution(b), normalizer=counts)

    def restore(self, value: torch.Tensor) -> torch.Tensor:
        if self.kept_tokens == self.original_tokens:
            return value
        _check_value(value)
        out = torch.empty((value.shape[0], self.original_tokens, value.shape[-1]),
                          device=value.device, dtype=value.dtype)
        for b in range(value.shape[0]):
            index, weight = self._restore_map(b)
            top4_project(_as_rows(value[b]), index, weight, out=out[b])
        return out


# ----------------------------------------------------------------------------
# WeightedBilinearTokenPlan
# ----------------------------------------------------------------------------
@dataclass
class WeightedBilinearTokenPlan:
    """Compact attention plan with four-way, information-preserving pooling.

    Same fields and semantics as the reference (token_merging.py:253-426).
    The stable per-corner grouping the reference builds in __post_init__
    (argsort + bincount per corner) is one CSR of (destination, corner) pairs
    here, shared by Q/K/V compaction and the mass.
    """

    keep: torch.Tensor                         # [1,K] original physical ids
    source_original: torch.Tensor              # [1,M] removed source ids
    source_parent_compact: torch.Tensor        # [1,M,4] physical compact ids
    source_pool_weights: torch.Tensor          # [1,M,4], Q/K/V write weights
    source_restore_weights: torch.Tensor       # [1,M,4], output restore weights
    original_tokens: int
    normalizer: torch.Tensor                   # [1,K,1], physical + source mass
    pool_sources: bool = True
    preserve_queries: bool = False
    preserve_destination_keys: bool = False
    dense_special_queries: bool = False
    special_query_original: torch.Tensor | None = None
    special_query_compact: torch.Tensor | None = None
    pool_source_content: bool = True
    precomputed_qkv: torch.Tensor | None = None
    source_query_correction: bool = False
    source_attention_output: torch.Tensor | None = None
    key_log_mass: torch.Tensor | None = None
    query_keep: torch.Tensor | None = None
    query_source_original: torch.Tensor | None = None
    query_source_parent_compact: torch.Tensor | None = None
    query_restore_weights: torch.Tensor | None = None
    compact_mlp: bool = False
    metadata: dict[str, float | int] = field(default_factory=dict)
    _csr: _Csr = field(init=False, repr=False)
    _derived: dict = field(default_factory=dict, init=False, repr=False)

    def __post_init__(self) -> None:
        if self.source_parent_compact.shape[0] != 1:
            raise ValueError("weighted bilinear plans require one shared inference mapping")
        self._csr = _corner_csr(self.source_parent_compact, self.kept_tokens)

    @property
    def kept_tokens(self) -> int:
        return self.keep.shape[1]

    @property
    def keep_ratio(self) -> float:
        return self.kept_tokens / self.original_tokens

    @property
    def query_kept_tokens(self) -> int:
        return self.kept_tokens if self.query_keep is None else self.query_keep.shape[1]

    def plan_mass(self) -> tuple[torch.Tensor, torch.Tensor]:
        """(mass [K], log mass [K]) in the deterministic order of the normalizer."""
        return _kernels.segment_mass(self._csr.offsets, self.source_parent_compact.shape[-1],
                                     self._csr.order, self.source_pool_weights.reshape(-1),
                                     self.kept_tokens, 1.0, want_log=True)

    def _flat(self, name: str, tensor: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        if name not in self._derived:
            self._derived[name] = tensor.reshape(-1).to(dtype).contiguous()
        return self._derived[name]

    def _gather_into(self, rows: torch.Tensor, x: torch.Tensor, out: torch.Tensor,
                     layer_norm=None) -> torch.Tensor:
        return _kernels.compact_into(x, out, base_rows=rows,
                                     offsets=_zero_offsets(self._derived, rows.numel(), x.device),
                                     segs_per_row=1, items=None, item_shift=0, item_rows=None,
                                     weights=None, normalizer=None, layer_norm=layer_norm)

    def compact_into(self, x: torch.Tensor, out: torch.Tensor, *, layer_norm=None) -> torch.Tensor:
        """compact() between [N,C] / [H,N,64] views of the single batch element.

        `layer_norm` = (weight, bias, eps) normalises every gathered row per
        64-channel head before pooling (the q/k norm of the attention)."""
        keep = self._flat("keep", self.keep, torch.int64)
        if self.source_original.shape[1] == 0 or not self.pool_source_content:
            return self._gather_into(keep, x, out, layer_norm)
        return _kernels.compact_into(
            x, out, base_rows=keep, offsets=self._csr.offsets,
            segs_per_row=self.source_parent_compact.shape[-1], items=self._csr.order,
            item_shift=2 if self.source_parent_compact.shape[-1] == 4 else 0,
            item_rows=self._flat("source", self.source_original, torch.int64),
            weights=self._flat("pool_w", self.source_pool_weights, torch.float32),
            normalizer=self._flat("norm", self.normalizer, torch.float32), layer_norm=layer_norm)

    def compact(self, value: torch.Tensor, *, merge: bool = True) -> torch.Tensor:
        """Pool source Q/K/V mass into its four retained bilinear parents."""
        del merge
        _check_value(value)
        if self.source_parent_compact.shape[-1] != 4 and self.source_original.shape[1]:
            raise ValueError("weighted bilinear plans pool into exactly four parents")
        out = torch.empty((value.shape[0], self.kept_tokens, value.shape[-1]),
                          device=value.device, dtype=value.dtype)
        for b in range(value.shape[0]):
            self.compact_into(value[b], out[b])
        return out

    def compact_key_into(self, x: torch.Tensor, out: torch.Tensor, *, layer_norm=None) -> torch.Tensor:
        if not self.preserve_destination_keys:
            return self.compact_into(x, out, layer_norm=layer_norm)
        return self._gather_into(self._flat("keep", self.keep, torch.int64), x, out, layer_norm)

    def compact_key(self, value: torch.Tensor) -> torch.Tensor:
        """Keep physical keys unchanged for the Q-preserving KV-only path."""
        if not self.preserve_destination_keys:
            return self.compact(value)
        _check_value(value)
        out = torch.empty((value.shape[0], self.kept_tokens, value.shape[-1]),
                          device=value.device, dtype=value.dtype)
        for b in range(value.shape[0]):
            self.compact_key_into(value[b], out[b])
        return out

    def compact_query_into(self, x: torch.Tensor, out: torch.Tensor, *, layer_norm=None) -> torch.Tensor:
        if self.query_keep is None:
            return self.compact_into(x, out, layer_norm=layer_norm)
        return self._gather_into(self._flat("qkeep", self.query_keep, torch.int64), x, out,
                                 layer_norm)

    def compact_query(self, value: torch.Tensor) -> torch.Tensor:
        if self.query_keep is None:
            return self.compact(value)
        _check_value(value)
        out = torch.empty((value.shape[0], self.query_kept_tokens, value.shape[-1]),
                          device=value.device, dtype=value.dtype)
        for b in range(value.shape[0]):
            self.compact_query_into(value[b], out[b])
        return out

    def _restore_map(self, query: bool) -> tuple[torch.Tensor, torch.Tensor]:
        key = "qmap" if query else "map"
        if key not in self._derived:
            if query:
                has_src = self.query_source_original is not None and self.query_source_original.shape[1]
                self._derived[key] = _kernels.restore_map(
                    self.original_tokens, device=self.keep.device,
                    keep=self._flat("qkeep", self.query_keep, torch.int64),
                    source=self._flat("qsrc", self.query_source_original, torch.int64) if has_src else None,
                    parent=self._flat("qpar", self.query_source_parent_compact, torch.int64) if has_src else None,
                    weight=self._flat("qw", self.query_restore_weights, torch.float32) if has_src else None)
            else:
                has_src = self.source_original.shape[1] > 0
                self._derived[key] = _kernels.restore_map(
                    self.original_tokens, device=self.keep.device,
                    keep=self._flat("keep", self.keep, torch.int64),
                    source=self._flat("source", self.source_original, torch.int64) if has_src else None,
                    parent=self._flat("parent", self.source_parent_compact, torch.int64) if has_src else None,
                    weight=self._flat("restore_w", self.source_restore_weights, torch.float32) if has_src else None)
        return self._derived[key]

    def _project(self, value: torch.Tensor, query: bool) -> torch.Tensor:
        _check_value(value)
        index, weight = self._restore_map(query)
        out = torch.empty((value.shape[0], self.original_tokens, value.shape[-1]),
                          device=value.device, dtype=value.dtype)
        for b in range(value.shape[0]):
            top4_project(_as_rows(value[b]), index, weight, out=out[b])
        return out

    def restore_map_for(self, value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor] | None:
        """(index [N, 4] int32, weight [N, 4] float32) with which `restore(value)` projects
        value[0], for a caller that fuses the restore into its next pass; None when restore
        returns `value` itself, raises, or value holds more than one batch element (then
        call `restore`)."""
        if value.shape[0] != 1:
            return None
        if self.preserve_queries and value.shape[1] == self.original_tokens:
            return None
        if self.query_keep is not None:
            _check_value(value)
            return self._restore_map(True)
        if self.preserve_queries:
            return None
        _check_value(value)
        return self._restore_map(False)

    def restore(self, value: torch.Tensor) -> torch.Tensor:
        """Broadcast physical outputs and bilinearly recover source outputs."""
        if self.preserve_queries and value.shape[1] == self.original_tokens:
            return value
        if self.query_keep is not None:
            return self._project(value, query=True)
        if self.preserve_queries:
            if value.shape[1] != self.original_tokens:
                raise RuntimeError("Q-preserving KV compaction must produce one output per original query")
            return value
        if value.shape[0] != 1:
            raise RuntimeError("weighted bilinear compaction currently supports inference batch size one")
        return self._project(value, query=False)

    def restore_query(self, value: torch.Tensor) -> torch.Tensor:
        """Restore a tensor compacted with :meth:`compact_query`."""
        if self.query_keep is None:
            return self.restore(value)
        return self._project(value, query=True)


# ----------------------------------------------------------------------------
# FastVGGT bipartite planner
# ----------------------------------------------------------------------------
def _patch_ids(frames: int, tokens_per_frame: int, patch_token_start: int,
               device: torch.device | str = "cpu") -> torch.Tensor:
    """[frames, patches] original ids of the patch tokens (reference :1035-1041)."""
    patches = tokens_per_frame - patch_token_start
    frame_base = torch.arange(frames, device=device)[:, None] * tokens_per_frame
    return frame_base + patch_token_start + torch.arange(patches, device=device)


def _two_by_two_anchor_positions(frames: int, patch_hw: tuple[int, int], seed: int) -> torch.Tensor:
    """One seeded patch per 2x2 cell for every frame after the first.

    The draw is the reference's (token_merging.py:1072-1082,
    sparse_convex.py:2366-2371): a CPU generator seeded with `seed`, one
    uniform pair per cell, row = r0 + floor(u0 * min(2, H - r0)), same for cols.
    Returns [frames - 1, cells] patch positions.
    """
    height, width = patch_hw
    generator = torch.Generator(device="cpu").manual_seed(seed)
    row0 = torch.arange(0, height, 2)
    col0 = torch.arange(0, width, 2)
    u = torch.rand(frames - 1, len(row0), len(col0), 2, generator=generator)
    row_span = (height - row0).clamp(max=2)
    col_span = (width - col0).clamp(max=2)
    rows = row0[None, :, None] + (u[..., 0] * row_span[None, :, None]).long()
    cols = col0[None, None, :] + (u[..., 1] * col_span[None, None, :]).long()
    return (rows * width + cols).reshape(frames - 1, -1)


@functools.lru_cache(maxsize=64)
def _fastvggt_layout(total: int, frames: int, tokens_per_frame: int, patch_token_start: int,
                     patch_hw: tuple[int, int], protect_ratio: float, seed: int,
                     device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """(source ids, destination ids) on `device`, both ascending (reference :1067-1095)."""
    patch_ids = _patch_ids(frames, tokens_per_frame, patch_token_start)
    destination = torch.zeros(total, dtype=torch.bool)
    destination[patch_ids[0]] = True
    anchors = _two_by_two_anchor_positions(frames, patch_hw, seed)
    destination[patch_ids[1:].gather(1, anchors).flatten()] = True
    protected = torch.ones(total, dtype=torch.bool)
    protected[patch_ids.flatten()] = False
    protected[patch_ids[0]] = True
    count = int(total * protect_ratio)
    if count:
        protected[torch.arange(0, total, max(1, total // count))[:count]] = True
    sources = (~(destination | protected)).nonzero().flatten()
    destinations = destination.nonzero().flatten()
    return sources.to(device), destinations.to(device)


@torch.no_grad()
def build_fastvggt_plan(
    tokens: torch.Tensor,
    *,
    frames: int,
    tokens_per_frame: int,
    patch_token_start: int,
    patch_hw: tuple[int, int],
    merge_ratio: float = 0.9,
    protect_ratio: float = 0.10,
    seed: int = 0,
    match_chunk_size: int = FAST_MATCH_SOURCE_CHUNK,
    mass_bias: bool = False,
    prenormalized: bool = False,
    after_match: Callable[[], None] | None = None,
) -> TokenPlan:
    """FastVGGT bipartite plan on Omega's interleaved token layout (reference :1044-1122).

    With `prenormalized=True`, `tokens` already holds the bf16 unit rows
    `F.normalize(tokens, eps=1e-12).to(bfloat16)` of every token (as the fused
    norm1 row pass writes them, `SelfAttentionBlock.norm1_unit_rows`), and the
    matcher reads them directly instead of normalising the rows it gathers.

    Sources (non-protected, non-destination patches) are matched against all
    destinations with bf16 cosine scores; the `min(int(total*merge_ratio),
    #sources)` best-matched sources are merged into their best destination.
    `match_chunk_size` is accepted for signature compatibility; the HIP matcher
    streams the whole score matrix without materialising it.  With
    `mass_bias=True` the plan carries key_log_mass = log(cluster size).

    `after_match` (not in the reference) is called once, right after the
    matcher's kernels are enqueued on the current stream and before the
    rank-and-select: a caller can start plan-independent work on another stream
    there (the aggregator enqueues the block's qkv projection), which then runs
    beside the plan's short selection and cluster kernels instead of after them
    and never beside the matcher, whose work-groups hold every CU.
    """
    del match_chunk_size
    if not (0.0 <= merge_ratio <= 1.0 and 0.0 <= protect_ratio <= 1.0):
        raise ValueError("FastVGGT ratios must lie in [0, 1]")
    batch, total, _ = tokens.shape
    if total != frames * tokens_per_frame or patch_token_start + math.prod(patch_hw) != tokens_per_frame:
        raise ValueError("Invalid Omega FastVGGT frame/patch/special-token layout")
    device = tokens.device

    def identity_plan():
        identity = torch.arange(total, device=device).expand(batch, -1)
        return TokenPlan(identity, identity, total)

    if frames == 1 or merge_ratio == 0:
        return identity_plan()
    sources, destinations = _fastvggt_layout(
        total, frames, tokens_per_frame, patch_token_start, tuple(patch_hw), float(protect_ratio),
        int(seed), device)
    removed = min(int(total * merge_ratio), sources.numel())
    if removed == 0:
        return identity_plan()
    if not tokens.is_cuda:
        raise RuntimeError("vgo kernels run on the GPU only; got a CPU tensor")

    best = torch.empty((batch, sources.numel()), device=device, dtype=torch.float32)
    target = torch.empty((batch, sources.numel()), device=device, dtype=torch.int32)
    if prenormalized and tokens.dtype != torch.bfloat16:
        raise ValueError("prenormalized FastVGGT tokens must be bf16 unit rows")
    for b in range(batch):
        x = _as_rows(tokens[b])
        if prenormalized:
            src, src_rows = x, sources
            dst = x.index_select(0, destinations)
        else:
            src, src_rows = _kernels.normalize_rows(x, sources, 1e-12), None
            dst = _kernels.normalize_rows(x, destinations, 1e-12)
        _kernels.similarity_topk(src, dst, 1, src_rows=src_rows, index_dtype=torch.int32,
                                 out=(best[b].view(-1, 1), target[b].view(-1, 1)))
    if after_match is not None:
        after_match()
    keep = torch.empty((batch, total - removed), device=device, dtype=torch.int64)
    inverse = torch.empty((batch, total), device=device, dtype=torch.int64)
    flags = torch.empty((batch, sources.numel()), device=device, dtype=torch.uint8)
    lib = _kernels._lib.load()
    need = ctypes.c_size_t(0)
    _kernels._lib.check(lib.vgo_fastvggt_assemble_workspace(batch, sources.numel(), total,
                                                            ctypes.byref(need)))
    workspace = torch.empty(max(need.value // 4, 1), device=device, dtype=torch.int32)
    status = lib.vgo_fastvggt_assemble_ws(
        best.data_ptr(), target.data_ptr(), sources.data_ptr(), destinations.data_ptr(), batch,
        sources.numel(), destinations.numel(), total, removed, keep.data_ptr(), inverse.data_ptr(),
        flags.data_ptr(), workspace.data_ptr(), need.value, _kernels._lib.stream_of(tokens))
    _kernels._lib.check(status)
    plan = TokenPlan(keep, inverse, total)
    # Match results stay on the device for diagnostics and tests.
    plan._derived["match"] = (sources, destinations, best, target, flags)
    if mass_bias:
        if batch != 1:
            raise ValueError("mass-bias FastVGGT plans support batch size one")
        # One mass pass gives the cluster counts _cluster_csr caches and their logs.
        order, offsets = _kernels.csr_build(plan._inverse32(0), plan.kept_tokens)
        counts, log_mass = _kernels.segment_mass(offsets, 1, order, None, plan.kept_tokens, 0.0,
                                                 want_log=True)
        plan._derived[("csr", 0)] = (_Csr(order, offsets), counts, None)
        plan.key_log_mass = log_mass.view(1, -1)
    return plan
