"""Oracle: rebuilding a merge plan from a TTT trace record (test infrastructure only).

CPU restatement, in torch-CPU ops, of the step of
`build_ttt_protected_uniform_convex_plan` that turns the fields its trace
records hold (vggt_omega/models/sparse_convex.py:1907-1931: source_ids,
support_ids, weights, accepted, patches, frames) into the returned
`WeightedBilinearTokenPlan` (:1932-1976): accepted rows only, kept patches =
the patches that are no accepted source, keep = special tokens + kept patches
in ascending original order, parents = compact ids of the four supports (which
must be kept), mass = the deterministic normalizer of token_merging.py:40-59,
log-mass = log(mass).

Pinned in tests/test_oracle_plan_io.py: records made from oracle
`sparse_convex_plan` plans (themselves pinned by the reference's fixtures)
rebuild those plans exactly, up to the fp16 rounding of the trace's weights,
and the structural invariants of a plan hold on random records.
"""
from __future__ import annotations

import torch

from oracle.merging import deterministic_weighted_normalizer, patch_ids


def plan_from_ttt_record(record: dict, *, tokens_per_frame: int, patch_token_start: int) -> dict:
    """Plan tensors of one trace record (reference sparse_convex.py:1932-1976)."""
    frames, patches = int(record["frames"]), int(record["patches"])
    patch_count = frames * patches
    total = frames * tokens_per_frame
    rows = record["accepted"].nonzero().flatten()
    source_local = record["source_ids"].long().index_select(0, rows)
    support_local = record["support_ids"].long().index_select(0, rows)
    weights = record["weights"].index_select(0, rows).float()
    kept_mask = torch.ones(patch_count, dtype=torch.bool)
    kept_mask[source_local] = False
    keep_local = kept_mask.nonzero().flatten()
    ids = patch_ids(frames, tokens_per_frame, patch_token_start).flatten()
    basis_original = ids.index_select(0, keep_local)
    source_original = ids.index_select(0, source_local)
    support_original = ids.index_select(0, support_local.reshape(-1)).reshape_as(support_local)
    special = (torch.arange(frames)[:, None] * tokens_per_frame
               + torch.arange(patch_token_start)[None]).flatten()
    keep = torch.cat((special, basis_original)).sort().values.view(1, -1)
    o2c = torch.full((1, total), -1, dtype=torch.long)
    o2c.scatter_(1, keep, torch.arange(keep.shape[1]).view(1, -1))
    parent = o2c.gather(1, support_original.reshape(1, -1)).reshape_as(support_original)
    if (parent < 0).any():
        raise RuntimeError("protected TTT convex support must remain physical")
    m = len(source_local)
    mass = deterministic_weighted_normalizer(parent.view(1, m, 4), weights.view(1, m, 4), keep.shape[1])
    return dict(keep=keep, source_original=source_original.view(1, -1),
                parent_compact=parent.view(1, m, 4), weights=weights.view(1, m, 4),
                mass=mass, log_mass=mass[..., 0].log(), special=special,
                special_compact=o2c[0, special], total=total)


def ttt_record_from_plan(keep: torch.Tensor, source_original: torch.Tensor,
                         parent_compact: torch.Tensor, weights: torch.Tensor, *, frames: int,
                         tokens_per_frame: int, patch_token_start: int) -> dict:
    """The record fields a plan determines: patch-local source and support ids, fp16
    weights, every row accepted (the inverse of `plan_from_ttt_record`)."""
    patches = tokens_per_frame - patch_token_start

    def local(original: torch.Tensor) -> torch.Tensor:
        frame, offset = original // tokens_per_frame, original % tokens_per_frame - patch_token_start
        if (offset < 0).any():
            raise ValueError("a special token cannot be written as a patch-local id")
        return frame * patches + offset

    support_original = keep.reshape(-1)[parent_compact.reshape(-1, 4)]
    source = source_original.reshape(-1)
    return dict(frames=frames, patches=patches, source_ids=local(source).int(),
                support_ids=local(support_original).int(),
                weights=weights.reshape(-1, 4).half(),
                accepted=torch.ones(source.numel(), dtype=torch.bool))
