"""MI355X-native merged-token global attention (VGGT-Omega token merging path).

The directory name starts with a digit, so import it with
`importlib.import_module("4d_ttt_merging_amd")`.  Public names mirror the
reference package `vggt_omega` for the merged global-attention path:

* `mass_bias_attention`                  vggt_omega/models/mass_bias_attention.py
* `TokenPlan`, `WeightedBilinearTokenPlan`, `deterministic_weighted_normalizer`,
  `build_fastvggt_plan`                  vggt_omega/models/token_merging.py
* `build_sparse_convex_plan`             vggt_omega/models/sparse_convex.py
  (`start_sparse_convex_plan`: the same without waiting for its sizes)
* `streaming_top4`                       vggt_omega/models/sparse_convex_kernels.py
* `SelfAttention`, `SelfAttentionBlock`  vggt_omega/models/layers/{attention,block}.py
* `top4_project`                         the restore gather of the plans
* `plan_io` (`save_plan`, `load_plan`, `load_ttt_trace`, ...)  plan files and
  replay of the TTT planner's trace records (sparse_convex.py:77-80, 1907-1976)
* `use_tuned_gemms`                      recorded hipBLASLt selections for the
  block's torch GEMMs (TunableOp)
* `ops` -- the torch.library operators `torch.ops.vgo.*` (mass_bias_attention,
  top4_project, compaction, QKV epilogue, residual rows) with fake
  implementations for tracing

Every GPU computation of the path runs in the hand-written gfx950 HIP library
`libvgo.so` (built by `_build.build()`); there is no CPU fallback.
"""
from __future__ import annotations

from . import _lib, ops, plan_io
from .gemm_tuning import use_tuned_gemms
from .layers import LinearKMaskedBias, SelfAttention, SelfAttentionBlock
from .mass_bias_attention import dense_attention, mass_bias_attention
from .projection import top4_project
from .sparse_convex import build_sparse_convex_plan, convex_fit, start_sparse_convex_plan
from .sparse_convex_kernels import streaming_top4
from .token_merging import (
    TokenPlan,
    WeightedBilinearTokenPlan,
    build_fastvggt_plan,
    deterministic_weighted_normalizer,
)

__all__ = [
    "LinearKMaskedBias",
    "SelfAttention",
    "SelfAttentionBlock",
    "TokenPlan",
    "WeightedBilinearTokenPlan",
    "build_fastvggt_plan",
    "build_sparse_convex_plan",
    "convex_fit",
    "dense_attention",
    "deterministic_weighted_normalizer",
    "mass_bias_attention",
    "ops",
    "plan_io",
    "start_sparse_convex_plan",
    "streaming_top4",
    "top4_project",
    "use_tuned_gemms",
]
