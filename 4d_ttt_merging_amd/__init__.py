"""MI355X-native merged-token global attention (VGGT-Omega token merging path).

The directory name starts with a digit, so import it with
`importlib.import_module("4d_ttt_merging_amd")`.  Public names mirror the
reference package `vggt_omega` for the merged global-attention path:

* `mass_bias_attention`                (vggt_omega/models/mass_bias_attention.py)
* `top4_project`                       (the restore gather of token_merging.py)

Every GPU computation runs in the hand-written gfx950 HIP library `libvgo.so`
(built by `_build.build()`); there is no CPU fallback.
"""
from __future__ import annotations

from . import _lib
from .mass_bias_attention import dense_attention, mass_bias_attention
from .projection import top4_project

__all__ = [
    "dense_attention",
    "mass_bias_attention",
    "top4_project",
]
