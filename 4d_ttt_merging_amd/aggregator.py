"""Alternating frame / inter-frame attention encoder with merged global blocks.

The caller of the merged global-attention path: the per-block loop and the
global branch of vggt_omega/models/aggregator.py:49-1293, with the reference's
parameter names (frame_blocks, inter_frame_blocks, camera_token,
register_token) and merge setters (`set_fastvggt`, `set_sparse_convex`,
`set_input_patch_tokens_cache`).  Scope:

* global blocks run `build_fastvggt_plan` or `build_sparse_convex_plan`
  ("fixed_topology") and `SelfAttentionBlock.forward_compacted` on the HIP
  library; frame blocks (RoPE) and register blocks run the same block class
  (fused row passes, QKV epilogue and attention kernels under autocast);
* the DINOv3 patch encoder is not part of the merged path: forward() consumes the
  patch tokens installed with `set_input_patch_tokens_cache` (the reference's
  own bypass, aggregator.py:233-241, 735-743), or, when built with
  `patch_encoder`, runs `patch_encoder.PatchEncoder` on the normalised images
  (aggregator.py:725-739) while no cache is installed;
* the other planners (k-means, hash, TTT, temporal, reference-anchor, affine)
  are out of scope and rejected by the setters; plans they built can still
  run here through `set_sparse_convex_plans` (e.g. TTT trace records rebuilt
  by `plan_io.load_ttt_trace`), and `set_sparse_convex(reuse_plan=True)`
  reuses one plan across a forward's global blocks as the reference's reuse
  planners do.
"""
from __future__ import annotations

import dataclasses

import torch
import torch.nn as nn

from . import profiling
from .layers import Mlp, SelfAttentionBlock, init_weights_vit, rope_sincos
from .patch_encoder import PatchEncoder
from .sparse_convex import build_sparse_convex_plan, start_sparse_convex_plan
from .token_merging import build_fastvggt_plan

_DEFAULT_SPARSE_CONVEX_QKV_LAYERS = tuple(layer for layer in range(19) if layer not in {8, 10, 11, 12})
# Image normalisation in front of the patch encoder (aggregator.py:39-40, 729).
_RESNET_MEAN = (0.485, 0.456, 0.406)
_RESNET_STD = (0.229, 0.224, 0.225)


class Aggregator(nn.Module):
    def __init__(self, patch_size: int = 16, embed_dim: int = 1024, depth: int = 24,
                 num_heads: int = 16, mlp_ratio: float = 4.0, num_register_tokens: int = 16,
                 register_attention_block_indices: tuple[int, ...] = (2, 6, 9, 14, 20),
                 cached_layer_indices: tuple[int, ...] = (4, 11, 17, 23),
                 patch_encoder: bool | PatchEncoder = False, device=None) -> None:
        """`patch_encoder`: True builds the DINOv3 ViT-L/16 encoder of
        aggregator.py:66-68, 1296-1320 (random init); a PatchEncoder instance is used
        as given; False (the default) leaves forward() to cached patch tokens."""
        super().__init__()

        def block():
            return SelfAttentionBlock(dim=embed_dim, num_heads=num_heads, ffn_ratio=mlp_ratio,
                                      qkv_bias=True, proj_bias=True, ffn_bias=True, ffn_layer=Mlp,
                                      init_values=1e-5, use_qk_norm=True, mask_k_bias=True,
                                      device=device)

        self.frame_blocks = nn.ModuleList([block() for _ in range(depth)])
        self.inter_frame_blocks = nn.ModuleList([block() for _ in range(depth)])
        self.depth = depth
        self.patch_size = patch_size
        self.num_heads = num_heads
        self.cached_layer_indices = set(cached_layer_indices)
        self.camera_token = nn.Parameter(torch.empty(1, 2, 1, embed_dim, device=device))
        self.register_token = nn.Parameter(torch.empty(1, 2, num_register_tokens, embed_dim, device=device))
        self.patch_token_start = 1 + num_register_tokens
        self.inter_frame_attention_types = ["global"] * depth
        for idx in register_attention_block_indices:
            if idx < 0 or idx >= depth:
                raise ValueError(f"register_attention_block_indices contains invalid block index {idx}")
            self.inter_frame_attention_types[idx] = "register"
        self.fastvggt_enabled = False
        self.fastvggt_merge_ratio = 0.9
        self.fastvggt_protect_ratio = 0.10
        self.fastvggt_mass_bias = False
        self.fastvggt_last_plan_stats: list[dict[str, float | int]] = []
        self.sparse_convex_enabled = False
        self.sparse_convex_threshold = .90
        self.sparse_convex_planner = "fixed_topology"
        self.sparse_convex_qkv_global_blocks = 15
        self.sparse_convex_qkv_global_layers: frozenset[int] | None = frozenset(_DEFAULT_SPARSE_CONVEX_QKV_LAYERS)
        self.sparse_convex_physical_key_layers: frozenset[int] = frozenset()
        self.sparse_convex_dense_global_layers: frozenset[int] = frozenset()
        self.sparse_convex_last_plan_stats: list[dict[str, float | int]] = []
        self.sparse_convex_reuse_plan = False
        self.sparse_convex_refit_ordinal = -1
        self._sparse_convex_reuse_plan = None
        self._sparse_convex_replay: list | None = None
        self._input_patch_tokens_cache: torch.Tensor | None = None
        self.init_weights()
        if patch_encoder is True:
            patch_encoder = PatchEncoder(patch_size=patch_size, embed_dim=embed_dim, device=device)
        self.patch_embed = patch_encoder if isinstance(patch_encoder, PatchEncoder) else None
        for name, value in (("_resnet_mean", _RESNET_MEAN), ("_resnet_std", _RESNET_STD)):
            self.register_buffer(name, torch.tensor(value, device=device).view(1, 1, 3, 1, 1), persistent=False)

    # ---------------------------------------------------------- setters ----
    def set_fastvggt(self, enabled: bool = True, merge_ratio: float = 0.9,
                     protect_ratio: float = 0.10, mass_bias: bool = False) -> None:
        """FastVGGT bipartite merging (aggregator.py:219-231); `mass_bias` adds log(cluster
        size) as the per-key attention bias."""
        if not 0.0 <= merge_ratio <= 1.0 or not 0.0 <= protect_ratio <= 1.0:
            raise ValueError("FastVGGT ratios must lie in [0, 1]")
        if enabled and self.sparse_convex_enabled:
            raise ValueError("FastVGGT, temporal merging, reference-anchor, and reference-cluster merging are mutually exclusive")
        self.fastvggt_enabled, self.fastvggt_merge_ratio = enabled, merge_ratio
        self.fastvggt_protect_ratio, self.fastvggt_mass_bias = protect_ratio, mass_bias

    def set_sparse_convex(self, enabled: bool = True, threshold: float = .90,
                          qkv_global_blocks: int = 15,
                          qkv_global_layers: tuple[int, ...] | None = _DEFAULT_SPARSE_CONVEX_QKV_LAYERS,
                          physical_key_layers: tuple[int, ...] = (),
                          planner: str = "fixed_topology",
                          dense_global_layers: tuple[int, ...] = (), reuse_plan: bool = False,
                          refit_ordinal: int = -1) -> None:
        """Sparse-convex merging (aggregator.py:243-289), fixed-topology planner.

        `reuse_plan` builds the plan at the first merged global block of a
        forward and reuses it in the later ones, with the per-layer
        preserve_queries / preserve_destination_keys of each (the reuse of
        aggregator.py:980-1006, which the reference switches on with the
        kmeans_convex_reuse planner or VGGT_TTT_REUSE_PLAN=1); `refit_ordinal`
        (VGGT_TTT_REFIT_ORDINAL there) rebuilds the cached plan at that global
        ordinal."""
        if not -1.0 <= threshold <= 1.000001:
            raise ValueError("sparse-convex threshold must lie in [-1,1]")
        global_count = sum(kind == "global" for kind in self.inter_frame_attention_types)
        if not 0 <= qkv_global_blocks <= global_count:
            raise ValueError("invalid sparse-convex QKV global-block count")
        if planner != "fixed_topology":
            raise ValueError("only the fixed_topology sparse-convex planner is part of this path")
        for name, layers in (("qkv_global_layers", qkv_global_layers),
                             ("physical_key_layers", physical_key_layers),
                             ("dense_global_layers", dense_global_layers)):
            if layers is not None and any(not 0 <= int(layer) < global_count for layer in layers):
                raise ValueError(f"invalid sparse-convex {name}: {layers}")
        if enabled and self.fastvggt_enabled:
            raise ValueError("sparse-convex merging is mutually exclusive with other merge modes")
        self.sparse_convex_enabled = bool(enabled)
        self.sparse_convex_threshold = float(threshold)
        self.sparse_convex_planner = planner
        self.sparse_convex_qkv_global_blocks = int(qkv_global_blocks)
        self.sparse_convex_qkv_global_layers = (
            None if qkv_global_layers is None else frozenset(int(x) for x in qkv_global_layers))
        self.sparse_convex_physical_key_layers = frozenset(int(x) for x in physical_key_layers)
        self.sparse_convex_dense_global_layers = frozenset(int(x) for x in dense_global_layers)
        self.sparse_convex_reuse_plan = bool(reuse_plan)
        self.sparse_convex_refit_ordinal = int(refit_ordinal)

    def set_sparse_convex_plans(self, plans) -> None:
        """Replay given plans (e.g. `plan_io.load_ttt_trace` or `plan_io.load_plan` output)
        instead of building them: the k-th plan a forward would build is plans[k].

        The reference's TTT planner writes one trace record per plan it builds
        (sparse_convex.py:1907-1931), in this order.  Each plan takes the
        per-layer preserve flags as a reused plan does (aggregator.py:993-1001).
        None restores planning."""
        self._sparse_convex_replay = None if plans is None else list(plans)

    def set_input_patch_tokens_cache(self, tokens: torch.Tensor | None) -> None:
        """Install or clear the patch tokens consumed by forward() (aggregator.py:233-241)."""
        if tokens is not None:
            if tokens.ndim != 3 or tokens.shape[-1] != self.camera_token.shape[-1]:
                raise ValueError("cached patch tokens must be [batch*frames,patches,embed_dim]")
            if not bool(torch.isfinite(tokens).all()):
                raise ValueError("cached patch tokens must be finite")
            tokens = tokens.detach().contiguous()
        self._input_patch_tokens_cache = tokens

    def init_weights(self) -> None:
        nn.init.normal_(self.camera_token, std=1e-3)
        nn.init.normal_(self.register_token, std=1e-3)
        for blocks in (self.frame_blocks, self.inter_frame_blocks):
            for module in blocks.modules():
                init_weights_vit(module)

    # ---------------------------------------------------------- forward ----
    def forward(self, images: torch.Tensor) -> tuple[list[torch.Tensor | None], int]:
        batch_size, num_frames, num_channels, height, width = images.shape
        if num_channels != 3:
            raise ValueError(f"Expected 3 input channels, got {num_channels}")
        patch_tokens = self._input_patch_tokens_cache
        if patch_tokens is None:
            if self.patch_embed is None:
                raise RuntimeError("no patch tokens: install them with set_input_patch_tokens_cache() or "
                                   "build the aggregator with its patch encoder (patch_encoder=True)")
            normalized = (images - self._resnet_mean) / self._resnet_std
            with profiling.span("patch_embed"):
                patch_tokens = self.patch_embed(normalized.view(batch_size * num_frames, num_channels, height,
                                                                width))["x_norm_patchtokens"]
        grid = (height // self.patch_size, width // self.patch_size)
        if (patch_tokens.shape[0] != batch_size * num_frames
                or patch_tokens.shape[1] != grid[0] * grid[1]
                or patch_tokens.device != images.device):
            raise ValueError("cached patch tokens do not match the current model input")
        camera = _slice_expand_and_flatten(self.camera_token, batch_size, num_frames)
        register = _slice_expand_and_flatten(self.register_token, batch_size, num_frames)
        tokens = torch.cat([camera.to(patch_tokens.dtype), register.to(patch_tokens.dtype),
                            patch_tokens], dim=1)
        _, num_tokens, embed_dim = tokens.shape
        with torch.no_grad():
            sin, cos = rope_sincos(grid[0], grid[1], embed_dim // self.num_heads,
                                   device=patch_tokens.device)
        rope = (sin, cos)
        self.fastvggt_last_plan_stats = []
        self.sparse_convex_last_plan_stats = []
        self._sparse_convex_reuse_plan = None
        self._sparse_convex_replayed = 0
        outputs: list[torch.Tensor | None] = []
        for block_idx in range(self.depth):
            tokens = tokens.view(batch_size * num_frames, num_tokens, embed_dim)
            tokens = self.frame_blocks[block_idx](tokens, rope)
            frame_tokens = tokens.view(batch_size, num_frames, num_tokens, embed_dim)
            tokens = self._run_inter_frame_attention_block(
                tokens, batch_size, num_frames, num_tokens, embed_dim, block_idx, grid,
                reuse_input=block_idx not in self.cached_layer_indices)
            if block_idx in self.cached_layer_indices:
                outputs.append(torch.cat([frame_tokens, tokens], dim=-1))
            else:
                outputs.append(None)
        return outputs, self.patch_token_start

    def _side_qkv(self, block, x: torch.Tensor) -> "_SideQkv | None":
        """The side-stream projection of a FastVGGT block's qkv (see `_SideQkv`), or None
        to project in the block: off the GPU, or while a graph is being captured before
        the side stream exists (a stream is created outside capture only)."""
        if not x.is_cuda:
            return None
        streams = self.__dict__.setdefault("_qkv_streams", {})
        stream = streams.get(x.device)
        if stream is None:
            if torch.cuda.is_current_stream_capturing():
                return None
            stream = streams[x.device] = torch.cuda.Stream(device=x.device)
        return _SideQkv(stream, block, x)

    def _run_inter_frame_attention_block(self, tokens, batch_size, num_frames, num_tokens,
                                         embed_dim, block_idx, patch_hw,
                                         reuse_input: bool = False) -> torch.Tensor:
        """`reuse_input`: the caller keeps no other reference to `tokens`, so a register
        block may write its special rows into it instead of concatenating a new tensor."""
        kind = self.inter_frame_attention_types[block_idx]
        block = self.inter_frame_blocks[block_idx]
        tokens = tokens.view(batch_size, num_frames, num_tokens, embed_dim)
        if kind == "register":
            pts = self.patch_token_start
            special = tokens[:, :, :pts].reshape(batch_size, num_frames * pts, embed_dim)
            special = block(special, None).view(batch_size, num_frames, pts, embed_dim)
            if reuse_input and special.dtype == tokens.dtype and not torch.is_grad_enabled():
                tokens[:, :, :pts] = special
                return tokens
            return torch.cat([special, tokens[:, :, pts:]], dim=2)
        if kind != "global":
            raise ValueError(f"Unknown inter-frame attention type: {kind}")
        tokens = tokens.reshape(batch_size, num_frames * num_tokens, embed_dim)
        global_ordinal = sum(k == "global" for k in self.inter_frame_attention_types[:block_idx])
        if not (self.fastvggt_enabled or self.sparse_convex_enabled):
            tokens = block(tokens, None)
            return tokens.view(batch_size, num_frames, num_tokens, embed_dim)
        with profiling.span("global.block"):
            if self.sparse_convex_enabled and global_ordinal in self.sparse_convex_dense_global_layers:
                tokens = block(tokens, None)
                # The reference records the bypass too (aggregator.py:885-899).
                self.sparse_convex_last_plan_stats.append({
                    "block_index": block_idx, "global_ordinal": global_ordinal,
                    "original_tokens": int(tokens.shape[1]), "kept_tokens": int(tokens.shape[1]),
                    "merged_tokens": 0, "merge_ratio": 0.0, "compact_queries": False,
                    "physical_keys": True, "reused_plan": False,
                    "attention_query_tokens": int(tokens.shape[1]),
                    "planner": "dense_layer_bypass"})
                return tokens.view(batch_size, num_frames, num_tokens, embed_dim)
            layout = dict(frames=num_frames, tokens_per_frame=num_tokens,
                          patch_token_start=self.patch_token_start, patch_hw=patch_hw)
            precomputed_qkv = None
            side = None
            unit_rows = None if self.sparse_convex_enabled else block.norm1_unit_rows(tokens)
            if unit_rows is not None:
                normalized = None
                unit_rows, attn_input = unit_rows
            else:
                normalized, attn_input = block.norm1_for_plan(tokens)
            with profiling.span("global.plan_build"):
                if self.sparse_convex_enabled:
                    if self.sparse_convex_qkv_global_layers is not None:
                        compact_queries = global_ordinal in self.sparse_convex_qkv_global_layers
                    else:
                        compact_queries = global_ordinal < self.sparse_convex_qkv_global_blocks
                    preserve_queries = not compact_queries
                    preserve_keys = preserve_queries or global_ordinal in self.sparse_convex_physical_key_layers
                    reuse_plan = self.sparse_convex_reuse_plan
                    force_refit = reuse_plan and global_ordinal == self.sparse_convex_refit_ordinal >= 0
                    if reuse_plan and self._sparse_convex_reuse_plan is not None and not force_refit:
                        plan = _with_preserve_flags(self._sparse_convex_reuse_plan, preserve_queries,
                                                    preserve_keys)
                    else:
                        if self._sparse_convex_replay is not None:
                            if self._sparse_convex_replayed >= len(self._sparse_convex_replay):
                                raise RuntimeError("the replayed sparse-convex plans ran out at "
                                                   f"global ordinal {global_ordinal}")
                            plan = _with_preserve_flags(
                                self._sparse_convex_replay[self._sparse_convex_replayed],
                                preserve_queries, preserve_keys)
                            self._sparse_convex_replayed += 1
                        else:
                            # The plan's size reaches the host by an asynchronous copy; the
                            # qkv projection (independent of the plan) is enqueued before the
                            # wait for it, so the GPU stays busy while the host sizes the plan.
                            pending = start_sparse_convex_plan(
                                normalized, threshold=self.sparse_convex_threshold,
                                preserve_queries=preserve_queries,
                                preserve_destination_keys=preserve_keys, **layout)
                            with profiling.span("global.qkv_projection"):
                                precomputed_qkv = block.attn.qkv(attn_input)
                            plan = pending.result()
                        if reuse_plan:
                            self._sparse_convex_reuse_plan = plan
                    self.sparse_convex_last_plan_stats.append({
                        "block_index": block_idx, "global_ordinal": global_ordinal,
                        "original_tokens": plan.original_tokens, "kept_tokens": plan.kept_tokens,
                        "merged_tokens": plan.original_tokens - plan.kept_tokens,
                        "merge_ratio": 1.0 - plan.keep_ratio,
                        "compact_queries": bool(compact_queries), "physical_keys": bool(preserve_keys),
                        "reused_plan": bool(reuse_plan and global_ordinal > 0 and not force_refit),
                        "refit_plan": bool(force_refit),
                        "attention_query_tokens": int(plan.kept_tokens if compact_queries
                                                      else plan.original_tokens),
                        **plan.metadata})
                else:
                    side = self._side_qkv(block, attn_input)
                    plan = build_fastvggt_plan(
                        normalized if unit_rows is None else unit_rows,
                        merge_ratio=self.fastvggt_merge_ratio, protect_ratio=self.fastvggt_protect_ratio,
                        mass_bias=self.fastvggt_mass_bias, prenormalized=unit_rows is not None,
                        after_match=None if side is None else side.launch, **layout)
                    self.fastvggt_last_plan_stats.append({
                        "block_index": block_idx, "original_tokens": plan.original_tokens,
                        "kept_tokens": plan.kept_tokens,
                        "merged_tokens": plan.original_tokens - plan.kept_tokens,
                        "merge_ratio": 1.0 - plan.keep_ratio, **plan.metadata})
            if side is not None:
                # The wait for the side-stream projection: the part of the GEMM the plan's
                # kernels did not cover.
                with profiling.span("global.qkv_projection"):
                    precomputed_qkv = side.join()
            if precomputed_qkv is None:
                tokens = block.forward_compacted(tokens, plan, normalized=attn_input)
            else:
                # This layer's projection rides on the plan for this call only (a reused
                # plan serves later layers with their own projections).
                plan.precomputed_qkv = precomputed_qkv
                try:
                    tokens = block.forward_compacted(tokens, plan, normalized=attn_input)
                finally:
                    plan.precomputed_qkv = None
        return tokens.view(batch_size, num_frames, num_tokens, embed_dim)


class _SideQkv:
    """A global block's qkv projection on a side stream.

    `launch` (the FastVGGT builder's `after_match` hook) makes the side stream wait
    for the current stream's work so far -- the norm1 rows and the matcher -- and
    enqueues the projection there, so the GEMM runs beside the plan's short
    rank-and-select and cluster kernels, which occupy few CUs, and never beside the
    matcher, whose work-groups hold every CU.  `join` makes the current stream wait
    for the projection and returns it (None if `launch` was not called: plans that
    need no matching).  The projection is the same call the block makes itself, so
    the outputs are unchanged.
    """

    def __init__(self, stream: torch.cuda.Stream, block: SelfAttentionBlock, x: torch.Tensor) -> None:
        self.stream, self.block, self.x = stream, block, x
        self.qkv = None
        self.done = None

    def launch(self) -> None:
        ready = torch.cuda.Event()
        ready.record(torch.cuda.current_stream(self.x.device))
        with torch.cuda.stream(self.stream):
            self.stream.wait_event(ready)
            self.x.record_stream(self.stream)
            self.qkv = self.block.attn.qkv(self.x)
            self.done = torch.cuda.Event()
            self.done.record(self.stream)

    def join(self) -> torch.Tensor | None:
        if self.qkv is None:
            return None
        main = torch.cuda.current_stream(self.x.device)
        main.wait_event(self.done)
        self.qkv.record_stream(main)
        return self.qkv


def _slice_expand_and_flatten(token_tensor: torch.Tensor, batch_size: int, num_frames: int) -> torch.Tensor:
    first = token_tensor[:, 0:1].expand(batch_size, 1, *token_tensor.shape[2:])
    others = token_tensor[:, 1:].expand(batch_size, num_frames - 1, *token_tensor.shape[2:])
    tokens = torch.cat([first, others], dim=1)
    return tokens.view(batch_size * num_frames, *tokens.shape[2:])


def _with_preserve_flags(plan, preserve_queries: bool, preserve_keys: bool):
    """The plan with this layer's preserve flags (aggregator.py:993-1001)."""
    if (plan.preserve_queries == preserve_queries
            and plan.preserve_destination_keys == preserve_keys):
        return plan
    return dataclasses.replace(plan, preserve_queries=preserve_queries,
                               preserve_destination_keys=preserve_keys)
