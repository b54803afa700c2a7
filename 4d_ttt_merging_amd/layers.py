"""Transformer layers of the merged global-attention path.

`SelfAttention` and `SelfAttentionBlock` keep the parameter names, constructor
arguments and forward signatures of vggt_omega/models/layers/attention.py:195-439
and vggt_omega/models/layers/block.py:22-226, so reference state dicts load
unchanged.  With a token plan, `SelfAttention` runs the merged path on the HIP
library:

  qkv = Linear(x)                         (torch GEMM, hipBLASLt)
  Q/K/V compaction through the plan,      vgo_compact: q/k LayerNorm64 of every
  written head-major [H, N, 64]           gathered row before pooling
  preserved / special queries             vgo_qkv_epilogue (LayerNorm64, split)
  mass-bias attention                     vgo_mass_bias_attn_fwd_ws, written
                                          directly in [B, N, H, 64] order
  dense special queries                   the same launch
                                          (vgo_mass_bias_attn_pair_fwd_ws), then
                                          their rows copied over the result
  out = Linear(x)                         (torch GEMM)
  restore                                 vgo_top4_project

Frame and register blocks (no plan) in bf16/f16 run the same attention kernel
behind vgo_qkv_epilogue (LayerNorm64 + RoPE); other dtypes and layouts take
the reference's torch op sequence.
The reference's experimental hooks that import the absent module
`sampled_update_operator` (attention.py:267-299) and the source-query
correction branch (attention.py:304-312, 376-385) are not part of this path
and raise NotImplementedError if a caller enables them.
"""
from __future__ import annotations

import math
from typing import Callable

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import _kernels, profiling
from .mass_bias_attention import _attention_into, _attention_pair_into


class _null:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


def rope_rotate_half(x: Tensor) -> Tensor:
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat([-x2, x1], dim=-1)


def rope_apply(x: Tensor, sin: Tensor, cos: Tensor) -> Tensor:
    return (x * cos) + (rope_rotate_half(x) * sin)


class Linear(nn.Linear):
    """nn.Linear whose autocast inference casts its parameters once.

    Under CUDA bf16/f16 autocast, F.linear casts the fp32 weight and bias to the
    autocast dtype on every call (a copy kernel each).  When no gradient is
    recorded, the cast copies are kept and reused until a parameter changes
    (its version counter or its storage), so the GEMM gets the operands that
    autocast would give it and the result is the same.  Writes that bypass the
    version counter (through `.data`) must be followed by `clear_cast_cache()`.

    The cache is neither used nor built while the current stream is being
    captured into a graph (a copy made there would only be filled when the
    graph replays, and a replay must re-cast parameters updated in place
    since), nor when autocast's own cast cache is switched off
    (`cache_enabled=False`: every call then casts, as autocast does)."""

    def clear_cast_cache(self) -> None:
        self.__dict__.pop("_cast_cache", None)

    def _bias(self) -> Tensor | None:
        return self.bias

    def _cast_sources(self) -> tuple:
        return (self.weight, self.bias)

    def _cast_params(self, dtype: torch.dtype):
        try:
            key = (dtype,) + tuple(None if t is None else (t.data_ptr(), t._version)
                                   for t in self._cast_sources())
        except RuntimeError:  # inference tensors keep no version counter
            return None
        cache = self.__dict__.get("_cast_cache")
        if cache is None or cache[0] != key:
            bias = self._bias()
            cache = (key, self.weight.to(dtype), None if bias is None else bias.to(dtype))
            self.__dict__["_cast_cache"] = cache
        return cache[1], cache[2]

    def forward(self, input: Tensor) -> Tensor:
        dtype = _autocast_dtype()
        # A traced graph (torch.compile) keeps autocast's casts as graph nodes.
        if (dtype is not None and not torch.is_grad_enabled() and self.weight.is_cuda
                and not torch.compiler.is_compiling() and torch.is_autocast_cache_enabled()
                and not torch.cuda.is_current_stream_capturing()):
            cast = self._cast_params(dtype)
            if cast is not None:
                return F.linear(input, *cast)
        return F.linear(input, self.weight, self._bias())


class LinearKMaskedBias(Linear):
    """qkv projection whose K third of the bias is masked to zero (attention.py:195-207)."""

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        o = self.out_features
        assert o % 3 == 0
        if self.bias is not None:
            bias_mask = torch.ones_like(self.bias)
            bias_mask[o // 3: 2 * o // 3].fill_(0)
            self.register_buffer("bias_mask", bias_mask)

    def _bias(self) -> Tensor | None:
        return self.bias * self.bias_mask.to(self.bias.dtype) if self.bias is not None else None

    def _cast_sources(self) -> tuple:
        return (self.weight, self.bias, getattr(self, "bias_mask", None))


class LayerScale(nn.Module):
    def __init__(self, dim: int, init_values: float | Tensor = 1e-5, inplace: bool = False,
                 device=None) -> None:
        super().__init__()
        self.inplace = inplace
        self.gamma = nn.Parameter(torch.empty(dim, device=device))
        self.init_values = init_values
        self.reset_parameters()

    def reset_parameters(self):
        nn.init.constant_(self.gamma, self.init_values)

    def forward(self, x: Tensor) -> Tensor:
        return x.mul_(self.gamma) if self.inplace else x * self.gamma


class Mlp(nn.Module):
    def __init__(self, in_features: int, hidden_features: int | None = None,
                 out_features: int | None = None, act_layer: Callable[..., nn.Module] = nn.GELU,
                 drop: float = 0.0, bias: bool = True, device=None) -> None:
        super().__init__()
        out_features = out_features or in_features
        hidden_features = hidden_features or in_features
        self.fc1 = Linear(in_features, hidden_features, bias=bias, device=device)
        self.act = act_layer()
        self.fc2 = Linear(hidden_features, out_features, bias=bias, device=device)
        self.drop = nn.Dropout(drop)

    def forward(self, x: Tensor) -> Tensor:
        return self.drop(self.fc2(self.drop(self.act(self.fc1(x)))))


class SelfAttention(nn.Module):
    def __init__(self, dim: int, num_heads: int = 8, qkv_bias: bool = False,
                 proj_bias: bool = True, attn_drop: float = 0.0, proj_drop: float = 0.0,
                 mask_k_bias: bool = False, use_qk_norm: bool = False, device=None) -> None:
        super().__init__()
        self.num_heads = num_heads
        head_dim = dim // num_heads
        self.scale = head_dim ** -0.5
        self.use_qk_norm = use_qk_norm
        if use_qk_norm:
            self.q_norm = nn.LayerNorm(head_dim, eps=1e-5)
            self.k_norm = nn.LayerNorm(head_dim, eps=1e-5)
        else:
            self.q_norm = None
            self.k_norm = None
        linear_class = LinearKMaskedBias if mask_k_bias else Linear
        self.qkv = linear_class(dim, dim * 3, bias=qkv_bias, device=device)
        self.attn_drop = nn.Dropout(attn_drop)
        self.proj = Linear(dim, dim, bias=proj_bias, device=device)
        self.proj_drop = nn.Dropout(proj_drop)

    def apply_rope(self, q: Tensor, k: Tensor, rope) -> tuple[Tensor, Tensor]:
        q_dtype, k_dtype = q.dtype, k.dtype
        sin, cos = rope
        q, k = q.to(sin.dtype), k.to(sin.dtype)
        prefix = q.shape[-2] - sin.shape[-2]
        assert prefix >= 0
        q = torch.cat((q[:, :, :prefix], rope_apply(q[:, :, prefix:], sin, cos)), dim=-2)
        k = torch.cat((k[:, :, :prefix], rope_apply(k[:, :, prefix:], sin, cos)), dim=-2)
        return q.to(q_dtype), k.to(k_dtype)

    def _check_hooks(self) -> None:
        for name in ("fixed_update_operator_config", "sampled_update_operator_config",
                     "dense_update_diagnostic_config", "baseline_trajectory_probe_config"):
            if getattr(self, name, None) is not None:
                raise NotImplementedError(f"{name} is outside the merged global-attention path")

    def forward(self, x: Tensor, attn_bias=None, rope: Tensor = None, token_plan=None) -> Tensor:
        if token_plan is not None and self.training:
            raise RuntimeError("token compaction is inference-only")
        self._check_hooks()
        if token_plan is None:
            qkv = self.qkv(x)
            return self.proj_drop(self.proj(self.compute_attention(qkv=qkv, attn_bias=attn_bias,
                                                                   rope=rope)))
        x = self._forward_merged(x, attn_bias, rope, token_plan)
        with profiling.span("global.update_restore"):
            return token_plan.restore(x)

    def _forward_merged(self, x: Tensor, attn_bias, rope, token_plan) -> Tensor:
        """The merged forward up to the output projection: attention.py:284-303 without
        the final `token_plan.restore`, which the caller applies (or fuses)."""
        qkv = getattr(token_plan, "precomputed_qkv", None)
        if qkv is None:  # a precomputed projection was timed where its caller made it
            with profiling.span("global.qkv_projection"):
                qkv = self.qkv(x)
        attn_v = self.compute_attention(qkv=qkv, attn_bias=attn_bias, rope=rope, token_plan=token_plan)
        with profiling.span("global.output_projection"):
            x = self.proj_drop(self.proj(attn_v))
        if (getattr(token_plan, "source_query_correction", False)
                and not getattr(token_plan, "preserve_queries", False)):
            raise NotImplementedError("source-query correction is outside the merged path")
        return x

    # ---------------------------------------------------------------------
    def _attention_dtype(self, qkv: Tensor) -> torch.dtype:
        """dtype the attention runs in: the autocast dtype, as the reference's SDPA /
        mass_bias_attention see it (mass_bias_attention.py:96-107), else qkv's."""
        if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") in (
                torch.bfloat16, torch.float16):
            return torch.get_autocast_dtype("cuda")
        return qkv.dtype

    def _norm_params(self):
        if not self.use_qk_norm:
            return None, None
        return ((self.q_norm.weight, self.q_norm.bias, self.q_norm.eps),
                (self.k_norm.weight, self.k_norm.bias, self.k_norm.eps))

    def _fusable(self, qkv: Tensor, C: int, H: int) -> bool:
        return (qkv.is_cuda and C == H * 64 and qkv.stride(-1) == 1
                and qkv.dtype in (torch.bfloat16, torch.float16, torch.float32)
                and (not self.use_qk_norm or (self.q_norm.eps == self.k_norm.eps)))

    def compute_attention(self, qkv: Tensor, attn_bias=None, rope=None, token_plan=None) -> Tensor:
        assert attn_bias is None
        B, N, _ = qkv.shape
        C = self.qkv.in_features
        H = self.num_heads
        D = C // H
        if self._fusable(qkv, C, H):
            if token_plan is not None and rope is None:
                return self._merged_fused(qkv, token_plan, B, N, C, H)
            if token_plan is None and self._attention_dtype(qkv) in (torch.bfloat16, torch.float16):
                return self._dense_fused(qkv, rope, B, N, C, H)
        # General path: the reference's op sequence (torch LayerNorm / RoPE / SDPA).
        q, k, v = torch.unbind(qkv.reshape(B, N, 3, H, D), 2)
        q, k, v = [t.transpose(1, 2) for t in (q, k, v)]
        with profiling.span("global.qk_norm_rope") if token_plan is not None else _null():
            if self.use_qk_norm:
                q = self.q_norm(q)
                k = self.k_norm(k)
            if rope is not None:
                q, k = self.apply_rope(q, k, rope)
        if token_plan is None:
            x = F.scaled_dot_product_attention(q, k, v)
            return x.transpose(1, 2).reshape(B, N, C)
        return self._merged_attention(q, k, v, token_plan, B, N, C, H, D)

    def _dense_fused(self, qkv: Tensor, rope, B: int, N: int, C: int, H: int) -> Tensor:
        """Frame/register attention: fused LayerNorm+RoPE epilogue, then the HIP kernel."""
        dtype = self._attention_dtype(qkv)
        qn, kn = self._norm_params()
        rope_prefix = 0
        if rope is not None:
            rope_prefix = N - rope[0].shape[-2]
            assert rope_prefix >= 0
        rows = qkv.reshape(B * N, 3 * C)
        q, k, v = _kernels.qkv_epilogue(
            rows, H, tokens_in=N, q_norm=None if qn is None else qn[:2],
            k_norm=None if kn is None else kn[:2], eps=qn[2] if qn is not None else 1e-5,
            rope=rope, rope_prefix=rope_prefix, out_dtype=dtype)
        out = torch.empty((B, N, H, 64), device=qkv.device, dtype=dtype)
        _attention_into(q, k, v, None, out.permute(0, 2, 1, 3))
        return out.view(B, N, C)

    def _merged_fused(self, qkv: Tensor, plan, B: int, N: int, C: int, H: int) -> Tensor:
        """Merged global attention straight from the packed projection.

        q/k LayerNorm happens inside the compaction (every pooled row is normalised
        first, as the reference normalises before packing, attention.py:337-375), and
        the pooled operands are written once, in the attention dtype, head-major."""
        dtype = self._attention_dtype(qkv)
        qn, kn = self._norm_params()
        preserve_queries = getattr(plan, "preserve_queries", False)
        weighted = hasattr(plan, "compact_query_into")
        kept = plan.kept_tokens
        n_query = N if preserve_queries else getattr(plan, "query_kept_tokens", kept)
        device = qkv.device
        with profiling.span("global.qkv_compaction"):
            k_c = torch.empty((B, H, kept, 64), device=device, dtype=dtype)
            v_c = torch.empty((B, H, kept, 64), device=device, dtype=dtype)
            q_c = None if preserve_queries else torch.empty((B, H, n_query, 64), device=device, dtype=dtype)
            for b in range(B):
                rows = qkv[b]
                qs, ks, vs = rows[:, :C], rows[:, C:2 * C], rows[:, 2 * C:]
                if weighted:
                    if preserve_queries:
                        plan.compact_key_into(ks, k_c[b], layer_norm=kn)
                    else:
                        plan.compact_query_into(qs, q_c[b], layer_norm=qn)
                        plan.compact_into(ks, k_c[b], layer_norm=kn)
                    plan.compact_into(vs, v_c[b])
                elif hasattr(plan, "compact_multi_into") and rows.stride(-1) == 1 and k_c.dtype == rows.dtype and (
                        qn is None or kn is None or qn[2] == kn[2]):
                    # q, k and v share the plan's clusters: one launch reads each
                    # member's packed row once for all three.
                    outputs = [] if preserve_queries else [(0, q_c[b], qn)]
                    outputs += [(C, k_c[b], kn), (2 * C, v_c[b], None)]
                    plan.compact_multi_into(rows, outputs, b=b, merge=plan.pool_sources)
                else:
                    merge = plan.pool_sources
                    if not preserve_queries:
                        plan.compact_into(qs, q_c[b], b=b, merge=merge, layer_norm=qn)
                    plan.compact_into(ks, k_c[b], b=b, merge=merge, layer_norm=kn)
                    plan.compact_into(vs, v_c[b], b=b, merge=merge)
            if preserve_queries:
                q_c = _kernels.qkv_epilogue(
                    qkv.reshape(B * N, 3 * C), H, tokens_in=N,
                    q_norm=None if qn is None else qn[:2], eps=qn[2] if qn is not None else 1e-5,
                    want=(True, False, False), out_dtype=dtype)[0]
        bias = None
        log_mass = getattr(plan, "key_log_mass", None)
        if log_mass is not None:
            bias = log_mass.reshape(-1).to(dtype)
            if bias.numel() != kept:
                raise ValueError("log_key_mass length does not match key tokens")
        out = torch.empty((B, n_query, H, 64), device=device, dtype=dtype)
        x = out.permute(0, 2, 1, 3)  # [B, H, Nq, 64] view written in [B, Nq, H, 64] order
        special = output_indices = None
        if getattr(plan, "dense_special_queries", False):
            original, output_indices = self._special_mapping(plan, preserve_queries, B)
            with profiling.span("global.special_attention"):
                rows = qkv.reshape(N, 3 * C)
                _, dense_k, dense_v = _kernels.qkv_epilogue(
                    rows, H, tokens_in=N, k_norm=None if kn is None else kn[:2],
                    eps=kn[2] if kn is not None else 1e-5, want=(False, True, True), out_dtype=dtype)
                special_q = _kernels.qkv_epilogue(
                    rows, H, tokens_in=N, tokens_out=original.numel(), rows=original,
                    q_norm=None if qn is None else qn[:2], eps=qn[2] if qn is not None else 1e-5,
                    want=(True, False, False), out_dtype=dtype)[0]
                special = (special_q, dense_k, dense_v, None, torch.empty_like(special_q))
        self._attend(q_c, k_c, v_c, bias, x, special, output_indices)
        return out.view(B, n_query, C)

    def _merged_attention(self, q, k, v, plan, B, N, C, H, D) -> Tensor:
        """Merged attention from already normalised [B, H, N, 64] q/k/v views (RoPE case)."""
        if D != 64:
            raise ValueError("the initial fused kernel supports head_dim=64 only")
        preserve_queries = getattr(plan, "preserve_queries", False)
        kept = plan.kept_tokens
        n_query = N if preserve_queries else getattr(plan, "query_kept_tokens", kept)

        def head_major(rows: int, dtype: torch.dtype) -> Tensor:
            return torch.empty((B, H, rows, D), device=q.device, dtype=dtype)

        with profiling.span("global.qkv_compaction"):
            k_c = head_major(kept, k.dtype)
            v_c = head_major(kept, v.dtype)
            q_c = q if preserve_queries else head_major(n_query, q.dtype)
            for b in range(B):
                if preserve_queries:
                    if hasattr(plan, "compact_key_into"):
                        plan.compact_key_into(k[b], k_c[b])
                    else:
                        plan.compact_into(k[b], k_c[b], b=b, merge=plan.pool_sources)
                else:
                    if hasattr(plan, "compact_query_into"):
                        plan.compact_query_into(q[b], q_c[b])
                        plan.compact_into(k[b], k_c[b])
                    else:
                        plan.compact_into(q[b], q_c[b], b=b, merge=plan.pool_sources)
                        plan.compact_into(k[b], k_c[b], b=b, merge=plan.pool_sources)
                if hasattr(plan, "compact_query_into"):
                    plan.compact_into(v[b], v_c[b])
                else:
                    plan.compact_into(v[b], v_c[b], b=b, merge=plan.pool_sources)

        dtype = q.dtype
        if (torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16
                and q.dtype == torch.float32):
            dtype = torch.bfloat16
        qa, ka, va = q_c.to(dtype), k_c.to(dtype), v_c.to(dtype)
        bias = None
        log_mass = getattr(plan, "key_log_mass", None)
        if log_mass is not None:
            bias = log_mass.reshape(-1).to(dtype)
            if bias.numel() != kept:
                raise ValueError("log_key_mass length does not match key tokens")
        out = torch.empty((B, n_query, H, D), device=q.device, dtype=dtype)
        x = out.permute(0, 2, 1, 3)
        special = output_indices = None
        if getattr(plan, "dense_special_queries", False):
            original, output_indices = self._special_mapping(plan, preserve_queries, B)
            with profiling.span("global.special_attention"):
                special_q = q.index_select(2, original).to(dtype)
                exact = torch.empty((B, H, original.numel(), D), device=q.device, dtype=dtype)
                special = (special_q, k.to(dtype), v.to(dtype), None, exact)
        self._attend(qa, ka, va, bias, x, special, output_indices)
        return out.view(B, n_query, C)

    @staticmethod
    def _special_mapping(plan, preserve_queries: bool, B: int) -> tuple[Tensor, Tensor]:
        """Special-token query rows and the output rows they replace (attention.py:406-414)."""
        original = plan.special_query_original
        output_indices = original if preserve_queries else plan.special_query_compact
        if original is None or output_indices is None:
            raise RuntimeError("dense-special attention plan has no special-token mapping")
        if B != 1:
            raise RuntimeError("dense special queries need the batch-1 plans they are built for")
        return original, output_indices

    @staticmethod
    def _attend(q: Tensor, k: Tensor, v: Tensor, bias, x: Tensor, special, output_indices) -> None:
        """Merged attention into x; with a dense special-query pass, both in one launch.

        The special rows then replace the merged result's rows, as the
        reference's `x.index_copy_` does (attention.py:420)."""
        with profiling.span("global.main_attention"):
            if special is None:
                _attention_into(q, k, v, bias, x)
            else:
                _attention_pair_into((q, k, v, bias, x), special)
        if special is not None:
            with profiling.span("global.special_attention"):
                x.index_copy_(2, output_indices, special[4])


class SelfAttentionBlock(nn.Module):
    def __init__(self, dim: int, num_heads: int, ffn_ratio: float = 4.0, qkv_bias: bool = False,
                 proj_bias: bool = True, ffn_bias: bool = True, drop: float = 0.0,
                 attn_drop: float = 0.0, init_values=None, drop_path: float = 0.0,
                 act_layer: Callable[..., nn.Module] = nn.GELU,
                 norm_layer: Callable[..., nn.Module] = nn.LayerNorm,
                 attn_class: Callable[..., nn.Module] = SelfAttention,
                 ffn_layer: Callable[..., nn.Module] = Mlp, mask_k_bias: bool = False,
                 use_qk_norm: bool = False, device=None) -> None:
        super().__init__()
        self.norm1 = norm_layer(dim)
        self.attn = attn_class(dim, num_heads=num_heads, qkv_bias=qkv_bias, proj_bias=proj_bias,
                               attn_drop=attn_drop, proj_drop=drop, mask_k_bias=mask_k_bias,
                               use_qk_norm=use_qk_norm, device=device)
        self.ls1 = LayerScale(dim, init_values=init_values, device=device) if init_values else nn.Identity()
        self.norm2 = norm_layer(dim)
        self.mlp = ffn_layer(in_features=dim, hidden_features=int(dim * ffn_ratio),
                             act_layer=act_layer, drop=drop, bias=ffn_bias, device=device)
        self.ls2 = LayerScale(dim, init_values=init_values, device=device) if init_values else nn.Identity()
        self.sample_drop_ratio = drop_path

    def forward(self, x: Tensor, rope=None) -> Tensor:
        """Inference forward of block.py:89-129 (no stochastic depth)."""
        if self._fused_rows(x):
            return self._fused_tail(x, self.attn(self._norm1_input(x), rope=rope))
        x_attn = x + self.ls1(self.attn(self.norm1(x), rope=rope))
        return x_attn + self.ls2(self.mlp(self.norm2(x_attn)))

    def forward_compacted(self, x: Tensor, token_plan, *, normalized: Tensor = None) -> Tensor:
        """Inference-only compact-Q/K/V attention block (block.py:219-226).

        `normalized` is norm1(x) as the attention input: fp32 as the reference
        computes it, or already cast to the autocast dtype (`norm1_for_plan`)."""
        if self.training:
            raise RuntimeError("token compaction is inference-only")
        if normalized is None:
            normalized = self._norm1_input(x) if self._fused_rows(x) else self.norm1(x)
        if self._fused_rows(x):
            self.attn._check_hooks()
            y = self.attn._forward_merged(normalized, None, None, token_plan)
            restore_map_for = getattr(token_plan, "restore_map_for", None)
            restore_map = restore_map_for(y) if restore_map_for is not None else None
            if restore_map is None:
                with profiling.span("global.update_restore"):
                    y = token_plan.restore(y)
                return self._fused_tail(x, y)
            return self._fused_restore_tail(x, y[0], *restore_map)
        x_attn = x + self.ls1(self.attn(normalized, token_plan=token_plan))
        return x_attn + self.ls2(self.mlp(self.norm2(x_attn)))

    def norm1_for_plan(self, x: Tensor) -> tuple[Tensor, Tensor]:
        """(norm1(x) in fp32 for the planners, the same rows as the attention input).

        With the fused row kernel both come from one pass, the second already in
        the autocast dtype the qkv Linear would cast it to; otherwise both are
        the reference's fp32 `norm1(x)` (aggregator.py:1002)."""
        if self._fused_rows(x):
            _, h, h32 = _kernels.residual_layer_norm(x, norm=_ln_args(self.norm1),
                                                     norm_dtype=_autocast_dtype(), norm_f32=True)
            return h32, h
        n = self.norm1(x)
        return n, n

    def norm1_unit_rows(self, x: Tensor, eps: float = 1e-12) -> tuple[Tensor, Tensor] | None:
        """(F.normalize(norm1(x), eps).to(bf16), norm1(x) in bf16) from one row pass.

        The first tensor is the FastVGGT matcher's input (token_merging.py:1102-1103),
        equal bit for bit to normalize_rows of the fp32 norm1 rows; the second is the
        qkv input.  None when the fused row kernel does not apply (or autocast is
        not bf16); then use `norm1_for_plan`."""
        if not self._fused_rows(x) or _autocast_dtype() != torch.bfloat16:
            return None
        _, h, _, unit = _kernels.residual_layer_norm(x, norm=_ln_args(self.norm1),
                                                     norm_dtype=torch.bfloat16, unit_eps=eps)
        return unit, h

    # ------------------------------------------------ fused residual rows ----
    def _fused_rows(self, x: Tensor) -> bool:
        """The residual stream runs through vgo_residual_layer_norm: inference under
        bf16/f16 autocast on an fp32 stream, torch LayerNorms over the last dim,
        LayerScale (not in place) or Identity, rows the kernel can address."""
        if torch.is_grad_enabled() or self.training or not x.is_cuda or x.dtype != torch.float32:
            return False
        if _autocast_dtype() is None:
            return False
        dim = x.shape[-1]
        for norm in (self.norm1, self.norm2):
            if type(norm) is not nn.LayerNorm or tuple(norm.normalized_shape) != (dim,):
                return False
        for ls in (self.ls1, self.ls2):
            if not (type(ls) is nn.Identity or (type(ls) is LayerScale and not ls.inplace)):
                return False
        # Row starts must be 16-byte aligned (the kernel's vector loads): eagerly, a view
        # at an odd storage offset takes the torch path.  A traced graph sees neither
        # pointers nor storage offsets; there the library's own check raises for such a
        # view (tensors of torch's allocator with dim % 4 == 0 are always aligned).
        aligned = torch.compiler.is_compiling() or x.data_ptr() % 16 == 0
        return dim % 4 == 0 and dim <= 2048 and x.is_contiguous() and aligned

    def _norm1_input(self, x: Tensor) -> Tensor:
        return _kernels.residual_layer_norm(x, norm=_ln_args(self.norm1), norm_dtype=_autocast_dtype())[1]

    def _fused_restore_tail(self, x: Tensor, table: Tensor, index: Tensor, weight: Tensor) -> Tensor:
        """_fused_tail of the plan's restore of `table` (the merged rows): the first row
        pass projects each row's parents itself, so the restored rows never go to memory.
        The `global.update_restore` label then spans restore, residual add and norm2."""
        with profiling.span("global.update_restore"):
            x_attn, h = _kernels.restore_residual_layer_norm(
                x, table, index, weight, _ls_gamma(self.ls1), _ln_args(self.norm2),
                norm_dtype=_autocast_dtype())
        out, _, _ = _kernels.residual_layer_norm(x_attn, self.mlp(h).reshape(x.shape),
                                                 _ls_gamma(self.ls2))
        return out

    def _fused_tail(self, x: Tensor, y: Tensor) -> Tensor:
        """x_attn = x + ls1(y); return x_attn + ls2(mlp(norm2(x_attn))) with two row passes."""
        if y.shape != x.shape or y.stride(-1) != 1:
            y = y.reshape(x.shape).contiguous()
        x_attn, h, _ = _kernels.residual_layer_norm(x, y, _ls_gamma(self.ls1), _ln_args(self.norm2),
                                                    norm_dtype=_autocast_dtype())
        out, _, _ = _kernels.residual_layer_norm(x_attn, self.mlp(h).reshape(x.shape),
                                                 _ls_gamma(self.ls2))
        return out


def _autocast_dtype() -> torch.dtype | None:
    if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") in (
            torch.bfloat16, torch.float16):
        return torch.get_autocast_dtype("cuda")
    return None


def _ln_args(norm: nn.LayerNorm):
    return (norm.weight, norm.bias, norm.eps)


def _ls_gamma(ls: nn.Module) -> Tensor | None:
    return ls.gamma if isinstance(ls, LayerScale) else None


def init_weights_vit(module: nn.Module, name: str = "") -> None:
    """Random init of vggt_omega/models/layers/vision_transformer.py:47-63."""
    if isinstance(module, nn.Linear):
        torch.nn.init.trunc_normal_(module.weight, std=0.02)
        if module.bias is not None:
            nn.init.zeros_(module.bias)
        if getattr(module, "bias_mask", None) is not None:
            o = module.out_features
            module.bias_mask.fill_(1)
            module.bias_mask[o // 3: 2 * o // 3].fill_(0)
    if isinstance(module, (nn.LayerNorm, LayerScale)):
        module.reset_parameters()


def rope_sincos(H: int, W: int, head_dim: int, base: float = 100.0,
                device=None) -> tuple[Tensor, Tensor]:
    """Axial RoPE tables of RopePositionEmbedding(normalize_coords="max") at inference
    (vggt_omega/models/layers/rope_position_encoding.py:51-127), fp32 [H*W, head_dim]."""
    dd = dict(device=device, dtype=torch.float32)
    periods = base ** (2 * torch.arange(head_dim // 4, **dd) / (head_dim // 2))
    m = max(H, W)
    coords_h = torch.arange(0.5, H, **dd) / m
    coords_w = torch.arange(0.5, W, **dd) / m
    coords = torch.stack(torch.meshgrid(coords_h, coords_w, indexing="ij"), dim=-1).flatten(0, 1)
    coords = 2.0 * coords - 1.0
    angles = 2 * math.pi * coords[:, :, None] / periods[None, None, :]
    angles = angles.flatten(1, 2).tile(2)
    return torch.sin(angles), torch.cos(angles)
