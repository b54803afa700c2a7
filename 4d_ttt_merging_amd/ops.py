"""torch.library operators of the merged global-attention path (namespace `vgo`).

Every kernel a merged block launches is a `torch.ops.vgo.*` operator, so the
dispatcher, `torch.compile` and fake-tensor tracing see them as single ops:

* `vgo::mass_bias_attention(q, k, v, log_key_mass?) -> Tensor`  -- the reference's
  operator (vggt_omega/models/mass_bias_attention.py:85-129) on already-cast
  inputs; `vgo::attention_into` / `vgo::attention_pair_into` write into given
  (strided) outputs, the pair form also running the dense special-query pass of
  vggt_omega/models/layers/attention.py:406-422 in the same launch;
* `vgo::top4_project(table, index, weight) -> Tensor`, `vgo::top4_project_into` and
  `vgo::top4_project_ordered_into` -- the plans' restore (token_merging.py:387-414,
  193-196);
* `vgo::compact_into`, `vgo::compact_multi_into` -- Q/K/V compaction
  (token_merging.py:343-385, 176-191) with the q/k LayerNorm fused;
* `vgo::qkv_epilogue` -- the packed projection split into head-major q/k/v with
  LayerNorm64 and RoPE (layers/attention.py:243-262, 334-341);
* `vgo::residual_layer_norm` -- LayerScale, residual add, LayerNorm and the
  autocast cast of a block (layers/block.py:126-127, 219-226);
  `vgo::restore_residual_layer_norm` -- the same with the plan restore
  (token_merging.py:387-414, 193-196) computed in the pass.

Each has a CUDA (HIP) implementation that calls `libvgo.so` through its C ABI
and a fake implementation that only describes the outputs (for tracing).
There is no CPU implementation: CPU tensors fail in the dispatcher.
"""
from typing import List, Optional

import torch

from . import _kernels
from . import mass_bias_attention as _mba
from . import projection as _proj

Tensor = torch.Tensor


def _split_code(split: int) -> Optional[bool]:
    return None if split < 0 else bool(split)


# ---------------------------------------------------------------- attention ----
@torch.library.custom_op("vgo::mass_bias_attention", mutates_args=(), device_types="cuda")
def mass_bias_attention(q: Tensor, k: Tensor, v: Tensor, log_key_mass: Optional[Tensor]) -> Tensor:
    """softmax(q k^T / 8 + log_key_mass) v for [B, H, N, 64] q/k/v of one dtype; the bias
    already rounded to that dtype (or None); a new contiguous output."""
    out = torch.empty(q.shape, device=q.device, dtype=q.dtype)
    _mba._attention_into_impl(q, k, v, log_key_mass, out)
    return out


@mass_bias_attention.register_fake
def _(q, k, v, log_key_mass):
    return torch.empty(q.shape, device=q.device, dtype=q.dtype)


@torch.library.custom_op("vgo::attention_into", mutates_args={"out"}, device_types="cuda")
def attention_into(q: Tensor, k: Tensor, v: Tensor, bias: Optional[Tensor], out: Tensor,
                   split: int) -> None:
    """The same into `out` (any strides with a unit channel stride); split: -1 picks the
    entry by key length, 0 the entry without a workspace, 1 the workspace entry."""
    _mba._attention_into_impl(q, k, v, bias, out, split=_split_code(split))


@attention_into.register_fake
def _(q, k, v, bias, out, split):
    return None


@torch.library.custom_op("vgo::attention_pair_into", mutates_args={"out", "special_out"},
                         device_types="cuda")
def attention_pair_into(q: Tensor, k: Tensor, v: Tensor, bias: Optional[Tensor], out: Tensor,
                        special_q: Tensor, special_k: Tensor, special_v: Tensor,
                        special_bias: Optional[Tensor], special_out: Tensor) -> None:
    """Merged attention and the dense special-query pass in one launch."""
    _mba._attention_pair_into_impl((q, k, v, bias, out),
                                   (special_q, special_k, special_v, special_bias, special_out))


@attention_pair_into.register_fake
def _(q, k, v, bias, out, special_q, special_k, special_v, special_bias, special_out):
    return None


# --------------------------------------------------------------- projection ----
@torch.library.custom_op("vgo::top4_project", mutates_args=(), device_types="cuda")
def top4_project(table: Tensor, index: Tensor, weight: Tensor) -> Tensor:
    """out[i] = sum_c weight[i, c] * table[index[i, c]]: table [M, D], index [N, 4] int32,
    weight [N, 4] fp32 -> [N, D] in the table's dtype."""
    return _proj._top4_project_impl(table, index, weight)


@top4_project.register_fake
def _(table, index, weight):
    return table.new_empty((index.shape[0], table.shape[1]))


@torch.library.custom_op("vgo::top4_project_into", mutates_args={"out"}, device_types="cuda")
def top4_project_into(table: Tensor, index: Tensor, weight: Tensor, out: Tensor) -> None:
    _proj._top4_project_impl(table, index, weight, out=out)


@top4_project_into.register_fake
def _(table, index, weight, out):
    return None


@torch.library.custom_op("vgo::top4_project_ordered_into", mutates_args={"out"}, device_types="cuda")
def top4_project_ordered_into(table: Tensor, index: Tensor, weight: Tensor, order: Tensor,
                              out: Tensor) -> None:
    """top4_project_into with the rows computed in `order` (same result)."""
    _proj._top4_project_impl(table, index, weight, out=out, order=order)


@top4_project_ordered_into.register_fake
def _(table, index, weight, order, out):
    return None


# --------------------------------------------------------------- compaction ----
@torch.library.custom_op("vgo::compact_into", mutates_args={"out"}, device_types="cuda")
def compact_into(x: Tensor, out: Tensor, base_rows: Optional[Tensor], offsets: Tensor,
                 segs_per_row: int, items: Optional[Tensor], item_shift: int,
                 item_rows: Optional[Tensor], weights: Optional[Tensor],
                 normalizer: Optional[Tensor], ln_weight: Optional[Tensor],
                 ln_bias: Optional[Tensor], ln_eps: float) -> None:
    """Segmented weighted pooling of x ([N, C] or [H, N, 64] view) into out."""
    layer_norm = None if ln_weight is None else (ln_weight, ln_bias, ln_eps)
    _kernels._compact_into_impl(x, out, base_rows=base_rows, offsets=offsets,
                                segs_per_row=segs_per_row, items=items, item_shift=item_shift,
                                item_rows=item_rows, weights=weights, normalizer=normalizer,
                                layer_norm=layer_norm)


@compact_into.register_fake
def _(x, out, base_rows, offsets, segs_per_row, items, item_shift, item_rows, weights,
      normalizer, ln_weight, ln_bias, ln_eps):
    return None


@torch.library.custom_op("vgo::compact_multi_into", mutates_args={"outs"}, device_types="cuda")
def compact_multi_into(x: Tensor, x_offsets: List[int], outs: List[Tensor],
                       ln_weights: List[Optional[Tensor]], ln_biases: List[Optional[Tensor]],
                       ln_eps: List[float], base_rows: Optional[Tensor], offsets: Tensor,
                       segs_per_row: int, items: Optional[Tensor], item_shift: int,
                       item_rows: Optional[Tensor], weights: Optional[Tensor],
                       normalizer: Optional[Tensor]) -> None:
    """1-3 channel ranges of one [N, W] row table pooled into outs in one launch."""
    outputs = [(off, out, None if w is None else (w, b, eps))
               for off, out, w, b, eps in zip(x_offsets, outs, ln_weights, ln_biases, ln_eps)]
    _kernels._compact_multi_into_impl(x, outputs, base_rows=base_rows, offsets=offsets,
                                      segs_per_row=segs_per_row, items=items, item_shift=item_shift,
                                      item_rows=item_rows, weights=weights, normalizer=normalizer)


@compact_multi_into.register_fake
def _(x, x_offsets, outs, ln_weights, ln_biases, ln_eps, base_rows, offsets, segs_per_row, items,
      item_shift, item_rows, weights, normalizer):
    return None


# ------------------------------------------------------------ QKV epilogue ----
def _epilogue_shape(qkv, heads, tokens_out, rows):
    n_out = qkv.shape[0] if rows is None else rows.numel()
    return (n_out // tokens_out, heads, tokens_out, 64)


@torch.library.custom_op("vgo::qkv_epilogue", mutates_args=(), device_types="cuda")
def qkv_epilogue(qkv: Tensor, heads: int, tokens_in: int, tokens_out: int, rows: Optional[Tensor],
                 q_weight: Optional[Tensor], q_bias: Optional[Tensor], k_weight: Optional[Tensor],
                 k_bias: Optional[Tensor], eps: float, rope_sin: Optional[Tensor],
                 rope_cos: Optional[Tensor], rope_prefix: int, want: List[bool],
                 out_dtype: torch.dtype) -> List[Tensor]:
    """[q, k, v] head-major [S, H, tokens_out, 64]; an unwanted one is an empty tensor."""
    outs = _kernels._qkv_epilogue_impl(
        qkv, heads, tokens_in=tokens_in, tokens_out=tokens_out, rows=rows,
        q_norm=None if q_weight is None else (q_weight, q_bias),
        k_norm=None if k_weight is None else (k_weight, k_bias), eps=eps,
        rope=None if rope_sin is None else (rope_sin, rope_cos), rope_prefix=rope_prefix,
        want=tuple(want), out_dtype=out_dtype)
    return [o if o is not None else qkv.new_empty((0,), dtype=out_dtype) for o in outs]


@qkv_epilogue.register_fake
def _(qkv, heads, tokens_in, tokens_out, rows, q_weight, q_bias, k_weight, k_bias, eps, rope_sin,
      rope_cos, rope_prefix, want, out_dtype):
    shape = _epilogue_shape(qkv, heads, tokens_out, rows)
    return [qkv.new_empty(shape if w else (0,), dtype=out_dtype) for w in want]


# ------------------------------------------------------------ residual rows ----
@torch.library.custom_op("vgo::residual_layer_norm", mutates_args=(), device_types="cuda")
def residual_layer_norm(x: Tensor, branch: Optional[Tensor], gamma: Optional[Tensor],
                        ln_weight: Optional[Tensor], ln_bias: Optional[Tensor], eps: float,
                        has_norm: bool, write_sum: bool, norm_dtype: Optional[torch.dtype],
                        norm_f32: bool, unit_eps: float) -> List[Tensor]:
    """[x + gamma * branch, LN in norm_dtype, LN in fp32, LN / ||LN||]; outputs not asked for
    (no branch or write_sum false, no norm / norm_dtype, norm_f32 false, unit_eps < 0) are
    empty tensors."""
    res = _kernels._residual_layer_norm_impl(
        x, branch, gamma, (ln_weight, ln_bias, eps) if has_norm else None, write_sum=write_sum,
        norm_dtype=norm_dtype, norm_f32=norm_f32, unit_eps=None if unit_eps < 0 else unit_eps)
    res = list(res) + [None] * (4 - len(res))
    return [t if t is not None else x.new_empty((0,)) for t in res]


@residual_layer_norm.register_fake
def _(x, branch, gamma, ln_weight, ln_bias, eps, has_norm, write_sum, norm_dtype, norm_f32, unit_eps):
    empty = x.new_empty((0,))
    total = x.new_empty(x.shape) if write_sum and branch is not None else empty
    normed = x.new_empty(x.shape, dtype=norm_dtype) if has_norm and norm_dtype is not None else empty
    normed32 = x.new_empty(x.shape) if has_norm and norm_f32 else empty
    unit = x.new_empty(x.shape, dtype=norm_dtype) if unit_eps >= 0 and norm_dtype is not None else empty
    return [total, normed, normed32, unit]


@torch.library.custom_op("vgo::restore_residual_layer_norm", mutates_args=(), device_types="cuda")
def restore_residual_layer_norm(x: Tensor, table: Tensor, index: Tensor, weight: Optional[Tensor],
                                gamma: Optional[Tensor], ln_weight: Optional[Tensor],
                                ln_bias: Optional[Tensor], eps: float,
                                norm_dtype: torch.dtype) -> List[Tensor]:
    """[x + gamma * restore(table), LN of that in norm_dtype] with restore = the top-4
    projection of `table` by (index, weight) -- or, without weight, the one-hot gather
    table[index] -- never written to memory."""
    return list(_kernels._restore_residual_layer_norm_impl(x, table, index, weight, gamma,
                                                           (ln_weight, ln_bias, eps), norm_dtype))


@restore_residual_layer_norm.register_fake
def _(x, table, index, weight, gamma, ln_weight, ln_bias, eps, norm_dtype):
    return [x.new_empty(x.shape), x.new_empty(x.shape, dtype=norm_dtype)]
