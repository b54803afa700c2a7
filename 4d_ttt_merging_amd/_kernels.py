"""Typed wrappers over the merge-path entry points of `libvgo.so`.

Each wrapper validates shapes/dtypes on the host, allocates outputs and
workspaces with torch (device memory only), and launches on torch's current
stream.  No wrapper synchronises the device.  The kernels a merged block runs
(compaction, the QKV epilogue, the residual rows) go through the torch.library
operators of `ops.py` (`torch.ops.vgo.*`), whose implementations are the
`_*_impl` functions here; the plan-building kernels are called directly.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


def _c(ptr_or_tensor):
    if ptr_or_tensor is None:
        return None
    return ptr_or_tensor.data_ptr()


def normalize_rows(x: torch.Tensor, rows: torch.Tensor | None, eps: float,
                   out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """out[r] = x[rows[r]] / max(||x[rows[r]]||, eps) for a 2-D x (unit column stride)."""
    lib = _lib.load()
    _lib.require_gpu(x, rows)
    if x.ndim != 2 or x.stride(-1) != 1:
        x = x.reshape(-1, x.shape[-1]).contiguous()
    if rows is not None:
        rows = rows.to(torch.int64).contiguous()
    n = x.shape[0] if rows is None else rows.numel()
    out = torch.empty((n, x.shape[1]), device=x.device, dtype=out_dtype)
    status = lib.vgo_normalize_rows(
        x.data_ptr(), x.stride(0), x.shape[0], _lib.dtype_code(x.dtype), _c(rows), n, x.shape[1],
        float(eps), out.data_ptr(), out.stride(0), _lib.dtype_code(out_dtype), _lib.stream_of(x))
    _lib.check(status)
    return out


def similarity_topk(src: torch.Tensor, dictionary: torch.Tensor, topk: int, *,
                    src_rows: torch.Tensor | None = None,
                    n_src_device: torch.Tensor | None = None, n_src: int | None = None,
                    dict_ranges: tuple[int, int, int] | None = None,
                    index_map: torch.Tensor | None = None, want_values: bool = True,
                    index_dtype: torch.dtype = torch.int64,
                    scores: torch.Tensor | None = None,
                    out: tuple[torch.Tensor, torch.Tensor] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-K bf16 cosine matches of every source row against a dictionary.

    dict_ranges = (n0, off1, n_dict): dictionary position j reads row j for
    j < n0 and row off1 + j - n0 otherwise (default: all rows).  Returns
    (values [n, K] fp32, indices [n, K]) with ties going to the lower position,
    written into `out` = (values, indices) when given (contiguous, those shapes).
    """
    lib = _lib.load()
    _lib.require_gpu(src, dictionary, src_rows, n_src_device, index_map, scores)
    if src.dtype != torch.bfloat16 or dictionary.dtype != torch.bfloat16:
        raise ValueError("similarity_topk expects bf16 operands")
    if src.stride(-1) != 1:
        src = src.contiguous()
    if dictionary.stride(-1) != 1:
        dictionary = dictionary.contiguous()
    if dict_ranges is None:
        dict_ranges = (dictionary.shape[0], 0, dictionary.shape[0])
    n0, off1, n_dict = dict_ranges
    if n_src is None:
        n_src = src.shape[0] if src_rows is None else src_rows.numel()
    if src_rows is not None:
        src_rows = src_rows.to(torch.int64).contiguous()
    parts = ctypes.c_int(0)
    need = ctypes.c_size_t(0)
    _lib.check(lib.vgo_similarity_topk_workspace(n_src, n_dict, topk, ctypes.byref(parts),
                                                 ctypes.byref(need)))
    workspace = torch.empty(max(1, need.value // 8), device=src.device, dtype=torch.int64)
    if out is not None:
        values, index = out
        _lib.require_gpu(values, index)
        if (values.shape != (n_src, topk) or index.shape != (n_src, topk) or not values.is_contiguous()
                or not index.is_contiguous() or values.dtype != torch.float32 or index.dtype != index_dtype):
            raise ValueError("similarity_topk: `out` must be contiguous [n, K] fp32 values and indices")
    else:
        values = torch.empty((n_src, topk), device=src.device, dtype=torch.float32) if want_values else None
        index = torch.empty((n_src, topk), device=src.device, dtype=index_dtype)
    idx64 = index if index_dtype == torch.int64 else None
    idx32 = index if index_dtype == torch.int32 else None
    if index_map is not None:
        index_map = index_map.to(torch.int64).contiguous()
    status = lib.vgo_similarity_topk(
        src.data_ptr(), src.stride(0), src.shape[0], _c(src_rows), _c(n_src_device), n_src,
        dictionary.data_ptr(), dictionary.stride(0), dictionary.shape[0], n0, off1, n_dict,
        src.shape[1], topk, workspace.data_ptr(), workspace.numel() * 8, _c(values), _c(idx64),
        _c(idx32), _c(index_map), _c(scores), 0 if scores is None else scores.stride(0),
        _lib.stream_of(src))
    _lib.check(status)
    return values, index


def csr_build(keys: torch.Tensor, n_buckets: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Stable bucket order: (order [n] int32 item ids, offsets [n_buckets+1] int32)."""
    lib = _lib.load()
    _lib.require_gpu(keys)
    keys = keys.to(torch.int32).contiguous()
    n = keys.numel()
    need = ctypes.c_size_t(0)
    _lib.check(lib.vgo_csr_workspace(n, n_buckets, ctypes.byref(need)))
    workspace = torch.empty(max(256, need.value + 256), device=keys.device, dtype=torch.uint8)
    base = workspace.data_ptr()
    pad = (-base) % 256
    order = torch.empty(n, device=keys.device, dtype=torch.int32)
    offsets = torch.empty(n_buckets + 1, device=keys.device, dtype=torch.int32)
    status = lib.vgo_csr_build(keys.data_ptr(), n, n_buckets, base + pad, need.value,
                               order.data_ptr(), offsets.data_ptr(), _lib.stream_of(keys))
    _lib.check(status)
    return order, offsets


def segment_mass(offsets: torch.Tensor, segs_per_row: int, order: torch.Tensor,
                 weights: torch.Tensor | None, rows: int, start: float,
                 want_log: bool = True) -> tuple[torch.Tensor, torch.Tensor | None]:
    lib = _lib.load()
    device = offsets.device
    mass = torch.empty(rows, device=device, dtype=torch.float32)
    log_mass = torch.empty(rows, device=device, dtype=torch.float32) if want_log else None
    if weights is not None:
        weights = weights.to(torch.float32).contiguous()
    status = lib.vgo_segment_mass(
        offsets.data_ptr(), segs_per_row, order.data_ptr(), _c(weights),
        0 if weights is None else weights.numel(), rows, float(start), mass.data_ptr(),
        _c(log_mass), _lib.stream_of(offsets))
    _lib.check(status)
    return mass, log_mass


def token_layout(t: torch.Tensor) -> tuple[int, int]:
    """(token stride, head stride) of a [N, C] or [H, N, 64] view for vgo_compact."""
    if t.ndim == 2:
        if t.stride(1) != 1:
            raise ValueError("channel stride must be 1")
        return t.stride(0), 64
    if t.ndim == 3 and t.shape[-1] == 64 and t.stride(-1) == 1:
        return t.stride(1), t.stride(0)
    raise ValueError("compaction operands must be [N, C] or [H, N, 64] views")


def _compact_into_impl(x: torch.Tensor, out: torch.Tensor, *, base_rows: torch.Tensor | None,
                 offsets: torch.Tensor, segs_per_row: int, items: torch.Tensor | None,
                 item_shift: int, item_rows: torch.Tensor | None, weights: torch.Tensor | None,
                 normalizer: torch.Tensor | None,
                 layer_norm: tuple[torch.Tensor, torch.Tensor, float] | None = None) -> torch.Tensor:
    """Segmented weighted pooling; x/out are [N, C] or head-major [H, N, 64] views.

    `layer_norm` = (weight [64], bias [64], eps) normalises every gathered row per
    64-channel head first; `out` may be narrower than `x` (one final rounding).
    """
    lib = _lib.load()
    _lib.require_gpu(x, out)
    xts, xhs = token_layout(x)
    ots, ohs = token_layout(out)
    n_rows_x = x.shape[0] if x.ndim == 2 else x.shape[1]
    rows = out.shape[0] if out.ndim == 2 else out.shape[1]
    dim = out.shape[1] if out.ndim == 2 else out.shape[0] * 64
    ln_w = ln_b = None
    ln_eps = 0.0
    if layer_norm is not None:
        ln_w, ln_b, ln_eps = layer_norm
        ln_w = ln_w.detach().to(torch.float32).contiguous()
        ln_b = ln_b.detach().to(torch.float32).contiguous()
    status = lib.vgo_compact(
        x.data_ptr(), xts, xhs, n_rows_x, _c(base_rows), offsets.data_ptr(), segs_per_row,
        _c(items), item_shift, _c(item_rows), _c(weights), 0 if weights is None else weights.numel(),
        _c(normalizer), rows, dim, _c(ln_w), _c(ln_b), float(ln_eps), out.data_ptr(), ots, ohs,
        _lib.dtype_code(x.dtype), _lib.dtype_code(out.dtype), _lib.stream_of(x))
    _lib.check(status)
    return out


def _compact_multi_into_impl(x: torch.Tensor, outputs, *, base_rows: torch.Tensor | None,
                       offsets: torch.Tensor, segs_per_row: int, items: torch.Tensor | None,
                       item_shift: int, item_rows: torch.Tensor | None, weights: torch.Tensor | None,
                       normalizer: torch.Tensor | None) -> None:
    """compact_into for 1-3 outputs sharing the segments, in one launch.

    `x` is the [N, W] row table (unit channel stride); `outputs` holds
    (channel offset, out, layer_norm or None) per output, out being an
    [K, C] or head-major [H, K, 64] view as in compact_into (all outputs one
    dtype, that of x; one shared LayerNorm eps)."""
    lib = _lib.load()
    _lib.require_gpu(x, *[o[1] for o in outputs])
    n = len(outputs)
    if not 1 <= n <= 3:
        raise ValueError(f"compact_multi_into: 1-3 outputs, got {n}")
    if x.ndim != 2 or x.stride(1) != 1:
        raise ValueError("compact_multi_into: x must be an [N, W] row table with unit channel stride")
    first = outputs[0][1]
    rows = first.shape[0] if first.ndim == 2 else first.shape[1]
    dim = first.shape[1] if first.ndim == 2 else first.shape[0] * 64
    eps_values = set()
    for off, out, ln in outputs:
        o_rows = out.shape[0] if out.ndim == 2 else out.shape[1]
        o_dim = out.shape[1] if out.ndim == 2 else out.shape[0] * 64
        if (o_rows, o_dim) != (rows, dim):
            raise ValueError(f"compact_multi_into: every output must be {rows} rows x {dim} "
                             f"channels, got {o_rows} x {o_dim}")
        if int(off) < 0 or int(off) + dim > x.shape[1]:
            raise ValueError(f"compact_multi_into: channels {int(off)}..{int(off) + dim} lie "
                             f"outside x's {x.shape[1]}")
        if ln is not None:
            eps_values.add(float(ln[2]))
    if len(eps_values) > 1:
        raise ValueError("compact_multi_into: the outputs' LayerNorms must share one eps")
    keep = []
    offs = (ctypes.c_int64 * n)(*[int(o[0]) for o in outputs])
    lw = (ctypes.c_void_p * n)()
    lb = (ctypes.c_void_p * n)()
    outs = (ctypes.c_void_p * n)()
    ots = (ctypes.c_int64 * n)()
    ohs = (ctypes.c_int64 * n)()
    eps = 0.0
    for g, (_, out, ln) in enumerate(outputs):
        if out.dtype != x.dtype:
            raise ValueError("compact_multi_into: outputs must have x's dtype")
        ots[g], ohs[g] = token_layout(out)
        outs[g] = out.data_ptr()
        if ln is not None:
            w = ln[0].detach().to(torch.float32).contiguous()
            b = ln[1].detach().to(torch.float32).contiguous()
            keep += [w, b]
            lw[g], lb[g], eps = w.data_ptr(), b.data_ptr(), float(ln[2])
    status = lib.vgo_compact_multi(
        x.data_ptr(), x.stride(0), 64, x.shape[0], _c(base_rows), offsets.data_ptr(), segs_per_row,
        _c(items), item_shift, _c(item_rows), _c(weights), 0 if weights is None else weights.numel(),
        _c(normalizer), rows, dim, n, offs, lw, lb, eps, outs, ots, ohs, _lib.dtype_code(x.dtype),
        _lib.stream_of(x))
    _lib.check(status)
    del keep


def restore_map(total: int, *, device: torch.device, keep: torch.Tensor | None = None,
                source: torch.Tensor | None = None, parent: torch.Tensor | None = None,
                weight: torch.Tensor | None = None,
                inverse: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense [total, 4] (int32 index, fp32 weight) rows consumed by top4_project."""
    lib = _lib.load()
    # With `inverse` the kernel writes every row; otherwise rows outside keep and
    # source stay zero (zero weights, as the reference's `new_zeros` output).
    alloc = torch.empty if inverse is not None else torch.zeros
    index_out = alloc((total, 4), device=device, dtype=torch.int32)
    weight_out = alloc((total, 4), device=device, dtype=torch.float32)
    n_keep = 0 if keep is None else keep.numel()
    n_source = 0 if source is None else source.numel()
    status = lib.vgo_restore_map(
        _c(keep), n_keep, _c(source), _c(parent), _c(weight), n_source, _c(inverse), total,
        index_out.data_ptr(), weight_out.data_ptr(), torch.cuda.current_stream(device).cuda_stream)
    _lib.check(status)
    return index_out, weight_out


def _qkv_epilogue_impl(qkv: torch.Tensor, heads: int, *, tokens_in: int, tokens_out: int | None = None,
                 rows: torch.Tensor | None = None, q_norm=None, k_norm=None, eps: float = 1e-5,
                 rope: tuple[torch.Tensor, torch.Tensor] | None = None, rope_prefix: int = 0,
                 want=(True, True, True), out_dtype: torch.dtype | None = None):
    """Split packed qkv rows [T, 3C] into head-major [S, H, tokens_out, 64] q/k/v.

    q_norm / k_norm are (weight, bias) of the per-head LayerNorm(64); rope is
    (sin, cos) [positions, 64] applied to tokens at position >= rope_prefix of
    each tokens_in-long sequence.  Returns (q, k, v) with None for unwanted ones.
    """
    lib = _lib.load()
    _lib.require_gpu(qkv, rows)
    if qkv.ndim != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv_epilogue expects [rows, 3C] projection rows")
    out_dtype = out_dtype or qkv.dtype
    n_out = qkv.shape[0] if rows is None else rows.numel()
    tokens_out = tokens_out or tokens_in
    seqs = n_out // tokens_out
    if rows is not None:
        rows = rows.to(torch.int64).contiguous()
    outs = [torch.empty((seqs, heads, tokens_out, 64), device=qkv.device, dtype=out_dtype) if w else None
            for w in want]
    f32 = lambda t: None if t is None else t.detach().to(torch.float32).contiguous()  # noqa: E731
    qw, qb = (f32(q_norm[0]), f32(q_norm[1])) if q_norm is not None else (None, None)
    kw, kb = (f32(k_norm[0]), f32(k_norm[1])) if k_norm is not None else (None, None)
    rs = rc = None
    rope_rows = 0
    if rope is not None:
        rs, rc = f32(rope[0]), f32(rope[1])
        rope_rows = rs.shape[0]
    status = lib.vgo_qkv_epilogue(
        qkv.data_ptr(), qkv.stride(0), qkv.shape[0], _lib.dtype_code(qkv.dtype), _c(rows), n_out,
        tokens_in, tokens_out, heads, _c(qw), _c(qb), _c(kw), _c(kb), float(eps), _c(rs), _c(rc),
        rope_prefix, rope_rows, _c(outs[0]), _c(outs[1]), _c(outs[2]), _lib.dtype_code(out_dtype),
        _lib.stream_of(qkv))
    _lib.check(status)
    return tuple(outs)


def _residual_layer_norm_impl(x: torch.Tensor, branch: torch.Tensor | None = None,
                        gamma: torch.Tensor | None = None,
                        norm: tuple[torch.Tensor | None, torch.Tensor | None, float] | None = None, *,
                        write_sum: bool = True, norm_dtype: torch.dtype | None = torch.bfloat16,
                        norm_f32: bool = False, unit_eps: float | None = None):
    """One pass over fp32 rows [..., dim]: s = x + gamma * branch, n = LayerNorm(s).

    `norm` = (weight, bias, eps) of the LayerNorm (affine tensors may be None).
    Returns (s, n, n_f32[, u]): s when `write_sum` (and a branch is given), n in
    `norm_dtype` and its fp32 copy when asked, else None in their places; with
    `unit_eps`, also u = n / max(||n||, unit_eps) in `norm_dtype` (the planners'
    F.normalize front end, equal bit for bit to normalize_rows of n_f32).
    """
    lib = _lib.load()
    _lib.require_gpu(x, branch)
    if x.dtype != torch.float32:
        raise ValueError("residual_layer_norm: x must be float32")
    dim = x.shape[-1]
    rows = x.reshape(-1, dim)
    b_rows = None
    if branch is not None:
        if branch.shape != x.shape:
            raise ValueError(f"residual_layer_norm: branch {tuple(branch.shape)} != x {tuple(x.shape)}")
        b_rows = branch.reshape(-1, dim)
    n = rows.shape[0]
    total = (torch.empty_like(x, memory_format=torch.contiguous_format)
             if write_sum and branch is not None else None)
    w = b = None
    eps = 0.0
    normed = normed32 = None
    if norm is not None:
        w, b, eps = norm
        w = None if w is None else w.detach().to(torch.float32).contiguous()
        b = None if b is None else b.detach().to(torch.float32).contiguous()
        if norm_dtype is not None:
            normed = torch.empty(x.shape, device=x.device, dtype=norm_dtype)
        if norm_f32:
            normed32 = torch.empty(x.shape, device=x.device, dtype=torch.float32)
    unit = None
    if unit_eps is not None:
        if normed is None:
            raise ValueError("residual_layer_norm: unit rows need a norm and norm_dtype")
        unit = torch.empty(x.shape, device=x.device, dtype=normed.dtype)
    if gamma is not None:
        gamma = gamma.detach().to(torch.float32).contiguous()
    status = lib.vgo_residual_layer_norm(
        rows.data_ptr(), rows.stride(0), _c(b_rows), 0 if b_rows is None else b_rows.stride(0),
        _lib.dtype_code(branch.dtype) if branch is not None else _lib.VGO_F32, _c(gamma), _c(w), _c(b),
        float(eps), n, dim, _c(total), dim, _c(normed), dim,
        _lib.dtype_code(normed.dtype) if normed is not None else _lib.VGO_BF16, _c(normed32), dim,
        _c(unit), dim, float(unit_eps or 0.0), _lib.stream_of(x))
    _lib.check(status)
    if unit_eps is not None:
        return total, normed, normed32, unit
    return total, normed, normed32


def _restore_residual_layer_norm_impl(x: torch.Tensor, table: torch.Tensor, index: torch.Tensor,
                                      weight: torch.Tensor | None, gamma: torch.Tensor | None,
                                      norm: tuple[torch.Tensor | None, torch.Tensor | None, float],
                                      norm_dtype: torch.dtype):
    """One pass over fp32 rows x [N, dim] with the branch restored from `table` on the fly:
    branch = top4_project(table, index, weight) (same rounding), s = x + gamma * branch,
    n = LayerNorm(s) in `norm_dtype`.  With weight None, index is a one-hot int32 [N]
    map (a token plan's inverse): branch = table[index] (zero rows for index < 0).
    Returns (s, n)."""
    lib = _lib.load()
    _lib.require_gpu(x, table, index, weight, gamma)
    if x.dtype != torch.float32:
        raise ValueError("restore_residual_layer_norm: x must be float32")
    dim = x.shape[-1]
    rows = x.reshape(-1, dim)
    n = rows.shape[0]
    if table.ndim != 2 or table.shape[1] != dim:
        raise ValueError(f"restore_residual_layer_norm: table {tuple(table.shape)} must be [M, {dim}]")
    if weight is None:
        if index.shape != (n,):
            raise ValueError("restore_residual_layer_norm: a one-hot index must be [rows]")
    elif index.shape != (n, 4) or weight.shape != (n, 4):
        raise ValueError("restore_residual_layer_norm: index and weight must be [rows, 4]")
    if index.dtype != torch.int32 or (weight is not None and weight.dtype != torch.float32):
        raise ValueError("restore_residual_layer_norm: int32 indices and float32 weights")
    if norm_dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("restore_residual_layer_norm: norm_dtype must be bfloat16 or float16")
    index = index.contiguous()
    weight = None if weight is None else weight.contiguous()
    if table.stride(-1) != 1:
        table = table.contiguous()
    w, b, eps = norm
    w = None if w is None else w.detach().to(torch.float32).contiguous()
    b = None if b is None else b.detach().to(torch.float32).contiguous()
    if gamma is not None:
        gamma = gamma.detach().to(torch.float32).contiguous()
    total = torch.empty_like(x, memory_format=torch.contiguous_format)
    normed = torch.empty(x.shape, device=x.device, dtype=norm_dtype)
    status = lib.vgo_restore_residual_layer_norm(
        rows.data_ptr(), rows.stride(0), table.data_ptr(), table.stride(0), table.shape[0],
        _lib.dtype_code(table.dtype), index.data_ptr(), _c(weight), _c(gamma), _c(w), _c(b),
        float(eps), n, dim, total.data_ptr(), dim, normed.data_ptr(), dim,
        _lib.dtype_code(norm_dtype), _lib.stream_of(x))
    _lib.check(status)
    return total, normed


# --------------------------------------------- operator-backed entry points ----
def compact_into(x: torch.Tensor, out: torch.Tensor, *, base_rows: torch.Tensor | None,
                 offsets: torch.Tensor, segs_per_row: int, items: torch.Tensor | None,
                 item_shift: int, item_rows: torch.Tensor | None, weights: torch.Tensor | None,
                 normalizer: torch.Tensor | None,
                 layer_norm: tuple[torch.Tensor, torch.Tensor, float] | None = None) -> torch.Tensor:
    """Segmented weighted pooling into `out` (torch.ops.vgo.compact_into); see _compact_into_impl."""
    ln_w, ln_b, eps = layer_norm if layer_norm is not None else (None, None, 0.0)
    torch.ops.vgo.compact_into(x, out, base_rows, offsets, segs_per_row, items, item_shift, item_rows,
                               weights, normalizer, ln_w, ln_b, float(eps))
    return out


def compact_multi_into(x: torch.Tensor, outputs, *, base_rows: torch.Tensor | None,
                       offsets: torch.Tensor, segs_per_row: int, items: torch.Tensor | None,
                       item_shift: int, item_rows: torch.Tensor | None, weights: torch.Tensor | None,
                       normalizer: torch.Tensor | None) -> None:
    """1-3 outputs of one segment structure in one launch (torch.ops.vgo.compact_multi_into);
    `outputs` holds (channel offset, out, layer_norm or None) per output."""
    torch.ops.vgo.compact_multi_into(
        x, [int(off) for off, _, _ in outputs], [out for _, out, _ in outputs],
        [None if ln is None else ln[0] for _, _, ln in outputs],
        [None if ln is None else ln[1] for _, _, ln in outputs],
        [0.0 if ln is None else float(ln[2]) for _, _, ln in outputs],
        base_rows, offsets, segs_per_row, items, item_shift, item_rows, weights, normalizer)


def qkv_epilogue(qkv: torch.Tensor, heads: int, *, tokens_in: int, tokens_out: int | None = None,
                 rows: torch.Tensor | None = None, q_norm=None, k_norm=None, eps: float = 1e-5,
                 rope: tuple[torch.Tensor, torch.Tensor] | None = None, rope_prefix: int = 0,
                 want=(True, True, True), out_dtype: torch.dtype | None = None):
    """Head-major q/k/v from packed projection rows (torch.ops.vgo.qkv_epilogue); see
    _qkv_epilogue_impl.  Returns (q, k, v) with None for unwanted ones."""
    outs = torch.ops.vgo.qkv_epilogue(
        qkv, heads, tokens_in, tokens_out or tokens_in, rows,
        None if q_norm is None else q_norm[0], None if q_norm is None else q_norm[1],
        None if k_norm is None else k_norm[0], None if k_norm is None else k_norm[1], float(eps),
        None if rope is None else rope[0], None if rope is None else rope[1], rope_prefix,
        [bool(w) for w in want], out_dtype or qkv.dtype)
    return tuple(o if w else None for o, w in zip(outs, want))


def residual_layer_norm(x: torch.Tensor, branch: torch.Tensor | None = None,
                        gamma: torch.Tensor | None = None,
                        norm: tuple[torch.Tensor | None, torch.Tensor | None, float] | None = None, *,
                        write_sum: bool = True, norm_dtype: torch.dtype | None = torch.bfloat16,
                        norm_f32: bool = False, unit_eps: float | None = None):
    """One residual-row pass (torch.ops.vgo.residual_layer_norm); see _residual_layer_norm_impl.
    Returns (s, n, n_f32[, u]) with None for outputs not asked for."""
    w, b, eps = norm if norm is not None else (None, None, 0.0)
    outs = torch.ops.vgo.residual_layer_norm(
        x, branch, gamma, w, b, float(eps), norm is not None, write_sum, norm_dtype, norm_f32,
        -1.0 if unit_eps is None else float(unit_eps))
    total = outs[0] if write_sum and branch is not None else None
    normed = outs[1] if norm is not None and norm_dtype is not None else None
    normed32 = outs[2] if norm is not None and norm_f32 else None
    if unit_eps is not None:
        return total, normed, normed32, outs[3]
    return total, normed, normed32


def restore_residual_layer_norm(x: torch.Tensor, table: torch.Tensor, index: torch.Tensor,
                                weight: torch.Tensor | None, gamma: torch.Tensor | None,
                                norm: tuple[torch.Tensor | None, torch.Tensor | None, float], *,
                                norm_dtype: torch.dtype = torch.bfloat16):
    """The residual-row pass with the plan restore fused in
    (torch.ops.vgo.restore_residual_layer_norm); see _restore_residual_layer_norm_impl.
    Returns (s, n)."""
    w, b, eps = norm
    total, normed = torch.ops.vgo.restore_residual_layer_norm(x, table, index, weight, gamma, w, b,
                                                              float(eps), norm_dtype)
    return total, normed
