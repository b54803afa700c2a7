"""Mass-bias attention on gfx950: softmax(QK^T/sqrt(d) + log_key_mass) V.

Drop-in for `vggt_omega.models.mass_bias_attention.mass_bias_attention`
(reference vggt_omega/models/mass_bias_attention.py:85-129): same argument
meaning, same autocast cast, same exception types and messages, same output
allocation.  The arithmetic runs in the hand-written HIP kernel
`vgo_mass_bias_attn_fwd` (csrc/attention.hip); there is no CPU path.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


def _problem(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, bias: torch.Tensor | None,
             out: torch.Tensor) -> tuple[_lib.AttnProblem, tuple[torch.Tensor, ...]]:
    """Checks one attention problem and describes it for the C ABI.

    Returns the `vgo_attn_problem` and the tensors it points into (kept alive
    by the caller until the launch is queued)."""
    _lib.require_gpu(q, k, v, bias, out)
    if not (q.dtype == k.dtype == v.dtype == out.dtype):
        raise ValueError("q, k, v and the output must share one dtype")
    if bias is not None:
        if bias.dtype != q.dtype:
            raise ValueError("the log-mass bias must be rounded to the query dtype")
        bias = bias.contiguous()
    views = []
    for t in (q, k, v):
        if t.stride(-1) != 1:
            t = t.contiguous()
        views.append(t)
    q, k, v = views
    if out.stride(-1) != 1:
        raise ValueError("output channel stride must be 1")
    batch, heads, n_query, head_dim = q.shape
    problem = _lib.AttnProblem(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.ptr(bias), out.data_ptr(),
        batch, heads, n_query, k.shape[-2], head_dim,
        _lib.strides3(q), _lib.strides3(k), _lib.strides3(v), _lib.strides3(out))
    return problem, (q, k, v, bias, out)


# Key lengths up to this run faster on the entry without a workspace.  Measured
# on MI355X over 32,928 queries x 16 heads split into equal self-attention
# problems: at 1,029 / 1,536 / 2,058 keys the register-staged kernel takes
# 0.79 / 0.86 / 0.97 of the ping-pong kernel's time, at 3,087 / 4,116 / 8,232
# keys 1.05 / 1.08 / 1.19.  With few key tiles per 512-query task the ping-pong
# kernel's V^T pack, pipeline fill and partly empty tasks do not pay off.
REG_MAX_KEYS = 2560


def _attention_into(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    bias: torch.Tensor | None, out: torch.Tensor, *,
                    split: bool | None = None) -> torch.Tensor:
    """`_attention_into_impl` through the operator torch.ops.vgo.attention_into."""
    torch.ops.vgo.attention_into(q, k, v, bias, out, -1 if split is None else int(split))
    return out


def _attention_pair_into(main: tuple, special: tuple) -> None:
    """`_attention_pair_into_impl` through the operator torch.ops.vgo.attention_pair_into."""
    torch.ops.vgo.attention_pair_into(*main, *special)


def _attention_into_impl(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         bias: torch.Tensor | None, out: torch.Tensor, *,
                         split: bool | None = None) -> torch.Tensor:
    """Run the kernel on [B,H,N,64] views (any batch/head/token strides) into `out`.

    split=True takes the workspace entry: V^T packed per head, 512-query
    blocks on the 8-wave kernel, (query block, key tile) work balanced over
    the resident work-groups (stream-K, partial states merged by a third
    kernel); split=False takes the entry without a workspace (one
    work-group per 256-query block).  split=None picks by key length
    (REG_MAX_KEYS).
    """
    if split is None:
        split = k.shape[-2] > REG_MAX_KEYS
    lib = _lib.load()
    p, keep = _problem(q, k, v, bias, out)
    dtype = _lib.dtype_code(q.dtype)
    args = (p.q, p.k, p.v, p.log_mass, p.out, p.batch, p.heads, p.n_query, p.n_key, p.head_dim,
            p.q_stride, p.k_stride, p.v_stride, p.o_stride, dtype)
    need = ctypes.c_size_t(0)
    if split:
        _lib.check(lib.vgo_mass_bias_attn_workspace(p.batch, p.heads, p.n_query, p.n_key, dtype,
                                                    ctypes.byref(need)))
    if need.value == 0:
        status = lib.vgo_mass_bias_attn_fwd(*args, _lib.stream_of(q))
    else:
        workspace = torch.empty(need.value // 4, device=q.device, dtype=torch.float32)
        status = lib.vgo_mass_bias_attn_fwd_ws(*args, workspace.data_ptr(), need.value,
                                               _lib.stream_of(q))
    _lib.check(status)
    del keep
    return out


def _attention_pair_into_impl(main: tuple, special: tuple) -> None:
    """Merged attention and the dense special-query pass in one launch.

    `main` and `special` are (q, k, v, bias, out) as for `_attention_into`;
    each output receives its problem's result (vgo_mass_bias_attn_pair_fwd_ws).
    """
    lib = _lib.load()
    if main[0].dtype != special[0].dtype or main[0].device != special[0].device:
        raise ValueError("both attention problems must share one dtype and device")
    p0, keep0 = _problem(*main)
    p1, keep1 = _problem(*special)
    problems = (_lib.AttnProblem * 2)(p0, p1)
    dtype = _lib.dtype_code(main[0].dtype)
    need = ctypes.c_size_t(0)
    _lib.check(lib.vgo_mass_bias_attn_pair_workspace(problems, 2, dtype, ctypes.byref(need)))
    workspace = None
    if need.value:
        workspace = torch.empty(need.value // 4, device=main[0].device, dtype=torch.float32)
    _lib.check(lib.vgo_mass_bias_attn_pair_fwd_ws(
        problems, 2, dtype, _lib.ptr(workspace), need.value, _lib.stream_of(main[0])))
    del keep0, keep1


def mass_bias_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        log_key_mass: torch.Tensor) -> torch.Tensor:
    """Compute softmax(QK^T/sqrt(d) + log_key_mass)V exactly.

    q, k, v: [batch, heads, tokens, 64] on the GPU; log_key_mass: Nk values
    shared by every batch and head.  Under CUDA/HIP bf16 autocast fp32 inputs
    are cast to bf16 first, as autocast SDPA would
    (reference mass_bias_attention.py:96-107).  The bias is rounded to the
    query dtype (reference :109).
    """
    try:
        _lib.load()
    except _lib.ExtensionUnavailable as error:
        raise RuntimeError(str(error)) from error
    _lib.require_gpu(q, k, v, log_key_mass)
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k and v must be [batch, heads, tokens, channels]")
    if q.shape[-1] != 64 or k.shape[-1] != 64 or v.shape[-1] != 64:
        raise ValueError("the initial fused kernel supports head_dim=64 only")
    if k.shape != v.shape or q.shape[:2] != k.shape[:2]:
        raise ValueError("incompatible q/k/v shapes")
    autocast_bf16 = bool(
        torch.is_autocast_enabled("cuda") and q.dtype == torch.float32
        and torch.get_autocast_dtype("cuda") == torch.bfloat16
    )
    if autocast_bf16:
        q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    output_dtype = q.dtype
    if output_dtype not in _lib.DTYPE_CODE:
        raise ValueError(f"unsupported dtype {output_dtype}")
    k, v = k.to(output_dtype), v.to(output_dtype)
    bias = log_key_mass.reshape(-1).to(q.dtype)
    if bias.numel() != k.shape[-2]:
        raise ValueError("log_key_mass length does not match key tokens")
    return torch.ops.vgo.mass_bias_attention(q, k, v, bias)


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Unbiased attention (the dense special-query pass), same kernel, no bias."""
    if q.shape[-1] != 64:
        raise ValueError("the initial fused kernel supports head_dim=64 only")
    _lib.require_gpu(q, k, v)
    return torch.ops.vgo.mass_bias_attention(q, k.to(q.dtype), v.to(q.dtype), None)
