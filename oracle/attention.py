"""Oracle: mass-bias attention (test infrastructure only).

Restates vggt_omega/models/mass_bias_attention.py:17-129:
  logits = (q . k) * log2(e)/sqrt(d) + bf16(log m) * log2(e)     (:56-58, :109)
  P      = exp2(logits - rowmax)                                  (:60-63)
  O      = (P rounded to v.dtype) @ V / sum(P)                    (:64, :74, :76)
in float64, with the reference's two roundings to the input dtype: the bias
(:109) and P before the P.V product (:74).  The Triton kernel's running max per
32-key block only rescales P by a per-block constant before that rounding; the
closed form below uses the row max, a difference far inside the bf16 tolerance.
"""
from __future__ import annotations

import math

import torch

LOG2E = 1.4426950408889634


def mass_bias_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        log_key_mass: torch.Tensor | None) -> torch.Tensor:
    """q [B,H,Nq,d], k/v [B,H,Nk,d] (CPU), log_key_mass [Nk] or None -> [B,H,Nq,d]."""
    dtype = q.dtype
    low_precision = dtype in (torch.bfloat16, torch.float16)
    scale_log2 = LOG2E / math.sqrt(q.shape[-1])
    logits = (q.double() @ k.double().transpose(-1, -2)) * scale_log2
    if log_key_mass is not None:
        bias = log_key_mass.reshape(-1).to(dtype).double()
        logits = logits + bias * LOG2E
    logits = logits - logits.amax(dim=-1, keepdim=True)
    p = torch.exp2(logits)
    denominator = p.sum(dim=-1, keepdim=True)
    if low_precision:
        p = p.to(dtype).double()
    out = (p @ v.double()) / denominator
    return out.to(dtype)


def sdpa_with_log_mass(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       log_key_mass: torch.Tensor | None) -> torch.Tensor:
    """The reference's own fallback (vggt_omega/models/layers/attention.py:400).

    `scaled_dot_product_attention(q, k, v, attn_mask=bias)` with the bias laid
    out as [1,1,1,Nk] (attention.py:386-388); a library routine, used to pin
    `mass_bias_attention` above.
    """
    mask = None
    if log_key_mass is not None:
        mask = log_key_mass.reshape(1, 1, 1, -1).to(q.dtype)
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask)
