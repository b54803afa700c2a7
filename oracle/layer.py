"""Oracle: one merged global-attention layer (test infrastructure only).

CPU restatement of SelfAttention.forward / compute_attention with a
WeightedBilinearTokenPlan, or a TokenPlan that carries key_log_mass
(vggt_omega/models/layers/attention.py:195-207, 264-314, 328-439), in float32:
  qkv = x W^T + b * mask_K; q, k = LayerNorm64(q), LayerNorm64(k)
  K/V (and Q unless preserve_queries) compacted through the plan
  softmax(q k^T / 8 + log mass) v, special queries against the dense K/V
  out = proj(x); restore through the plan.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from oracle import attention as oracle_attention
from oracle import merging as oracle_merging


def _linear(x, weight, bias, autocast_bf16: bool):
    if autocast_bf16:  # bf16 operands, fp32 accumulation, bf16 result (CUDA autocast GEMM)
        return torch.nn.functional.linear(x.bfloat16(), weight.bfloat16(), bias.bfloat16())
    return x @ weight.T + bias


def self_attention(x: torch.Tensor, state: dict[str, torch.Tensor], num_heads: int,
                   plan: dict, preserve_queries: bool, autocast_bf16: bool = False) -> torch.Tensor:
    """x [N, C] float32 -> [N, C]; plan holds keep/source_original/parent_compact/
    weights/mass/special_original/special_compact as 1-D/2-D CPU tensors, or, for a
    TokenPlan (FastVGGT, token_merging.py:143-196), `inverse` [N]: clusters mean-pooled
    in ascending token order, key bias log(cluster size), outputs restored by inverse,
    and no dense special-query pass (a TokenPlan has none).

    autocast_bf16 reproduces the dtypes the reference sees under bf16 autocast
    (vggt_omega/models/vggt_omega.py:48-54): bf16 qkv/proj GEMMs, fp32 q/k
    LayerNorm and compaction, bf16 v, attention on bf16 operands.
    """
    n, c = x.shape
    d = c // num_heads
    bias = state["qkv.bias"] * state["qkv.bias_mask"]
    qkv = _linear(x, state["qkv.weight"], bias, autocast_bf16)
    q, k, v = qkv.reshape(n, 3, num_heads, d).unbind(1)  # [N, H, d]
    q = F.layer_norm(q.float(), (d,), state["q_norm.weight"], state["q_norm.bias"], 1e-5)
    k = F.layer_norm(k.float(), (d,), state["k_norm.weight"], state["k_norm.bias"], 1e-5)
    flat = lambda t: t.reshape(n, c)  # noqa: E731
    if "inverse" in plan:
        inverse = plan["inverse"]
        kept = int(inverse.max()) + 1
        mass = torch.bincount(inverse, minlength=kept).float()

        def compact(t):
            return oracle_merging.token_plan_compact(inverse, kept, flat(t))
    else:
        keep, src, parent, w, mass = (plan["keep"], plan["source_original"], plan["parent_compact"],
                                      plan["weights"], plan["mass"])

        def compact(t):
            return oracle_merging.weighted_compact(keep, src, parent, w, mass, flat(t))

    if preserve_queries:
        if "inverse" in plan:
            raise ValueError("a TokenPlan compacts queries")
        q_c = flat(q)
        k_c = flat(k)[keep]
    else:
        q_c = compact(q)
        k_c = compact(k)
    v_c = compact(v)
    attn_dtype = torch.bfloat16 if autocast_bf16 else torch.float32

    def heads(t):
        return t.to(attn_dtype).reshape(t.shape[0], num_heads, d).transpose(0, 1)[None]

    out = oracle_attention.mass_bias_attention(heads(q_c), heads(k_c), heads(v_c), mass.log())
    if "inverse" in plan:
        return oracle_merging.token_plan_restore(inverse, _project(out, state, c, autocast_bf16))
    special = plan["special_original"]
    dense = oracle_attention.mass_bias_attention(heads(flat(q)[special]), heads(flat(k)),
                                                 heads(flat(v)), None)
    index = special if preserve_queries else plan["special_compact"]
    out[:, :, index] = dense
    y = _project(out, state, c, autocast_bf16)
    if preserve_queries:
        return y
    return oracle_merging.weighted_restore(keep, src, parent, w, n, y)


def _project(out: torch.Tensor, state: dict[str, torch.Tensor], c: int, autocast_bf16: bool):
    """[1, H, K, d] attention output -> proj(x) [K, C] (attention.py:291-293, 436-438)."""
    y = out[0].transpose(0, 1).reshape(-1, c)
    return _linear(y, state["proj.weight"], state["proj.bias"], autocast_bf16)
