"""Parity of the gfx950 mass-bias attention kernel against the CPU oracle."""
from __future__ import annotations

import pytest
import torch

from oracle import attention as oracle
from tests._tol import RTOL, assert_close

pytestmark = pytest.mark.gpu


def _inputs(seed, b, h, nq, nk, dtype, mass_max=8, std=0.125):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(b, h, nq, 64, generator=g) * std).to(dtype)
    k = (torch.randn(b, h, nk, 64, generator=g) * std).to(dtype)
    v = torch.randn(b, h, nk, 64, generator=g).to(dtype)
    mass = torch.randint(1, mass_max + 1, (nk,), generator=g).float()
    return q, k, v, mass


SHAPES = [
    (1, 1, 1, 1),        # single query, single key
    (1, 2, 37, 29),      # ragged, smaller than one tile
    (1, 16, 1044, 522),  # C1 shape (S=4, 16x16 patches + 5 specials, ratio 0.5)
    (2, 3, 300, 257),    # batch > 1, tile remainders on both axes
    (1, 4, 129, 64),     # exactly one key tile, query remainder of 1
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", SHAPES)
def test_matches_oracle(vgo, device, dtype, shape):
    b, h, nq, nk = shape
    print(f"[attn] dtype={dtype} shape={shape}", flush=True)
    q, k, v, mass = _inputs(sum(shape), b, h, nq, nk, dtype, std=1.0 if dtype == torch.float32 else 0.125)
    out = vgo.mass_bias_attention(q.to(device), k.to(device), v.to(device), mass.log().to(device))
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == q.shape
    ref = oracle.mass_bias_attention(q, k, v, mass.log())
    assert_close(out, ref, dtype, what=f"attention {dtype} {shape}")


def test_unit_mass_and_no_bias_match_sdpa(vgo, device):
    q, k, v, _ = _inputs(11, 1, 4, 333, 190, torch.float32, std=1.0)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v)
    zero = vgo.mass_bias_attention(qd, kd, vd, torch.zeros(190, device=device))
    none = vgo.dense_attention(qd, kd, vd)
    assert_close(zero, ref, torch.float32, what="unit mass")
    assert_close(none, ref, torch.float32, what="no bias")


def test_strided_qkv_views(vgo, device):
    # q/k/v as head views of one packed [B, N, 3, H, 64] projection, the layout
    # vggt_omega/models/layers/attention.py:334-336 produces.
    g = torch.Generator().manual_seed(5)
    b, n, h = 1, 515, 16
    qkv = (torch.randn(b, n, 3, h, 64, generator=g) * 0.125).to(torch.bfloat16)
    mass = torch.randint(1, 9, (n,), generator=g).float()
    q, k, v = [t.transpose(1, 2) for t in torch.unbind(qkv.to(device), 2)]
    out = vgo.mass_bias_attention(q, k, v, mass.log().to(device))
    qc, kc, vc = [t.transpose(1, 2).contiguous() for t in torch.unbind(qkv, 2)]
    ref = oracle.mass_bias_attention(qc, kc, vc, mass.log())
    assert_close(out, ref, torch.bfloat16, what="strided views")


def test_autocast_casts_fp32_inputs_to_bf16(vgo, device):
    q, k, v, mass = _inputs(7, 1, 2, 100, 80, torch.float32, std=0.125)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = vgo.mass_bias_attention(q.to(device), k.to(device), v.to(device), mass.log().to(device))
    assert out.dtype == torch.bfloat16
    ref = oracle.mass_bias_attention(q.bfloat16(), k.bfloat16(), v.bfloat16(), mass.log())
    assert_close(out, ref, torch.bfloat16, what="autocast")


def test_large_mass_range_c5_style(vgo, device):
    q, k, v, mass = _inputs(8, 1, 2, 700, 1500, torch.bfloat16, mass_max=16)
    out = vgo.mass_bias_attention(q.to(device), k.to(device), v.to(device), mass.log().to(device))
    ref = oracle.mass_bias_attention(q, k, v, mass.log())
    assert_close(out, ref, torch.bfloat16, what="mass 1..16")


def test_errors_match_reference(vgo, device):
    q = torch.zeros(1, 2, 8, 64, device=device)
    with pytest.raises(ValueError, match=r"\[batch, heads, tokens, channels\]"):
        vgo.mass_bias_attention(q[0], q, q, torch.zeros(8, device=device))
    with pytest.raises(ValueError, match="head_dim=64"):
        vgo.mass_bias_attention(q[..., :32], q[..., :32], q[..., :32], torch.zeros(8, device=device))
    with pytest.raises(ValueError, match="incompatible"):
        vgo.mass_bias_attention(q, q[:, :1], q[:, :1], torch.zeros(8, device=device))
    with pytest.raises(ValueError, match="log_key_mass length"):
        vgo.mass_bias_attention(q, q, q, torch.zeros(7, device=device))


def test_deterministic_run_twice(vgo, device):
    q, k, v, mass = _inputs(9, 1, 4, 500, 400, torch.bfloat16)
    args = (q.to(device), k.to(device), v.to(device), mass.log().to(device))
    assert torch.equal(vgo.mass_bias_attention(*args), vgo.mass_bias_attention(*args))
    assert RTOL[torch.bfloat16] == 2e-2


def _attention_split(vgo, q, k, v, bias, split):
    from importlib import import_module
    mba = import_module(vgo.__name__ + ".mass_bias_attention")
    out = torch.empty_like(q)
    return mba._attention_into(q, k, v, bias, out, split=split)


@pytest.mark.parametrize("shape", [
    (1, 16, 1044, 522),   # 80 tasks of 9 key tiles spread over ~90 work-groups
    (1, 2, 100, 20000),   # 2 tasks of 313 tiles: each cut over dozens of work-groups
    (2, 3, 700, 1333),    # batch > 1, ragged query and key tails
])
def test_stream_k_and_plain_schedules_match_oracle(vgo, device, shape):
    b, h, nq, nk = shape
    print(f"[attn schedules] shape={shape}", flush=True)
    q, k, v, mass = _inputs(31 + nq, b, h, nq, nk, torch.bfloat16)
    bias = mass.log().to(torch.bfloat16)
    ref = oracle.mass_bias_attention(q, k, v, mass.log())
    args = (q.to(device), k.to(device), v.to(device), bias.to(device))
    for split in (True, False):
        out = _attention_split(vgo, *args, split=split)
        torch.cuda.synchronize()
        assert_close(out, ref, torch.bfloat16, what=f"attention split={split} {shape}")


def test_full_c4_size_rows_match_oracle(vgo, device):
    """C4 global-attention size (16 heads x 16,464 compacted tokens): sampled query rows."""
    b, h, n = 1, 16, 16464
    print(f"[attn c4] heads={h} tokens={n}", flush=True)
    g = torch.Generator().manual_seed(44)
    q = (torch.randn(b, h, n, 64, generator=g) * 0.125).bfloat16()
    k = (torch.randn(b, h, n, 64, generator=g) * 0.125).bfloat16()
    v = torch.randn(b, h, n, 64, generator=g).bfloat16()
    mass = torch.randint(1, 6, (n,), generator=g).float()
    args = (q.to(device), k.to(device), v.to(device), mass.log().bfloat16().to(device))
    split = _attention_split(vgo, *args, split=True)
    plain = _attention_split(vgo, *args, split=False)
    rows = torch.randperm(n, generator=g)[:97].sort().values
    rows = torch.cat([rows, torch.tensor([0, 255, 256, n - 1])]).unique()
    ref = oracle.mass_bias_attention(q[:, :, rows], k, v, mass.log())
    assert_close(split[:, :, rows.to(device)], ref, torch.bfloat16, what="C4 stream-K rows")
    assert_close(plain[:, :, rows.to(device)], ref, torch.bfloat16, what="C4 plain rows")
    # Same math on every row: the two schedules differ only in summation order.
    assert_close(split, plain.float(), torch.bfloat16, what="C4 stream-K vs plain")
