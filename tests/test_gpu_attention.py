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
    (1, 2, 1, 2600),     # ping-pong kernel, one query: seven idle waves, all stream-K pieces
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


def _pair(vgo, main, special):
    from importlib import import_module
    mba = import_module(vgo.__name__ + ".mass_bias_attention")
    outs = (torch.empty_like(main[0]), torch.empty_like(special[0]))
    mba._attention_pair_into((*main, outs[0]), (*special, None, outs[1]))
    return outs


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shapes", [
    ((1, 16, 1044, 522), (1, 16, 20, 1044)),     # C1: merged pass + 4 frames x 5 specials
    ((1, 2, 100, 20000), (1, 2, 7, 3000)),       # both problems cut over many work-groups
    ((1, 2, 64, 52968), (1, 1, 5, 100)),         # C5's key count (fp32: 1e-5 at 52,968 keys)
    ((2, 3, 700, 1333), (1, 3, 513, 2100)),      # different batch; special tasks > 512 queries
    ((1, 1, 1, 1), (1, 1, 1, 65)),               # single rows
])
def test_pair_launch_matches_oracle(vgo, device, dtype, shapes):
    """Merged attention and the dense special-query pass in one launch."""
    (b0, h0, nq0, nk0), (b1, h1, nq1, nk1) = shapes
    # fp32: each output averages nk unit-variance values to ~1/sqrt(nk) of their scale,
    # so the rounding of the running sums sets the error; the kernel sums 32 keys at a
    # time before adding them to the totals, which keeps it under the 1e-5 bar at
    # 20,000 keys (1.3e-5 with one running sum).
    print(f"[attn pair] dtype={dtype} shapes={shapes}", flush=True)
    std = 1.0 if dtype == torch.float32 else 0.125
    q, k, v, mass = _inputs(7 + nq0 + nk1, b0, h0, nq0, nk0, dtype, std=std)
    sq, sk, sv, _ = _inputs(9 + nq1, b1, h1, nq1, nk1, dtype, std=std)
    bias = mass.log().to(dtype)
    main = (q.to(device), k.to(device), v.to(device), bias.to(device))
    special = (sq.to(device), sk.to(device), sv.to(device))
    out0, out1 = _pair(vgo, main, special)
    torch.cuda.synchronize()
    err = assert_close(out0, oracle.mass_bias_attention(q, k, v, bias.float()), dtype,
                       what=f"pair main {shapes}")
    print(f"[attn pair] main error {err:.3e}", flush=True)
    ref1 = oracle.mass_bias_attention(sq, sk, sv, torch.zeros(nk1))
    assert_close(out1, ref1, dtype, what=f"pair special {shapes}")


def test_pair_launch_c4_special_pass(vgo, device):
    """C4 sizes: 16,464 merged tokens with bias + 160 special queries over 32,928 keys."""
    print("[attn pair c4]", flush=True)
    q, k, v, mass = _inputs(61, 1, 16, 16464, 16464, torch.bfloat16)
    sq, sk, sv, _ = _inputs(62, 1, 16, 160, 32928, torch.bfloat16)
    bias = mass.log().bfloat16()
    out0, out1 = _pair(vgo, (q.to(device), k.to(device), v.to(device), bias.to(device)),
                       (sq.to(device), sk.to(device), sv.to(device)))
    single = _attention_split(vgo, q.to(device), k.to(device), v.to(device), bias.to(device), True)
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(63)
    rows = torch.cat([torch.randperm(16464, generator=g)[:61], torch.tensor([0, 16463])]).unique()
    assert_close(out0[:, :, rows.to(device)], oracle.mass_bias_attention(q[:, :, rows], k, v, bias.float()),
                 torch.bfloat16, what="C4 pair main rows")
    assert_close(out0, single.float(), torch.bfloat16, what="C4 pair main vs single launch")
    assert_close(out1, oracle.mass_bias_attention(sq, sk, sv, torch.zeros(32928)), torch.bfloat16,
                 what="C4 special pass")


def test_pair_launch_empty_problems_and_errors(vgo, device):
    from importlib import import_module
    mba = import_module(vgo.__name__ + ".mass_bias_attention")
    q, k, v, mass = _inputs(3, 1, 2, 300, 200, torch.bfloat16)
    args = (q.to(device), k.to(device), v.to(device), mass.log().bfloat16().to(device))
    empty_q = torch.empty(1, 2, 0, 64, device=device, dtype=torch.bfloat16)
    out0, out1 = _pair(vgo, args, (empty_q, args[1], args[2]))
    assert out1.shape == (1, 2, 0, 64)
    assert_close(out0, oracle.mass_bias_attention(q, k, v, mass.log().bfloat16().float()), torch.bfloat16,
                 what="pair with empty special pass")
    out0, out1 = _pair(vgo, (empty_q, args[1], args[2], args[3]), args[:3])
    assert_close(out1, oracle.mass_bias_attention(q, k, v, torch.zeros(200)), torch.bfloat16,
                 what="pair with empty main pass")
    with pytest.raises(ValueError, match="one dtype"):
        _pair(vgo, args, (args[0].half(), args[1].half(), args[2].half()))
    with pytest.raises(ValueError, match="head_dim=64"):
        _pair(vgo, args, (args[0][..., :32], args[1][..., :32], args[2][..., :32]))
    with pytest.raises(RuntimeError, match="workspace too small"):
        problems = (mba._lib.AttnProblem * 2)(mba._problem(*args, torch.empty_like(args[0]))[0],
                                             mba._problem(*args[:3], None, torch.empty_like(args[0]))[0])
        lib = mba._lib.load()
        mba._lib.check(lib.vgo_mass_bias_attn_pair_fwd_ws(problems, 2, 1, None, 0, None))
    with pytest.raises(ValueError, match="1 or 2 problems"):
        mba._lib.check(mba._lib.load().vgo_mass_bias_attn_pair_fwd_ws(problems, 3, 1, None, 0, None))


def test_kernel_timing_records_each_workspace_launch(vgo, device):
    """vgo_attn_kernel_timing brackets each attention-kernel launch with an event
    pair while it is on, records nothing while it is off, and leaves results alone;
    vgo_attn_kernel_clock_read reports the clock of the same launches from their
    work-groups' counters (a shader clock within the chip's range, and a constant
    counter whose ticks over the launch spans do not run ahead of the events' 100 MHz)."""
    prof = __import__("4d_ttt_merging_amd.profiling", fromlist=["profiling"])
    print("[attn] kernel timing, 1x2x600x3000 bf16", flush=True)
    q, k, v, mass = _inputs(11, 1, 2, 600, 3000, torch.bfloat16)
    q, k, v, bias = q.to(device), k.to(device), v.to(device), mass.log().to(device)
    untimed = vgo.mass_bias_attention(q, k, v, bias)
    prof.attention_kernel_summary()
    prof.attention_kernel_timing(True)
    try:
        timed = [vgo.mass_bias_attention(q, k, v, bias) for _ in range(3)]
    finally:
        prof.attention_kernel_timing(False)
    clock = prof.attention_kernel_clock()
    print(f"[attn] kernel clock {clock}", flush=True)
    assert clock is not None and clock["launches"] == 3
    assert 0.3 < clock["clock_ghz"] < 3.0
    assert 0.0 < clock["const_mhz"] <= 101.0
    total_ms, launches = prof.attention_kernel_summary()
    assert launches == 3 and total_ms > 0.0
    assert prof.attention_kernel_clock() is None
    for out in timed:
        assert torch.equal(out, untimed)
    vgo.mass_bias_attention(q, k, v, bias)
    assert prof.attention_kernel_summary() == (0.0, 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("std", [1.0, 2.0, 3.0])
@pytest.mark.parametrize("nk", [1500, 3000])
def test_wide_logits_match_oracle(vgo, device, dtype, std, nk):
    """q, k at unit scale (the aggregator's operating point: per-head LayerNorm'd
    q and k) and at 2-3x unit scale (logits of tens in the exp2 domain, which take
    the lazy softmax's rescaling path on many tiles); both kernels (1,500 keys:
    register-staged, 3,000: ping-pong) stay within the tolerance of the oracle.
    657 queries leave a wave with 17 (past 2 x 256 + 128), which the
    register-staged kernel runs as one 32-query block.  The measured error is
    printed beside the bar."""
    print(f"[attn] wide logits dtype={dtype} std={std} nk={nk}", flush=True)
    q, k, v, mass = _inputs(int(std * 10) + nk, 1, 4, 657, nk, dtype, mass_max=16, std=std)
    out = vgo.mass_bias_attention(q.to(device), k.to(device), v.to(device), mass.log().to(device))
    torch.cuda.synchronize()
    ref = oracle.mass_bias_attention(q, k, v, mass.log())
    assert torch.isfinite(out).all()
    err = assert_close(out.cpu(), ref, dtype, what=f"std={std} nk={nk}")
    print(f"[attn] wide logits dtype={dtype} std={std} nk={nk}: rel err {err:.3e} (bar {RTOL[dtype]:.0e})",
          flush=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_c4_unit_scale_rows_match_oracle(vgo, device, dtype):
    """The C4 global attention where the aggregator runs it: 16 heads, 16,464 queries
    over 16,464 merged keys with integer masses in [1, 8] (a ratio-0.5 FastVGGT plan
    of 32,928 tokens), q and k at unit scale as the per-head LayerNorm leaves them.
    Sampled query rows (the first and last included) of every head against the
    float64 oracle."""
    print(f"[attn] C4 unit-scale rows dtype={dtype}", flush=True)
    q, k, v, mass = _inputs(71, 1, 16, 16464, 16464, dtype, mass_max=8, std=1.0)
    bias = mass.log().to(dtype)
    qd, kd, vd, bd = q.to(device), k.to(device), v.to(device), bias.to(device)
    out = vgo.mass_bias_attention(qd, kd, vd, bd)
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(72)
    rows = torch.cat([torch.randperm(16464, generator=g)[:62], torch.tensor([0, 16463])]).unique()
    ref = oracle.mass_bias_attention(q[:, :, rows], k, v, bias.float())
    err = assert_close(out[:, :, rows.to(device)].cpu(), ref, dtype, what=f"C4 unit-scale rows {dtype}")
    print(f"[attn] C4 unit-scale rows dtype={dtype}: rel err {err:.3e} over {rows.numel()} rows x 16 heads "
          f"(bar {RTOL[dtype]:.0e})", flush=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("nk", [1029, 3000])
def test_zero_mass_leading_keys_match_oracle(vgo, device, dtype, nk):
    """Keys of mass 0 (log-mass bias -inf) take no weight.  With the first 80 keys
    and a scattered tenth of the rest at mass 0, the first key tile of every task
    holds no finite logit: the register-staged kernel (1,029 keys) starts its
    first-tile softmax with the reference max still at -inf, the ping-pong kernel
    (3,000 keys) its rescaling path, and both must leave those keys out."""
    print(f"[attn] zero-mass leading keys dtype={dtype} nk={nk}", flush=True)
    q, k, v, mass = _inputs(97 + nk, 1, 3, 657, nk, dtype, mass_max=8, std=1.0 if dtype == torch.float32 else 0.5)
    g = torch.Generator().manual_seed(98)
    mass[:80] = 0.0
    mass[torch.randperm(nk, generator=g)[: nk // 10]] = 0.0
    bias = mass.log()  # -inf where the mass is 0
    out = vgo.mass_bias_attention(q.to(device), k.to(device), v.to(device), bias.to(device))
    torch.cuda.synchronize()
    ref = oracle.mass_bias_attention(q, k, v, bias)
    assert torch.isfinite(out).all()
    err = assert_close(out.cpu(), ref, dtype, what=f"zero-mass nk={nk}")
    print(f"[attn] zero-mass leading keys dtype={dtype} nk={nk}: rel err {err:.3e} (bar {RTOL[dtype]:.0e})",
          flush=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("case", [
    (8, 1100, 3000),   # split: 24 tasks, every segment a stream-K piece of 4-5 key tiles
    (64, 2100, 700),   # split: 320 tasks, a round of whole tasks, then stream-K pieces
])
def test_late_heavy_keys_rescale_mid_segment(vgo, device, dtype, split, case):
    """Keys whose log-mass bias steps up by 11 (more than the lazy softmax's 15 ln 2
    headroom) several tiles into the key sequence: every query's probabilities leave
    the fast path's range on those tiles, which are not the first tile of their
    segment, so the rescaling path runs mid-segment (in the ping-pong kernel, split,
    at the start of the following MFMA phase for both wave groups; in the
    register-staged kernel before its P.V) and must rescale O and the sums that
    earlier tiles left.  fp32 runs its own kernel either way."""
    h, nq, nk = case
    if dtype == torch.float32 and not split:
        pytest.skip("fp32 takes the same kernel for both entries")
    print(f"[attn] late heavy keys dtype={dtype} split={split} heads={h} nq={nq} nk={nk}", flush=True)
    q, k, v, mass = _inputs(311 + nk, 1, h, nq, nk, dtype, mass_max=4, std=0.5)
    bias = mass.log()
    steps = {nk // 7: 11.0, nk // 3: 22.0, (2 * nk) // 3: 33.0, nk - 40: 33.0}
    for pos, b in steps.items():
        bias[pos] = b
    bias = bias.to(dtype).float()  # the entry takes the bias in the query dtype; the oracle gets the same values
    out = _attention_split(vgo, q.to(device), k.to(device), v.to(device), bias.to(dtype).to(device), split)
    torch.cuda.synchronize()
    out = out.cpu()
    assert torch.isfinite(out).all()
    ref = torch.cat([oracle.mass_bias_attention(q[:, i:i + 1], k[:, i:i + 1], v[:, i:i + 1], bias)
                     for i in range(h)], dim=1)
    err = assert_close(out, ref, dtype, what=f"late heavy keys split={split} heads={h} nq={nq} nk={nk}")
    print(f"[attn] late heavy keys dtype={dtype} split={split} heads={h} nq={nq} nk={nk}: rel err {err:.3e} "
          f"(bar {RTOL[dtype]:.0e})", flush=True)
