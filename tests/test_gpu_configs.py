"""GPU parity at BASELINE.json's full sizes (configs C2-C5).

The oracle runs on the CPU in seconds only on slices of these problems, so
each test checks (a) exactness on the kernel's own intermediate results over
the whole problem (selection from the kernel's scores, plan invariants,
bit-exact compaction / restore / projection of sampled or all rows), and
(b) sampled rows against the oracle's independent computation (exact-dot
scores, float64 attention).

* C2: top-4 projection, 1,048,576 rows from a 65,536 x 1,024 table, distinct
  uniform indices, Dirichlet(1,1,1,1) weights, bf16 and fp32.
* C3: one merged global block, S=16 x 1,029 tokens, dim 1,024, 16 heads.
* C4 sizes: the FastVGGT match (23,808 x 8,960 x 1,024, top-1 and top-4) and
  the q/k/v compaction of a 32,928-token plan.
* C5: S=200 x 1,029 = 205,800 tokens merged to 52,968 (protect 0, ratio
  0.75), and mass-bias attention of all 205,800 queries over those keys.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

import bench
from oracle import attention as oa
from oracle import merging as om
from oracle import projection as oproj
from tests._tol import assert_close
from tests.conftest import import_package
from tests.test_gpu_merge import score_tolerance

pytestmark = pytest.mark.gpu

DIM, HEADS = 1024, 16


@pytest.fixture(scope="module")
def kern():
    return import_package("_kernels")


def _layout(frames: int) -> dict:
    return dict(frames=frames, tokens_per_frame=1029, patch_token_start=5, patch_hw=(32, 32))


def _check_fastvggt_plan(plan, tokens_total: int, frames: int, ratio: float, protect: float) -> None:
    """Plan invariants and exact selection on the kernel's own scores."""
    sources, dests, best, target, flags = plan._derived["match"]
    removed = min(int(tokens_total * ratio), sources.numel())
    assert plan.kept_tokens == tokens_total - removed
    keep, inverse = plan.keep[0].cpu(), plan.inverse[0].cpu()
    rk, ri = om.fastvggt_select(best[0].cpu(), target[0].cpu().long(), sources.cpu(), dests.cpu(),
                                tokens_total, removed)
    assert torch.equal(keep, rk) and torch.equal(inverse, ri)
    # keep ascending, removed ∪ keep = all, specials and frame-0 patches kept
    assert (keep[1:] > keep[:-1]).all()
    is_kept = torch.zeros(tokens_total, dtype=torch.bool)
    is_kept[keep] = True
    assert int((~is_kept).sum()) == removed
    ids = om.patch_ids(frames, 1029, 5)
    special = torch.ones(tokens_total, dtype=torch.bool)
    special[ids.flatten()] = False
    assert is_kept[special].all() and is_kept[ids[0]].all()
    # every token maps to a kept token; kept tokens map to themselves
    assert torch.equal(inverse[keep], torch.arange(keep.numel()))
    assert inverse.min() >= 0 and inverse.max() < keep.numel()
    # integer masses = cluster sizes, summing to N
    counts = plan.cluster_counts(0).cpu()
    assert torch.equal(counts, torch.bincount(inverse, minlength=keep.numel()).float())
    assert int(counts.sum()) == tokens_total


def _check_sampled_match(unit_cpu: torch.Tensor, plan, n_sample: int, seed: int) -> None:
    """Kernel best/target of sampled sources against exact-dot bf16 scores."""
    sources, dests, best, target, _ = plan._derived["match"]
    g = torch.Generator().manual_seed(seed)
    pick = torch.randperm(sources.numel(), generator=g)[:n_sample]
    exact = om.bf16_scores(unit_cpu[sources.cpu()[pick]], unit_cpu[dests.cpu()])
    ref_best, ref_target = exact.max(dim=1)
    kb, kt = best[0].cpu()[pick], target[0].cpu().long()[pick]
    assert ((kb - ref_best).abs() <= score_tolerance(ref_best)).all()
    # the kernel's target is the exact argmax, or within one ulp of it (tie band)
    picked = exact.gather(1, kt[:, None])[:, 0]
    assert ((ref_best - picked) <= score_tolerance(ref_best)).all()
    assert (kt == ref_target).float().mean() > 0.97


# ------------------------------------------------------------------ C2 ----
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_c2_projection_full_size(vgo, device, dtype):
    n, m, d = 1 << 20, 65536, DIM
    print(f"[C2] projection {n} x {m} x {d} {dtype}", flush=True)
    index, weight = bench.c2_inputs(n, m)
    assert (index.sort(dim=1).values.diff(dim=1) > 0).all(), "indices must be distinct per row"
    assert torch.allclose(weight.double().sum(1), torch.ones(n, dtype=torch.float64), atol=1e-6)
    g = torch.Generator().manual_seed(2)
    table = torch.randn(m, d, generator=g).to(dtype)
    table_d, index_d, weight_d = table.to(device), index.to(device), weight.to(device)
    out = vgo.top4_project(table_d, index_d, weight_d)
    torch.cuda.synchronize()
    # sampled rows, and the first and last ones, bit-exact against the oracle
    rows = torch.cat((torch.arange(64), torch.randperm(n, generator=g)[:4096], torch.arange(n - 64, n)))
    ref = oproj.top4_project(table, index[rows], weight[rows])
    assert torch.equal(out[rows.to(device)].cpu(), ref)
    # whole output: one-hot weights reduce to a gather of the first index
    one_hot = torch.zeros_like(weight_d)
    one_hot[:, 0] = 1.0
    gathered = vgo.top4_project(table_d, index_d, one_hot)
    assert torch.equal(gathered, table_d.index_select(0, index_d[:, 0].long()))
    del out, gathered


# ------------------------------------------------------------------ C3 ----
def _torch_reference_block(block, x, plan):
    """The reference's global-block op sequence (block.py:219-226, attention.py:328-439,
    token_merging.py:176-196) in torch on the GPU under bf16 autocast, attention in fp32."""
    B, N, C = x.shape
    normalized = block.norm1(x)
    attn = block.attn
    qkv = attn.qkv(normalized).reshape(B, N, 3, HEADS, C // HEADS)
    q, k, v = [t.transpose(1, 2) for t in torch.unbind(qkv, 2)]
    q, k = attn.q_norm(q), attn.k_norm(k)
    inverse, kept = plan.inverse, plan.kept_tokens

    def pool(t):
        rows = t.transpose(1, 2).reshape(B, N, C).float()
        sums = torch.zeros(B, kept, C, device=x.device).scatter_add_(1, inverse[..., None].expand_as(rows), rows)
        counts = torch.zeros(B, kept, 1, device=x.device).scatter_add_(
            1, inverse[..., None], torch.ones(B, N, 1, device=x.device))
        return (sums / counts).to(t.dtype).reshape(B, kept, HEADS, C // HEADS).transpose(1, 2)

    qc, kc, vc = pool(q), pool(k), pool(v)
    bias = plan.key_log_mass.reshape(1, 1, 1, -1).to(torch.bfloat16).float()
    with torch.autocast("cuda", enabled=False):
        o = F.scaled_dot_product_attention(qc.bfloat16().float(), kc.bfloat16().float(),
                                           vc.bfloat16().float(), attn_mask=bias)
    y = attn.proj(o.to(torch.bfloat16).transpose(1, 2).reshape(B, kept, C))
    restored = y.gather(1, inverse[..., None].expand(-1, -1, C))
    x_attn = x + block.ls1(restored)
    return x_attn + block.ls2(block.mlp(block.norm2(x_attn)))


def test_c3_global_block(vgo, device):
    frames, n = 16, 16 * 1029
    print(f"[C3] global block S={frames} N={n}", flush=True)
    torch.manual_seed(0)
    block = vgo.SelfAttentionBlock(DIM, HEADS, qkv_bias=True, init_values=0.5, mask_k_bias=True,
                                   use_qk_norm=True).eval().to(device)
    with torch.no_grad():
        block.attn.q_norm.weight.normal_(1.0, 0.1)
        block.attn.k_norm.bias.normal_(0.0, 0.1)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, n, DIM, generator=g).to(device)
    layout = _layout(frames)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        unit, h = block.norm1_unit_rows(x)
        plan = vgo.build_fastvggt_plan(unit, merge_ratio=0.5, protect_ratio=0.0, mass_bias=True,
                                       prenormalized=True, **layout)
        out = block.forward_compacted(x, plan, normalized=h)
        qkv = block.attn.qkv(h)
        ref_out = _torch_reference_block(block, x, plan)
    assert plan.kept_tokens == 8232
    _check_fastvggt_plan(plan, n, frames, 0.5, 0.0)
    unit_cpu = unit[0].cpu()
    _check_sampled_match(unit_cpu, plan, 256, seed=31)
    inverse, keep, kept = plan.inverse[0].cpu(), plan.keep[0].cpu(), plan.kept_tokens
    # compaction: v bit-exact against the oracle; q with the fused LayerNorm to bf16 rounding
    v_rows = qkv[0, :, 2 * DIM:]
    v_c = torch.empty((HEADS, kept, 64), device=device, dtype=torch.bfloat16)
    plan.compact_into(v_rows, v_c)
    ref_v = om.token_plan_compact(inverse, kept, v_rows.cpu())
    assert torch.equal(v_c.transpose(0, 1).reshape(kept, DIM).cpu(), ref_v)
    qn = block.attn.q_norm
    q_c = torch.empty((HEADS, kept, 64), device=device, dtype=torch.bfloat16)
    plan.compact_into(qkv[0, :, :DIM], q_c, layer_norm=(qn.weight, qn.bias, qn.eps))
    q_normed = F.layer_norm(qkv[0, :, :DIM].float().cpu().view(n, HEADS, 64), (64,),
                            qn.weight.detach().cpu(), qn.bias.detach().cpu(), qn.eps).view(n, DIM)
    ref_q = om.token_plan_compact(inverse, kept, q_normed)
    assert_close(q_c.transpose(0, 1).reshape(kept, DIM).cpu(), ref_q, rtol=8e-3, what="C3 q compaction")
    # attention: sampled query rows of every head against the float64 oracle
    k_c = torch.empty_like(q_c)
    kn = block.attn.k_norm
    plan.compact_into(qkv[0, :, DIM:2 * DIM], k_c, layer_norm=(kn.weight, kn.bias, kn.eps))
    bias = plan.key_log_mass.reshape(-1)
    o = vgo.mass_bias_attention(q_c[None], k_c[None], v_c[None], bias)
    rows = torch.randperm(kept, generator=g)[:64]
    ref_o = oa.mass_bias_attention(q_c[None, :, rows.to(device)].cpu(), k_c[None].cpu(), v_c[None].cpu(),
                                   bias.cpu())
    assert_close(o[:, :, rows.to(device)].cpu(), ref_o, torch.bfloat16, what="C3 attention rows")
    # restore: bit-exact gather through the plan
    y = torch.randn(1, kept, DIM, generator=g).bfloat16()
    restored = plan.restore(y.to(device))
    assert torch.equal(restored[0].cpu(), om.token_plan_restore(inverse, y[0]))
    assert torch.equal(restored[0, keep.to(device)].cpu(), y[0])
    # the whole block against the reference op sequence on the same plan
    assert out.dtype == torch.float32
    assert_close(out[0].cpu(), ref_out[0].float().cpu(), torch.bfloat16, what="C3 block output")


# ------------------------------------------------------------ C4 sizes ----
@pytest.mark.parametrize("topk", [1, 4])
def test_c4_similarity_full_size(kern, device, topk):
    ns, nd = 23808, 8960
    print(f"[C4] similarity {ns} x {nd} top-{topk}", flush=True)
    g = torch.Generator().manual_seed(40 + topk)
    src = F.normalize(torch.randn(ns, DIM, generator=g), dim=-1).bfloat16()
    dst = F.normalize(torch.randn(nd, DIM, generator=g), dim=-1).bfloat16()
    dst[17] = dst[9]  # exact duplicate: ties across the whole source range
    # sources correlated with the dictionary, as matched tokens are
    src[::3] = F.normalize(dst[torch.randint(0, nd, (src[::3].shape[0],), generator=g)].float()
                           + 0.3 * torch.randn(src[::3].shape[0], DIM, generator=g), dim=-1).bfloat16()
    scores = torch.empty((ns, nd), dtype=torch.bfloat16, device=device)
    values, index = kern.similarity_topk(src.to(device), dst.to(device), topk, scores=scores)
    ks = scores.float().cpu()
    ref_v, ref_i = om.topk_lowest_index(ks, topk)
    assert torch.equal(index.cpu(), ref_i) and torch.equal(values.cpu(), ref_v)
    rows = torch.randperm(ns, generator=g)[:384]
    exact = om.bf16_scores(src[rows], dst)
    mismatch = ks[rows] != exact
    assert mismatch.float().mean() < 5e-3
    assert ((ks[rows] - exact).abs()[mismatch] <= score_tolerance(exact)[mismatch]).all()


def test_c4_plan_and_compaction_full_size(vgo, device):
    frames, n = 32, 32 * 1029
    print(f"[C4] plan + q/k/v compaction N={n}", flush=True)
    g = torch.Generator().manual_seed(44)
    tokens = torch.randn(1, n, DIM, generator=g).to(device)
    plan = vgo.build_fastvggt_plan(tokens, merge_ratio=0.5, protect_ratio=0.0, mass_bias=True,
                                   **_layout(frames))
    assert plan.kept_tokens == 16464
    _check_fastvggt_plan(plan, n, frames, 0.5, 0.0)
    unit_cpu = F.normalize(tokens[0].cpu(), dim=-1, eps=1e-12).bfloat16()
    _check_sampled_match(unit_cpu, plan, 256, seed=45)
    kept, inverse = plan.kept_tokens, plan.inverse[0].cpu()
    qkv = torch.randn(n, 3 * DIM, generator=g).bfloat16()
    qkv_d = qkv.to(device)
    outs = [torch.empty((HEADS, kept, 64), device=device, dtype=torch.bfloat16) for _ in range(3)]
    plan.compact_multi_into(qkv_d, [(0, outs[0], None), (DIM, outs[1], None), (2 * DIM, outs[2], None)])
    for i, out in enumerate(outs):
        ref = om.token_plan_compact(inverse, kept, qkv[:, i * DIM:(i + 1) * DIM])
        assert torch.equal(out.transpose(0, 1).reshape(kept, DIM).cpu(), ref), f"output {i}"


# ------------------------------------------------------------------ C5 ----
def test_c5_long_sequence(vgo, device):
    frames, n = 200, 200 * 1029
    print(f"[C5] plan + attention N={n}", flush=True)
    torch.cuda.reset_peak_memory_stats()
    g = torch.Generator().manual_seed(9)
    tokens = torch.randn(1, n, DIM, generator=g).to(device)
    plan = vgo.build_fastvggt_plan(tokens, merge_ratio=0.75, protect_ratio=0.0, mass_bias=True,
                                   **_layout(frames))
    # destination floor of the 2x2 rule: frame-0 patches + one anchor per 2x2 cell + specials
    assert plan.kept_tokens == 1024 + 199 * 256 + 200 * 5 == 52968
    _check_fastvggt_plan(plan, n, frames, 0.75, 0.0)
    unit_cpu = F.normalize(tokens[0].cpu(), dim=-1, eps=1e-12).bfloat16()
    _check_sampled_match(unit_cpu, plan, 96, seed=46)
    del tokens, unit_cpu
    counts = plan.cluster_counts(0)
    print(f"[C5] masses {int(counts.min())}..{int(counts.max())}", flush=True)
    nk = plan.kept_tokens
    q = (torch.randn(1, HEADS, n, 64, generator=g) * 0.125).bfloat16().to(device)
    k = (torch.randn(1, HEADS, nk, 64, generator=g) * 0.125).bfloat16().to(device)
    v = torch.randn(1, HEADS, nk, 64, generator=g).bfloat16().to(device)
    bias = plan.key_log_mass.reshape(-1)
    out = vgo.mass_bias_attention(q, k, v, bias)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() / 2 ** 30
    rows = torch.cat((torch.arange(8), torch.randperm(n, generator=g)[:48], torch.arange(n - 8, n)))
    ref = oa.mass_bias_attention(q[:, :, rows.to(device)].cpu(), k.cpu(), v.cpu(), bias.cpu())
    err = assert_close(out[:, :, rows.to(device)].cpu(), ref, torch.bfloat16, what="C5 attention rows")
    print(f"[C5] attention rows rel err {err:.2e}; peak memory {peak:.1f} GiB "
          f"(flops {4 * HEADS * n * nk * 64:.3e})", flush=True)
    assert math.isfinite(peak)
