"""GPU parity of the merge path (normalize, match, rank/select, CSR, mass,
compaction, restore, convex fit, both planners) against the CPU oracle and the
reference fixtures.

Integer outputs (indices, keep/inverse, CSR order, integer masses) are
compared bit-exactly.  Float reductions that the kernels perform in the
oracle's operation order (segmented sums, masses, compaction, projection) are
bit-exact too; scores and the convex fit are compared to tolerance, and any
index difference must sit inside an exact bf16 tie.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import layer as oracle_layer
from oracle import merging as om
from tests._tol import assert_close, rel_error
from tests.conftest import import_package
from tests.golden.inputs import attention_weights, seeded_values, structured_tokens

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).parent / "golden"
KW = dict(frames=4, tokens_per_frame=261, patch_token_start=5, patch_hw=(16, 16))


@pytest.fixture(scope="module")
def kern():
    return import_package("_kernels")


@pytest.fixture(scope="module")
def fx():
    return np.load(GOLDEN / "fixtures_c1.npz")


def ulp_bf16(x: torch.Tensor) -> torch.Tensor:
    """bf16 spacing at |x| (float32 tensor of bf16 values)."""
    e = torch.frexp(x.abs().clamp_min(1e-30))[1]
    return torch.ldexp(torch.ones_like(x), e - 8)


def score_tolerance(exact: torch.Tensor) -> torch.Tensor:
    """One bf16 ulp, or the fp32 accumulation error of a unit-norm dot product
    (about 2^-17 absolute) for scores so close to zero that it exceeds an ulp."""
    return torch.maximum(ulp_bf16(exact) * 1.01, torch.full_like(exact, 2.0 ** -17))


# ------------------------------------------------------------ normalize ----
@pytest.mark.parametrize("dim,eps", [(1024, 1e-12), (1024, 1e-6), (64, 1e-6), (200, 1e-12)])
def test_normalize_rows(kern, device, dim, eps):
    print(f"[normalize] dim={dim}", flush=True)
    g = torch.Generator().manual_seed(dim)
    x = torch.randn(300, dim, generator=g) * 3
    x[7] = 0.0  # eps path
    rows = torch.randperm(300, generator=g)[:150]
    out = kern.normalize_rows(x.to(device), rows.to(device), eps).cpu()
    ref = F.normalize(x[rows], dim=-1, eps=eps).to(torch.bfloat16)
    diff = out.float() != ref.float()
    assert diff.float().mean() < 2e-3
    if diff.any():
        assert ((out.float() - ref.float()).abs()[diff] <= ulp_bf16(ref.float())[diff] * 1.01).all()
    f32 = kern.normalize_rows(x.to(device), rows.to(device), eps, torch.float32).cpu()
    assert rel_error(f32, F.normalize(x[rows], dim=-1, eps=eps)) < 1e-6


# ------------------------------------------------------------- matching ----
@pytest.mark.parametrize("topk", [1, 4])
@pytest.mark.parametrize("ns,nd,dim", [(37, 11, 64), (300, 777, 1024), (1000, 130, 128), (260, 300, 72),
                                        # one or two 32-wide K chunks in all: fewer steps than the
                                        # ring's look-ahead (regression: the DMA count must stay uniform)
                                        (513, 40, 32), (700, 257, 32), (90, 600, 64)])
def test_similarity_selection_is_exact_on_kernel_scores(kern, device, topk, ns, nd, dim):
    print(f"[similarity] topk={topk} ns={ns} nd={nd} dim={dim}", flush=True)
    g = torch.Generator().manual_seed(ns + nd + topk)
    src = F.normalize(torch.randn(ns, dim, generator=g), dim=-1).bfloat16()
    dst = F.normalize(torch.randn(nd, dim, generator=g), dim=-1).bfloat16()
    dst[5] = dst[3]  # exact duplicate column: guaranteed ties
    scores = torch.full((ns, nd), float("nan"), dtype=torch.bfloat16, device=device)
    values, index = kern.similarity_topk(src.to(device), dst.to(device), topk, scores=scores)
    scores = scores.float().cpu()
    # (1) the kernel's bf16 scores are the exact-dot bf16 scores up to rare 1-ulp cases
    exact = om.bf16_scores(src, dst)
    mismatch = scores != exact
    assert mismatch.float().mean() < 5e-3
    if mismatch.any():
        assert ((scores - exact).abs()[mismatch] <= score_tolerance(exact)[mismatch]).all()
    # (2) given those scores, the selection is bit-exact (ties to the lower index)
    ref_v, ref_i = om.topk_lowest_index(scores, topk)
    assert torch.equal(index.cpu(), ref_i)
    assert torch.equal(values.cpu(), ref_v)


@pytest.mark.parametrize("dim", [64, 72])
@pytest.mark.parametrize("topk", [1, 4])
@pytest.mark.parametrize("nd", [768, 1000])
def test_similarity_topk_on_crafted_rounding_ties(kern, device, nd, topk, dim):
    """With dim 64, full 256-row dictionary tiles take the two-pass top-1 epilogue (the
    fp32 maximum, then the first score at or above the lower bound of its bf16 rounding
    interval); dim 72 takes the 128-row kernel.  The dictionary puts scores exactly on
    bf16 midpoints (ties to even, up and down), a quarter ulp either side of them and on
    bf16 values, so several fp32 scores at several positions round to each row's maximum;
    source rows negate them, zero them, and one row (in another wave, which then takes the
    per-score path) makes inf scores and a NaN (inf * 0, whose sign bit the hardware sets)
    that must rank above +inf after the dictionary parts are merged.  All products and
    sums are exact in fp32, so the kernel's scores equal the exact ones and the selection
    must be the lowest indices of the bf16 maxima."""
    print(f"[similarity] crafted rounding ties nd={nd} topk={topk} dim={dim}", flush=True)
    g = torch.Generator().manual_seed(nd)
    half = 2.0 ** -9
    k = torch.randint(-2, 3, (nd,), generator=g).float()
    c = torch.tensor([-1.0, -0.5, 0.0, 0.5, 1.0])[torch.randint(0, 5, (nd,), generator=g)]
    dst = torch.zeros(nd, dim)
    dst[:, 0] = 0.75 + k * 2.0 ** -8
    dst[:, 1] = c
    dst[7, 0], dst[7, 1] = 0.0, 1.0  # inf * 0: a NaN score for the overflow row
    kinds = [(1.0, half), (-1.0, -half), (0.0, 0.0), (1.0, -half), (0.5, half), (-0.5, half)]
    src = torch.zeros(128, dim)
    for i in range(128):
        src[i, :2] = torch.tensor(kinds[i % len(kinds)])
    src[100, :2] = torch.tensor([float("inf"), 0.0])
    src_b, dst_b = src.bfloat16(), dst.bfloat16()
    assert torch.equal(src_b.float(), src) and torch.equal(dst_b.float(), dst)
    scores = torch.full((128, nd), float("nan"), dtype=torch.bfloat16, device=device)
    values, index = kern.similarity_topk(src_b.to(device), dst_b.to(device), topk, scores=scores)
    ks = scores.float().cpu()
    exact = om.bf16_scores(src_b, dst_b)
    assert torch.equal(ks.isnan(), exact.isnan()) and torch.equal(ks.nan_to_num(), exact.nan_to_num())
    ref_v, ref_i = om.topk_lowest_index(ks, topk)
    assert ref_i[100, 0] == 7  # the NaN ranks first
    assert torch.equal(index.cpu(), ref_i)
    assert torch.equal(values.cpu().isnan(), ref_v.isnan())
    assert torch.equal(values.cpu().nan_to_num(), ref_v.nan_to_num())
    # the data really tie: rows whose maximum several positions reach, with different fp32 scores
    fp32 = src_b.double() @ dst_b.double().T
    row = 0
    at_max = ks[row] == ks[row].max()
    assert int(at_max.sum()) > 1 and fp32[row][at_max].unique().numel() > 1


def test_similarity_ranges_rows_and_device_count(kern, device):
    g = torch.Generator().manual_seed(3)
    src = F.normalize(torch.randn(500, 256, generator=g), dim=-1).bfloat16()
    dst = F.normalize(torch.randn(900, 256, generator=g), dim=-1).bfloat16()
    rows = torch.randperm(500, generator=g)[:300]
    count = torch.tensor([211], dtype=torch.int32)
    index_map = torch.arange(900) * 7 + 3
    n0, off1, n_dict = 128, 400, 128 + 300
    scores = torch.full((300, n_dict), float("nan"), dtype=torch.bfloat16, device=device)
    values, index = kern.similarity_topk(
        src.to(device), dst.to(device), 4, src_rows=rows.to(device), n_src_device=count.to(device),
        n_src=300, dict_ranges=(n0, off1, n_dict), index_map=index_map.to(device), scores=scores)
    positions = torch.cat((torch.arange(n0), torch.arange(off1, off1 + n_dict - n0)))
    kernel_scores = scores[:211].float().cpu()
    exact = om.bf16_scores(src[rows[:211]], dst[positions])
    assert ((kernel_scores - exact).abs() <= score_tolerance(exact)).all()
    ref_v, ref_i = om.topk_lowest_index(kernel_scores, 4)
    assert torch.equal(values[:211].cpu(), ref_v)
    assert torch.equal(index[:211].cpu(), index_map[positions[ref_i]])
    assert torch.isnan(scores[211:].float()).all()  # rows past the device count are untouched


@pytest.mark.parametrize("dim", [256, 72])
def test_similarity_invalid_source_ids_score_zero(kern, device, dim):
    # Row ids outside the source buffer read as zero rows: every score is 0 and
    # the lowest dictionary indices win (both kernels: dim 256 and dim 72).
    g = torch.Generator().manual_seed(6)
    src = F.normalize(torch.randn(200, dim, generator=g), dim=-1).bfloat16()
    dst = F.normalize(torch.randn(300, dim, generator=g), dim=-1).bfloat16()
    rows = torch.arange(200)
    rows[[0, 77, 150]] = torch.tensor([200, 10 ** 6, -1])
    for topk in (1, 4):
        values, index = kern.similarity_topk(src.to(device), dst.to(device), topk, src_rows=rows.to(device),
                                             n_src=200)
        v, i = values.cpu(), index.cpu()
        for r in (0, 77, 150):
            assert torch.equal(v[r].reshape(-1), torch.zeros(topk))
            assert torch.equal(i[r].reshape(-1), torch.arange(topk))
        good = torch.ones(200, dtype=torch.bool)
        good[[0, 77, 150]] = False
        exact = om.bf16_scores(src[rows[good]], dst)
        ref_v, ref_i = om.topk_lowest_index(exact, topk)
        ok = (v[good].reshape(ref_v.shape) == ref_v).all(-1)
        assert ok.float().mean() > 0.99  # exact-dot ties aside (see the selection test)


def test_streaming_top4_api(vgo, device):
    g = torch.Generator().manual_seed(4)
    q = torch.randn(64, 128, generator=g)
    basis_t = torch.randn(128, 40, generator=g)
    values, index = vgo.streaming_top4(q.to(device), basis_t.to(device))
    assert values.shape == (64, 4) and index.dtype == torch.int64
    exact = om.bf16_scores(q.bfloat16(), basis_t.T.bfloat16())
    ref_v, _ = om.topk_lowest_index(exact, 4)
    assert (values.cpu() - ref_v).abs().max() <= float(ulp_bf16(ref_v).max())
    with pytest.raises(ValueError, match="at least four"):
        vgo.streaming_top4(q.to(device), basis_t[:, :3].to(device))


# ------------------------------------------------------ rank and select ----
@pytest.mark.parametrize("batch,ns,nd,removed,keys", [
    (1, 50, 20, 1, "bf16"), (2, 3000, 900, 1700, "bf16"), (1, 5000, 100, 5000, "bf16"),
    (1, 20000, 7000, 12345, "bf16"), (1, 70000, 3000, 40000, "bf16"),
    (2, 23808, 8960, 16464, "fp32"),   # C4 sizes; full 32-bit keys with repeated values
    (1, 4097, 10, 2049, "fp32"),       # group boundaries of the multi-group path
])
@pytest.mark.parametrize("entry", ["one_group", "workspace"])
def test_fastvggt_assemble_exact(vgo, kern, device, batch, ns, nd, removed, keys, entry):
    print(f"[assemble] {entry} batch={batch} ns={ns} removed={removed} keys={keys}", flush=True)
    g = torch.Generator().manual_seed(ns + removed)
    total = ns + nd + 37
    perm = torch.randperm(total, generator=g)
    sources = perm[:ns].sort().values
    dests = perm[ns:ns + nd].sort().values
    if keys == "bf16":
        # bf16-valued scores with heavy ties
        best = (torch.randint(0, 40, (batch, ns), generator=g).float() / 64).to(torch.bfloat16).float()
    else:
        # fp32 scores: every bit of the key matters; a few values repeat, one is negative zero
        best = torch.rand(batch, ns, generator=g) * 2 - 1
        best[:, ::97] = best[:, 5:6]
        best[:, 3] = -0.0
        best[:, 4] = 0.0
    target = torch.randint(0, nd, (batch, ns), generator=g, dtype=torch.int32)
    keep = torch.empty((batch, total - removed), dtype=torch.int64, device=device)
    inverse = torch.empty((batch, total), dtype=torch.int64, device=device)
    flags = torch.empty((batch, ns), dtype=torch.uint8, device=device)
    best_d, target_d = best.to(device), target.to(device)
    sources_d, dests_d = sources.to(device), dests.to(device)
    lib = import_package("_lib")
    args = (best_d.data_ptr(), target_d.data_ptr(), sources_d.data_ptr(), dests_d.data_ptr(), batch,
            ns, nd, total, removed, keep.data_ptr(), inverse.data_ptr(), flags.data_ptr())
    stream = torch.cuda.current_stream().cuda_stream
    if entry == "one_group":
        status = lib.load().vgo_fastvggt_assemble(*args, stream)
    else:
        import ctypes
        need = ctypes.c_size_t(0)
        lib.check(lib.load().vgo_fastvggt_assemble_workspace(batch, ns, total, ctypes.byref(need)))
        ws = torch.full((need.value // 4,), 7, dtype=torch.int32, device=device)  # not zeroed on purpose
        status = lib.load().vgo_fastvggt_assemble_ws(*args, ws.data_ptr(), need.value, stream)
    lib.check(status)
    torch.cuda.synchronize()
    for b in range(batch):
        rk, ri = om.fastvggt_select(best[b], target[b].long(), sources, dests, total, removed)
        assert torch.equal(keep[b].cpu(), rk)
        assert torch.equal(inverse[b].cpu(), ri)
        removed_ids = torch.ones(total, dtype=torch.bool)
        removed_ids[rk] = False
        assert torch.equal(flags[b].cpu().bool(), removed_ids[sources])


# --------------------------------------------------------- FastVGGT plan ----
@pytest.mark.parametrize("tag,ratio,protect", [("fv50", 0.5, 0.0), ("fvdef", 0.9, 0.10)])
def test_fastvggt_plan_vs_reference(vgo, kern, device, fx, tag, ratio, protect):
    """The GPU plan against the reference's own plan, unconditionally.

    keep/inverse must equal the reference fixture, except where a source lies in
    the tie band of the scores: the kernel's bf16 scores and the reference's
    recorded bf16 scores each lie within one ulp of the exact dot product, so
    they may differ by up to two; a source whose best score is that close to
    the removal cutoff may swap removal status, and a source whose best and
    another destination's score are that close may swap target.  Every
    difference must be explained that way; the fractions are printed."""
    tokens = structured_tokens(1, 4, (16, 16), 5, 1024)
    plan = vgo.build_fastvggt_plan(tokens.to(device), merge_ratio=ratio, protect_ratio=protect, **KW)
    sources, dests, best, target, _ = plan._derived["match"]
    total, removed = 1044, plan.original_tokens - plan.kept_tokens
    # selection is exact given the kernel's scores
    rk, ri = om.fastvggt_select(best[0].cpu(), target[0].cpu().long(), sources.cpu(), dests.cpu(),
                                total, removed)
    assert torch.equal(plan.keep[0].cpu(), rk) and torch.equal(plan.inverse[0].cpu(), ri)
    # the kernel's full score matrix on the planner's operands
    x = tokens[0].to(device)
    src = kern.normalize_rows(x, sources, 1e-12)
    dst = kern.normalize_rows(x, dests, 1e-12)
    scores = torch.full((sources.numel(), dests.numel()), float("nan"), dtype=torch.bfloat16, device=device)
    kern.similarity_topk(src, dst, 1, scores=scores)
    ks = scores.float().cpu()
    assert torch.equal(ks.max(1).values, best[0].cpu())
    ref = torch.from_numpy(fx[f"{tag}_scores"]).view(torch.bfloat16).float()
    mismatch = ks != ref
    assert ((ks - ref).abs()[mismatch] <= 2 * score_tolerance(ref)[mismatch]).all()
    # the oracle's selection on the reference's own scores is the reference's plan
    ref_best, ref_target = ref.max(1)
    ok_keep, ok_inv = om.fastvggt_select(ref_best, ref_target, sources.cpu(), dests.cpu(), total, removed)
    assert np.array_equal(ok_keep.numpy(), fx[f"{tag}_keep"])
    assert np.array_equal(ok_inv.numpy(), fx[f"{tag}_inverse"])
    # GPU plan vs the reference's, source by source
    src_cpu, dst_cpu = sources.cpu(), dests.cpu()
    fx_keep = torch.from_numpy(fx[f"{tag}_keep"])
    fx_inv = torch.from_numpy(fx[f"{tag}_inverse"])
    removed_gpu = ~torch.isin(src_cpu, plan.keep[0].cpu())
    removed_ref = ~torch.isin(src_cpu, fx_keep)
    kbest = best[0].cpu()
    cutoff = kbest.sort(descending=True).values[removed - 1]
    rank_band = (kbest - cutoff).abs() <= 2 * score_tolerance(cutoff.expand_as(kbest))
    top2 = ks.topk(2, dim=1).values
    target_band = (top2[:, 0] - top2[:, 1]) <= 2 * score_tolerance(top2[:, 0])
    status_diff = removed_gpu != removed_ref
    assert rank_band[status_diff].all(), "a removal difference outside the tie band"
    both = removed_gpu & removed_ref
    gpu_target = plan.keep[0].cpu()[plan.inverse[0].cpu()[src_cpu]]
    ref_target_orig = fx_keep[fx_inv[src_cpu]]
    target_diff = both & (gpu_target != ref_target_orig)
    if target_diff.any():
        col = {int(d): j for j, d in enumerate(dst_cpu.tolist())}
        for i in target_diff.nonzero().flatten().tolist():
            other = ks[i, col[int(ref_target_orig[i])]]
            assert ks[i].max() - other <= 2 * score_tolerance(ks[i].max()), "target difference outside the tie band"
    if not (status_diff.any() or target_diff.any()):
        assert torch.equal(plan.keep[0].cpu(), fx_keep) and torch.equal(plan.inverse[0].cpu(), fx_inv)
    print(f"[fastvggt vs reference] {tag}: scores differ in {mismatch.float().mean().item():.2e} of "
          f"entries (<= 2 ulp); tie band: {target_band.float().mean().item():.3f} of sources (target), "
          f"{rank_band.float().mean().item():.3f} (cutoff); plan differences: "
          f"{int(status_diff.sum())} removal, {int(target_diff.sum())} target", flush=True)


def test_fastvggt_plan_batch_and_determinism(vgo, device):
    tokens = torch.cat([structured_tokens(s, 4, (16, 16), 5, 256) for s in (5, 6)]).to(device)
    a = vgo.build_fastvggt_plan(tokens, merge_ratio=0.5, protect_ratio=0.1, **KW)
    b = vgo.build_fastvggt_plan(tokens, merge_ratio=0.5, protect_ratio=0.1, **KW)
    assert torch.equal(a.keep, b.keep) and torch.equal(a.inverse, b.inverse)
    for i in range(2):
        single = vgo.build_fastvggt_plan(tokens[i:i + 1], merge_ratio=0.5, protect_ratio=0.1, **KW)
        assert torch.equal(single.keep[0], a.keep[i])
    with pytest.raises(ValueError, match="layout"):
        vgo.build_fastvggt_plan(tokens[:, :1000], merge_ratio=0.5, **KW)
    ident = vgo.build_fastvggt_plan(tokens, merge_ratio=0.0, **KW)
    assert ident.kept_tokens == 1044


# --------------------------------------------------- CSR, mass, compact ----
@pytest.mark.parametrize("n,buckets", [(1, 1), (1000, 37), (70000, 9000), (300000, 4)])
def test_csr_is_a_stable_bucket_sort(kern, device, n, buckets):
    g = torch.Generator().manual_seed(n)
    keys = torch.randint(0, buckets + 3, (n,), generator=g)  # some out of range: dropped
    order, offsets = kern.csr_build(keys.to(device), buckets)
    valid = keys < buckets
    ref_order = torch.argsort(torch.where(valid, keys, buckets), stable=True)[: int(valid.sum())]
    counts = torch.bincount(keys[valid], minlength=buckets)
    ref_offsets = torch.cat((torch.zeros(1, dtype=torch.long), counts.cumsum(0)))
    assert torch.equal(order.cpu()[: int(valid.sum())].long(), ref_order)
    assert torch.equal(offsets.cpu().long(), ref_offsets)


def _random_weighted_plan(seed, total, kept, sources, one_hot=False):
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(total, generator=g)
    keep = perm[:kept].sort().values
    src = perm[kept:kept + sources].sort().values
    parent = torch.stack([torch.randperm(kept, generator=g)[:4] for _ in range(sources)])
    e = -torch.rand(sources, 4, generator=g, dtype=torch.float64).log()
    w = (e / e.sum(1, keepdim=True)).float()
    if one_hot:
        w = torch.zeros(sources, 4)
        w[:, 0] = 1
    return keep, src, parent, w


@pytest.mark.parametrize("one_hot", [False, True])
def test_deterministic_mass_bit_exact(vgo, device, one_hot):
    keep, src, parent, w = _random_weighted_plan(11, 3000, 900, 2000, one_hot)
    mass = vgo.deterministic_weighted_normalizer(parent[None].to(device), w[None].to(device), 900)
    ref = om.deterministic_weighted_normalizer(parent[None], w[None], 900)
    assert torch.equal(mass.cpu(), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_weighted_plan_compact_restore_bit_exact(vgo, device, dtype):
    print(f"[weighted plan] dtype={dtype}", flush=True)
    keep, src, parent, w = _random_weighted_plan(12, 2500, 700, 1800)
    mass = om.deterministic_weighted_normalizer(parent[None], w[None], 700)
    plan = vgo.WeightedBilinearTokenPlan(
        keep=keep[None].to(device), source_original=src[None].to(device),
        source_parent_compact=parent[None].to(device), source_pool_weights=w[None].to(device),
        source_restore_weights=w[None].to(device), original_tokens=2500,
        normalizer=mass.to(device))
    value = seeded_values(5, (1, 2500, 1024), dtype)
    out = plan.compact(value.to(device))
    ref = om.weighted_compact(keep, src, parent, w, mass, value[0])
    assert torch.equal(out[0].cpu(), ref)
    small = seeded_values(6, (1, 700, 1024), dtype)
    restored = plan.restore(small.to(device))
    assert torch.equal(restored[0].cpu(), om.weighted_restore(keep, src, parent, w, 2500, small[0]))
    # head-major [H, N, 64] views compact the same way without copies
    hm = value[0].reshape(2500, 16, 64).transpose(0, 1).contiguous().to(device)
    out_hm = torch.empty((16, 700, 64), dtype=dtype, device=device)
    plan.compact_into(hm, out_hm)
    assert torch.equal(out_hm.transpose(0, 1).reshape(700, 1024).cpu(), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_weighted_plan_compact_edge_normalizers(vgo, device, dtype):
    """Normalizers outside the counts-and-masses range [1, 2^16] and rows of
    tiny values take the plain division; the result is still the oracle's."""
    print(f"[edge normalizers] dtype={dtype}", flush=True)
    keep, src, parent, w = _random_weighted_plan(13, 2000, 600, 1400)
    mass = om.deterministic_weighted_normalizer(parent[None], w[None], 600).clone()
    edges = [0.25, 1e-20, 1e20, 70000.3, 65536.0, 65535.5, float("inf"), 0.75, 1.0, 3.0]
    for i, e in enumerate(edges):
        mass[0, 7 * i] = e
    plan = vgo.WeightedBilinearTokenPlan(
        keep=keep[None].to(device), source_original=src[None].to(device),
        source_parent_compact=parent[None].to(device), source_pool_weights=w[None].to(device),
        source_restore_weights=w[None].to(device), original_tokens=2000,
        normalizer=mass.to(device))
    # scales: in range; straddling 2^-100; results down in the subnormals
    for scale in (1.0, 1e-28, 1e-37):
        value = (seeded_values(14, (1, 2000, 1024), torch.float32) * scale).to(dtype)
        out = plan.compact(value.to(device))
        ref = om.weighted_compact(keep, src, parent, w, mass[0], value[0])
        assert torch.equal(out[0].cpu(), ref), scale


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_compaction_of_rows_wider_than_1024_channels(vgo, device, dtype):
    """Rows of 1,536 and 2,048 channels (two 1,024-channel passes per wave): a weighted
    plan (four segments per row) and a token plan (one segment, no base row) against
    the oracle, bit for bit."""
    print(f"[compact] wide rows {dtype}", flush=True)
    keep, src, parent, w = _random_weighted_plan(15, 1500, 500, 900)
    mass = om.deterministic_weighted_normalizer(parent[None], w[None], 500)
    plan = vgo.WeightedBilinearTokenPlan(
        keep=keep[None].to(device), source_original=src[None].to(device),
        source_parent_compact=parent[None].to(device), source_pool_weights=w[None].to(device),
        source_restore_weights=w[None].to(device), original_tokens=1500, normalizer=mass.to(device))
    value = seeded_values(16, (1, 1500, 2048), dtype)
    out = plan.compact(value.to(device))
    assert torch.equal(out[0].cpu(), om.weighted_compact(keep, src, parent, w, mass, value[0]))
    tokens = structured_tokens(17, 4, (16, 16), 5, 256).to(device)
    tplan = vgo.build_fastvggt_plan(tokens, merge_ratio=0.5, protect_ratio=0.0, **KW)
    value = seeded_values(18, (1, tokens.shape[1], 1536), dtype)
    out = tplan.compact(value.to(device))
    ref = om.token_plan_compact(tplan.inverse[0].cpu(), tplan.kept_tokens, value[0])
    assert torch.equal(out[0].cpu(), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_token_plan_compact_restore_bit_exact(vgo, device, fx, dtype):
    inv = torch.from_numpy(fx["fv50_inverse"])
    keep = torch.from_numpy(fx["fv50_keep"])
    plan = vgo.TokenPlan(keep[None].to(device), inv[None].to(device), 1044)
    value = seeded_values(7, (1, 1044, 32), dtype)
    out = plan.compact(value.to(device))
    assert torch.equal(out[0].cpu(), om.token_plan_compact(inv, keep.numel(), value[0]))
    assert rel_error(out[0].cpu(), torch.from_numpy(fx[f"fv_compact_{'f32' if dtype == torch.float32 else 'bf16'}"])) <= (1e-6 if dtype == torch.float32 else 1e-2)
    gathered = plan.compact(value.to(device), merge=False)
    assert torch.equal(gathered[0].cpu(), value[0][keep])
    small = seeded_values(8, (1, keep.numel(), 32), dtype)
    restored = plan.restore(small.to(device))
    assert torch.equal(restored[0].cpu(), small[0][inv])


# ------------------------------------------------------------ convex fit ----
def test_convex_fit_matches_oracle(vgo, device):
    tokens = structured_tokens(1, 4, (16, 16), 5, 1024)
    o = om.sparse_convex_plan(tokens, threshold=0.9, **KW)
    hard = o["hard"]
    rows = o["candidate"][hard]
    supports = o["support"][hard].contiguous()
    fit, alpha = vgo.convex_fit(tokens[0].to(device), rows.to(device), supports.clone().to(device))
    normalized = F.normalize(tokens[0], dim=-1, eps=1e-6)
    ref_fit, ref_alpha = om.convex_fit(F.normalize(normalized[rows], dim=-1, eps=1e-6),
                                       F.normalize(normalized[supports], dim=-1, eps=1e-6))
    assert (fit.cpu() - ref_fit).abs().max() < 2e-5
    assert (alpha.cpu() - ref_alpha).abs().max() < 2e-3
    assert torch.allclose(alpha.sum(1).cpu(), torch.ones(len(hard)), atol=1e-5)


# --------------------------------------------------------- sparse convex ----
def test_sparse_convex_plan_vs_oracle_and_reference(vgo, device, fx):
    tokens = structured_tokens(1, 4, (16, 16), 5, 1024)
    plan = vgo.build_sparse_convex_plan(tokens.to(device), threshold=0.9, **KW)
    o = om.sparse_convex_plan(tokens, threshold=0.9, **KW)
    fit = plan._derived["fit"][0].cpu()
    # Decisions agree except for fits within fp32 rounding of the threshold.
    assert not ((o["fit"] - 0.9).abs() < 1e-5).any(), "fixture has a fit inside the rounding band"
    assert torch.equal(plan.keep[0].cpu(), o["keep"])
    assert torch.equal(plan.source_original[0].cpu(), o["source_original"])
    assert (fit - o["fit"]).abs().max() < 2e-5
    assert (plan.source_pool_weights[0].cpu() - o["weights"]).abs().max() < 2e-3
    same_parent = (plan.source_parent_compact[0].cpu() == o["parent_compact"]).all(1)
    assert same_parent.float().mean() > 0.99
    assert torch.equal(plan.special_query_compact.cpu(), o["special_compact"])
    # mass is the deterministic normalizer of the plan's own parents/weights, bit-exact
    ref_mass = om.deterministic_weighted_normalizer(plan.source_parent_compact.cpu(),
                                                    plan.source_pool_weights.cpu(), plan.kept_tokens)
    assert torch.equal(plan.normalizer.cpu(), ref_mass)
    assert rel_error(plan.key_log_mass.cpu().reshape(-1), ref_mass.reshape(-1).log()) < 1e-6
    # against the reference fixture: same keep/sources, weights to tolerance
    assert np.array_equal(plan.keep[0].cpu().numpy(), fx["sc_keep"])
    assert np.array_equal(plan.source_original[0].cpu().numpy(), fx["sc_source"])
    assert np.abs(plan.source_pool_weights[0].cpu().numpy() - fx["sc_weight"]).max() < 2e-3
    md = plan.metadata
    assert md["hard_candidates"] == 393 and md["fallback_candidates"] == 390
    assert abs(md["merge_ratio"] - 186 / 1044) < 1e-9


def test_sparse_convex_plan_without_merges(vgo, device):
    """Unstructured tokens: no source passes the fit threshold, so the plan keeps every
    token (as the oracle does), its mass is 1 and compaction / restore are copies."""
    print("[merge] sparse-convex plan with no merges", flush=True)
    tokens = torch.randn(1, 4 * 261, 256, generator=torch.Generator().manual_seed(3))
    o = om.sparse_convex_plan(tokens, threshold=0.9, **KW)
    assert o["source_original"].numel() == 0
    plan = vgo.build_sparse_convex_plan(tokens.to(device), threshold=0.9, **KW)
    assert torch.equal(plan.keep[0].cpu(), o["keep"]) and plan.source_original.numel() == 0
    assert plan.kept_tokens == plan.original_tokens == 1044
    assert torch.equal(plan.normalizer.reshape(-1).cpu(), torch.ones(1044))
    x = tokens.to(device)
    assert torch.equal(plan.compact(x), x)
    assert torch.equal(plan.restore(x), x)


# ---------------------------------------------------------- attention layer ----
@pytest.mark.parametrize("tag,preserve", [("attn_qkv", False), ("attn_kv", True)])
def test_self_attention_layer_vs_reference(vgo, device, fx, tag, preserve):
    print(f"[layer] {tag}", flush=True)
    x = structured_tokens(3, 4, (16, 16), 5, 128)
    layer = vgo.SelfAttention(128, num_heads=2, qkv_bias=True, mask_k_bias=True,
                              use_qk_norm=True).eval().to(device)
    layer.load_state_dict(attention_weights(4, 128))
    keep = torch.from_numpy(fx[f"{tag}_keep"])
    parent = torch.from_numpy(fx[f"{tag}_parent"])
    w = torch.from_numpy(fx[f"{tag}_weight"])
    mass = torch.from_numpy(fx[f"{tag}_mass"])
    special = (torch.arange(4)[:, None] * 261 + torch.arange(5)[None]).flatten()
    plan = vgo.WeightedBilinearTokenPlan(
        keep=keep[None].to(device), source_original=torch.from_numpy(fx[f"{tag}_source"])[None].to(device),
        source_parent_compact=parent[None].to(device), source_pool_weights=w[None].to(device),
        source_restore_weights=w[None].to(device), original_tokens=1044,
        normalizer=mass.view(1, -1, 1).to(device), preserve_queries=preserve,
        preserve_destination_keys=preserve, dense_special_queries=True,
        special_query_original=special.to(device),
        special_query_compact=torch.from_numpy(fx[f"{tag}_special_compact"]).to(device),
        key_log_mass=mass.log().view(1, -1).to(device))
    with torch.no_grad():
        out = layer(x.to(device), token_plan=plan)
    assert_close(out[0].cpu(), torch.from_numpy(fx[f"{tag}_out"]), torch.float32, rtol=2e-5,
                 what=f"{tag} fp32 layer")
    # bf16 autocast path against the oracle's bf16-autocast semantics
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        out_bf16 = layer(x.to(device), token_plan=plan)
    assert out_bf16.dtype == torch.bfloat16
    oplan = dict(keep=keep, source_original=torch.from_numpy(fx[f"{tag}_source"]),
                 parent_compact=parent, weights=w, mass=mass, special_original=special,
                 special_compact=torch.from_numpy(fx[f"{tag}_special_compact"]))
    ref_bf16 = oracle_layer.self_attention(x[0], attention_weights(4, 128), 2, oplan, preserve,
                                           autocast_bf16=True)
    assert_close(out_bf16[0].float().cpu(), ref_bf16.float(), torch.bfloat16,
                 what=f"{tag} bf16 layer")


def test_block_forward_compacted(vgo, device):
    torch.manual_seed(0)
    block = vgo.SelfAttentionBlock(256, 4, qkv_bias=True, init_values=0.5, mask_k_bias=True,
                                   use_qk_norm=True).eval().to(device)
    x = structured_tokens(9, 4, (16, 16), 5, 256).to(device)
    plan = vgo.build_sparse_convex_plan(block.norm1(x), threshold=0.9, **KW)
    with torch.no_grad():
        out = block.forward_compacted(x, plan)
        normalized = block.norm1(x)
        again = block.forward_compacted(x, plan, normalized=normalized)
    assert torch.equal(out, again)
    assert out.shape == x.shape and torch.isfinite(out).all()
    block.train()
    with pytest.raises(RuntimeError, match="inference-only"):
        block.forward_compacted(x, plan)


def test_aggregator_runs_both_planners(device):
    agg = import_package("aggregator")
    torch.manual_seed(0)
    model = agg.Aggregator(embed_dim=256, depth=3, num_heads=4, num_register_tokens=4,
                           register_attention_block_indices=(1,),
                           cached_layer_indices=(2,)).to(device).eval()
    patches = structured_tokens(2, 4, (16, 16), 5, 256)[0].view(4, 261, 256)[:, 5:].contiguous()
    model.set_input_patch_tokens_cache(patches.to(device))
    images = torch.zeros(1, 4, 3, 256, 256, device=device)
    with pytest.raises(RuntimeError, match="patch encoder"):
        fresh = agg.Aggregator(embed_dim=256, depth=1, num_heads=4, num_register_tokens=4,
                               register_attention_block_indices=()).to(device)
        fresh(images)
    model.set_fastvggt(True, merge_ratio=0.5, protect_ratio=0.0, mass_bias=True)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        outputs, start = model(images)
    assert start == 5 and outputs[2].shape == (1, 4, 261, 512) and torch.isfinite(outputs[2]).all()
    assert [s["kept_tokens"] for s in model.fastvggt_last_plan_stats] == [522, 522]
    model.set_fastvggt(False)
    model.set_sparse_convex(True, threshold=0.9, qkv_global_blocks=1, qkv_global_layers=(0,))
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        outputs, _ = model(images)
    assert torch.isfinite(outputs[2]).all() and len(model.sparse_convex_last_plan_stats) == 2
    with pytest.raises(ValueError, match="mutually exclusive"):
        model.set_fastvggt(True)


# ------------------------------------------------------- fused epilogue ----
def _ref_epilogue(qkv, heads, tokens, qn, kn, sin, cos, prefix):
    """Reference op sequence (attention.py:334-341, 243-262) in fp32 on the CPU."""
    n, c3 = qkv.shape
    c = c3 // 3
    x = qkv.float().view(n // tokens, tokens, 3, heads, 64)
    q, k, v = x[:, :, 0], x[:, :, 1], x[:, :, 2]  # [S, T, H, 64]
    q = F.layer_norm(q, (64,), qn[0], qn[1], 1e-5)
    k = F.layer_norm(k, (64,), kn[0], kn[1], 1e-5)

    def rope(t):
        body = t[:, prefix:]
        half = torch.cat([-body[..., 32:], body[..., :32]], dim=-1)
        return torch.cat([t[:, :prefix], body * cos[:, None] + half * sin[:, None]], dim=1)

    if sin is not None:
        q, k = rope(q), rope(k)
    hm = lambda t: t.permute(0, 2, 1, 3)  # noqa: E731
    return hm(q), hm(k), hm(v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_qkv_epilogue_layer_norm_and_rope(kern, device, dtype):
    layers = import_package("layers")
    g = torch.Generator().manual_seed(21)
    heads, tokens, seqs = 4, 261, 3
    qkv = torch.randn(seqs * tokens, 3 * heads * 64, generator=g).to(dtype)
    qn = (1 + 0.1 * torch.randn(64, generator=g), 0.1 * torch.randn(64, generator=g))
    kn = (1 + 0.1 * torch.randn(64, generator=g), 0.1 * torch.randn(64, generator=g))
    sin, cos = layers.rope_sincos(16, 16, 64)
    q, k, v = kern.qkv_epilogue(qkv.to(device), heads, tokens_in=tokens,
                                q_norm=(qn[0].to(device), qn[1].to(device)),
                                k_norm=(kn[0].to(device), kn[1].to(device)),
                                rope=(sin.to(device), cos.to(device)), rope_prefix=5, out_dtype=dtype)
    rq, rk, rv = _ref_epilogue(qkv, heads, tokens, qn, kn, sin, cos, 5)
    tol = 1e-5 if dtype == torch.float32 else 8e-3
    assert_close(q.cpu(), rq.to(dtype), rtol=tol, what="epilogue q")
    assert_close(k.cpu(), rk.to(dtype), rtol=tol, what="epilogue k")
    assert torch.equal(v.cpu(), rv.to(dtype))
    # row-list variant (special queries) and no-RoPE variant
    rows = torch.tensor([0, 5, 261, 700])
    (qs,) = kern.qkv_epilogue(qkv.to(device), heads, tokens_in=tokens, tokens_out=4, rows=rows.to(device),
                              q_norm=(qn[0].to(device), qn[1].to(device)), want=(True, False, False),
                              out_dtype=dtype)[:1]
    flat_ref = F.layer_norm(qkv.float().view(-1, 3, heads, 64)[:, 0], (64,), qn[0], qn[1], 1e-5)
    assert_close(qs[0].cpu(), flat_ref[rows].permute(1, 0, 2).to(dtype), rtol=tol, what="row list")


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_compaction_with_fused_layer_norm(vgo, device, out_dtype):
    keep, src, parent, w = _random_weighted_plan(31, 2000, 600, 1400)
    mass = om.deterministic_weighted_normalizer(parent[None], w[None], 600)
    plan = vgo.WeightedBilinearTokenPlan(
        keep=keep[None].to(device), source_original=src[None].to(device),
        source_parent_compact=parent[None].to(device), source_pool_weights=w[None].to(device),
        source_restore_weights=w[None].to(device), original_tokens=2000, normalizer=mass.to(device))
    g = torch.Generator().manual_seed(32)
    qkv = torch.randn(2000, 3 * 1024, generator=g).bfloat16()
    lw, lb = 1 + 0.1 * torch.randn(64, generator=g), 0.1 * torch.randn(64, generator=g)
    qkv_d = qkv.to(device)
    out = torch.empty((16, 600, 64), device=device, dtype=out_dtype)
    plan.compact_into(qkv_d[:, :1024], out, layer_norm=(lw.to(device), lb.to(device), 1e-5))
    normed = F.layer_norm(qkv[:, :1024].float().view(2000, 16, 64), (64,), lw, lb, 1e-5).view(2000, 1024)
    ref = om.weighted_compact(keep, src, parent, w, mass, normed)
    got = out.transpose(0, 1).reshape(600, 1024).cpu()
    assert_close(got, ref.to(out_dtype), rtol=1e-5 if out_dtype == torch.float32 else 8e-3,
                 what="LN-fused compaction")


def test_dense_fused_attention_matches_reference_ops(vgo, device):
    layers = import_package("layers")
    torch.manual_seed(3)
    layer = vgo.SelfAttention(256, num_heads=4, qkv_bias=True, mask_k_bias=True,
                              use_qk_norm=True).eval().to(device)
    with torch.no_grad():
        layer.q_norm.weight.normal_(1.0, 0.1)
        layer.k_norm.bias.normal_(0.0, 0.1)
    x = structured_tokens(4, 3, (16, 16), 5, 256)[0].view(3, 261, 256).to(device)
    sin, cos = layers.rope_sincos(16, 16, 64, device=device)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        fused = layer(x, rope=(sin, cos))
        layer._fusable = lambda *a: False  # reference op sequence: torch LN, RoPE, SDPA
        general = layer(x, rope=(sin, cos))
    assert_close(fused.float().cpu(), general.float().cpu(), torch.bfloat16, what="frame attention")


@pytest.mark.parametrize("case,n_out", [("fastvggt", 3), ("fastvggt", 2), ("pool_mask", 1), ("pool_mask", 3)])
def test_token_plan_compact_multi_equals_single(vgo, device, case, n_out):
    """q/k/v compaction of one plan in one launch (vgo_compact_multi) equals the
    single-output launches bit for bit.  `pool_mask` plans (reference
    token_merging.py:161-191: only masked members contribute) take the same CSR
    path with 0/1 member weights."""
    print(f"[merge] compact multi {case} outputs={n_out}", flush=True)
    tokens = structured_tokens(21, 4, (16, 16), 5, 256).to(device)
    plan = vgo.build_fastvggt_plan(tokens, merge_ratio=0.5, protect_ratio=0.0, mass_bias=True, **KW)
    if case == "pool_mask":
        g = torch.Generator().manual_seed(23)
        mask = torch.rand(1, plan.original_tokens, generator=g) < 0.6
        mask[0, plan.keep[0].cpu()] = True  # every cluster keeps its physical member
        plan = vgo.TokenPlan(plan.keep, plan.inverse, plan.original_tokens, pool_mask=mask.to(device))
    g = torch.Generator(device=device).manual_seed(22)
    qkv = torch.randn(tokens.shape[1], 3 * 256, device=device, generator=g).bfloat16()
    ln = (1 + 0.1 * torch.randn(64, device=device, generator=g), 0.1 * torch.randn(64, device=device, generator=g), 1e-5)
    specs = [(0, ln), (256, ln), (512, None)][3 - n_out:]
    kept = plan.kept_tokens
    multi = [torch.empty(4, kept, 64, device=device, dtype=torch.bfloat16) for _ in specs]
    single = [torch.empty_like(m) for m in multi]
    plan.compact_multi_into(qkv, [(off, out, norm) for (off, norm), out in zip(specs, multi)])
    for (off, norm), out in zip(specs, single):
        plan.compact_into(qkv[:, off:off + 256], out, layer_norm=norm)
    for a, b in zip(multi, single):
        assert torch.equal(a, b)
    if case == "pool_mask":
        # the masked mean in float64 (one bf16 rounding of the fp32 result)
        x = qkv[:, 512:].float().cpu().double()
        inv, m = plan.inverse[0].cpu(), plan.pool_mask[0].cpu().double()
        sums = torch.zeros(kept, 256, dtype=torch.float64).index_add_(0, inv, x * m[:, None])
        counts = torch.zeros(kept, dtype=torch.float64).index_add_(0, inv, m)
        ref = sums / counts[:, None]
        got = multi[-1].transpose(0, 1).reshape(kept, 256).double().cpu()
        assert_close(got, ref, torch.bfloat16, rtol=8e-3, what="pool_mask compaction")


def test_compact_multi_rejects_mismatched_outputs(vgo, device):
    tokens = structured_tokens(21, 4, (16, 16), 5, 256).to(device)
    plan = vgo.build_fastvggt_plan(tokens, merge_ratio=0.5, protect_ratio=0.0, **KW)
    qkv = torch.zeros(tokens.shape[1], 3 * 256, device=device, dtype=torch.bfloat16)
    kept = plan.kept_tokens
    a = torch.empty(4, kept, 64, device=device, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="every output"):
        plan.compact_multi_into(qkv, [(0, a, None), (256, torch.empty(2, kept, 64, device=device,
                                                                      dtype=torch.bfloat16), None)])
    with pytest.raises(ValueError, match="outside"):
        plan.compact_multi_into(qkv, [(600, a, None)])
    ln1 = (torch.ones(64, device=device), torch.zeros(64, device=device), 1e-5)
    ln2 = (torch.ones(64, device=device), torch.zeros(64, device=device), 1e-6)
    with pytest.raises(ValueError, match="eps"):
        plan.compact_multi_into(qkv, [(0, a, ln1), (256, torch.empty_like(a), ln2)])
