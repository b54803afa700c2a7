"""Residual-stream rows (vgo_residual_layer_norm) against torch's op sequence.

* s = x + branch * gamma is compared bit for bit with torch's fp32 result on
  the CPU (the kernel performs the same two IEEE operations).
* LayerNorm(s) in fp32 is within the fp32 bar (1e-5) of `F.layer_norm` in
  float64, and the 16-bit copy is within half an ulp of such a value (one
  rounding of an fp32 result, as autocast's cast of torch's fp32 LayerNorm).
* Shapes cover the 4- and 8-chunk instantiations, dims that are not a multiple
  of 256, one row, rows not a multiple of the four rows per work-group, no
  gamma / no affine / no branch, and the in-place form.
* SelfAttentionBlock.forward and forward_compacted with the fused rows match
  the reference op sequence (torch LayerNorm, LayerScale, add, autocast casts)
  within the bf16 bar.
* The restore variant (vgo_restore_residual_layer_norm) equals the plan's
  top-4 projection followed by the plain row pass bit for bit (one-hot and
  four-way weights, zero weights, out-of-range ids giving NaN rows, three table
  dtypes), and forward_compacted through it equals the unfused restore + rows.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests._tol import assert_close
from tests.conftest import import_package
from tests.golden.inputs import structured_tokens

pytestmark = pytest.mark.gpu

KW = dict(frames=4, patch_hw=(16, 16), tokens_per_frame=261, patch_token_start=5)


@pytest.fixture(scope="module")
def kern():
    return import_package("_kernels")


def _inputs(rows, dim, branch_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, dim, generator=g) * 3 + 0.5
    branch = (torch.randn(rows, dim, generator=g) * 2).to(branch_dtype)
    gamma = torch.rand(dim, generator=g) * 0.7 + 0.05
    w = 1 + 0.2 * torch.randn(dim, generator=g)
    b = 0.1 * torch.randn(dim, generator=g)
    return x, branch, gamma, w, b


def _rounded_close(actual: torch.Tensor, ref64: torch.Tensor, dtype: torch.dtype, what: str):
    """actual (16-bit) is a round-to-nearest of some value within the fp32 bar of ref64:
    |actual - ref| <= ulp(actual) / 2 + 1e-5 * max(|ref|, rms(ref))."""
    got = actual.double().cpu()
    ref = ref64.double().cpu()
    _, expo = torch.frexp(got)
    half_ulp = torch.ldexp(torch.full_like(got, torch.finfo(dtype).eps / 2), expo - 1)
    scale = torch.maximum(ref.abs(), ref.pow(2).mean().sqrt())
    bad = (got - ref).abs() > half_ulp + 1e-5 * scale
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond half an ulp + the fp32 bar"


@pytest.mark.parametrize("rows,dim,branch_dtype,norm_dtype", [
    (1029, 1024, torch.bfloat16, torch.bfloat16),
    (5, 1024, torch.float16, torch.float16),
    (1, 256, torch.float32, torch.bfloat16),
    (333, 1028, torch.bfloat16, torch.bfloat16),
    (77, 2048, torch.bfloat16, torch.bfloat16),
    (64, 1536, torch.float16, torch.bfloat16),
    (9, 4, torch.bfloat16, torch.float16),
])
def test_residual_layer_norm_matches_torch(kern, device, rows, dim, branch_dtype, norm_dtype):
    print(f"[rows] residual+LN rows={rows} dim={dim} {branch_dtype} -> {norm_dtype}", flush=True)
    x, branch, gamma, w, b = _inputs(rows, dim, branch_dtype, rows * 7 + dim)
    s, n, n32 = kern.residual_layer_norm(x.to(device), branch.to(device), gamma.to(device),
                                         (w.to(device), b.to(device), 1e-5), norm_dtype=norm_dtype,
                                         norm_f32=True)
    ref_s = x + branch * gamma  # torch's fp32 mul then add (block.py:126)
    assert s.dtype == torch.float32 and torch.equal(s.cpu(), ref_s)
    ref64 = F.layer_norm(ref_s.double(), (dim,), w.double(), b.double(), 1e-5)
    assert_close(n32.cpu(), ref64, torch.float32, what="fp32 LayerNorm")
    _rounded_close(n, ref64, norm_dtype, "16-bit LayerNorm")


def test_residual_layer_norm_variants(kern, device):
    print("[rows] variants", flush=True)
    x, branch, gamma, w, b = _inputs(130, 1024, torch.bfloat16, 3)
    xd, bd = x.to(device), branch.to(device)
    # No gamma (Identity LayerScale), no affine LayerNorm.
    s, n, _ = kern.residual_layer_norm(xd, bd, None, (None, None, 1e-6), norm_dtype=torch.bfloat16)
    ref_s = x + branch.float()
    assert torch.equal(s.cpu(), ref_s)
    _rounded_close(n, F.layer_norm(ref_s.double(), (1024,), eps=1e-6), torch.bfloat16, "no-affine LayerNorm")
    # LayerNorm only (norm1 of a block): no branch, no sum written.
    s, n, n32 = kern.residual_layer_norm(xd, norm=(w.to(device), b.to(device), 1e-5), norm_f32=True)
    assert s is None
    assert_close(n32.cpu(), F.layer_norm(x.double(), (1024,), w.double(), b.double(), 1e-5),
                 torch.float32, what="LN-only fp32")
    _rounded_close(n, F.layer_norm(x.double(), (1024,), w.double(), b.double(), 1e-5), torch.bfloat16,
                   "LN-only bf16")
    # Residual only, written in place over x.
    lib_mod = import_package("_lib")
    lib = lib_mod.load()
    xi = xd.clone()
    status = lib.vgo_residual_layer_norm(
        xi.data_ptr(), 1024, bd.data_ptr(), 1024, lib_mod.VGO_BF16, gamma.to(device).data_ptr(),
        None, None, 0.0, 130, 1024, xi.data_ptr(), 1024, None, 0, lib_mod.VGO_BF16, None, 0,
        None, 0, 0.0, torch.cuda.current_stream().cuda_stream)
    lib_mod.check(status)
    assert torch.equal(xi.cpu(), x + branch * gamma)
    # Zero rows is a no-op; bad sizes and misaligned rows are rejected on the host.
    lib_mod.check(lib.vgo_residual_layer_norm(None, 0, None, 0, 0, None, None, None, 0.0, 0, 1024, None,
                                              0, None, 0, 1, None, 0, None, 0, 0.0, None))
    with pytest.raises(ValueError, match="multiple of 4"):
        kern.residual_layer_norm(xd[:, :1022].contiguous(), norm=(None, None, 1e-5))
    with pytest.raises(ValueError, match="aligned"):
        kern.residual_layer_norm(xd.view(-1)[1:1 + 129 * 1024].view(129, 1024), norm=(None, None, 1e-5))


def _block(vgo, device, seed, init_values=0.3):
    torch.manual_seed(seed)
    block = vgo.SelfAttentionBlock(256, 4, qkv_bias=True, init_values=init_values, mask_k_bias=True,
                                   use_qk_norm=True).eval().to(device)
    with torch.no_grad():
        for norm in (block.norm1, block.norm2):
            norm.weight.normal_(1.0, 0.2)
            norm.bias.normal_(0.0, 0.1)
    return block


def _reference_rows(block):
    """Switch the block to the reference op sequence for its residual rows."""
    block._fused_rows = lambda x: False


@pytest.mark.parametrize("init_values", [0.3, None])
def test_block_forward_fused_rows_match_reference(vgo, device, init_values):
    print(f"[rows] block forward init_values={init_values}", flush=True)
    layers = import_package("layers")
    block = _block(vgo, device, 5, init_values)
    x = structured_tokens(6, 3, (16, 16), 5, 256)[0].view(3, 261, 256).to(device)
    sin, cos = layers.rope_sincos(16, 16, 64, device=device)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        assert block._fused_rows(x)
        fused = block(x, rope=(sin, cos))
        _reference_rows(block)
        ref = block(x, rope=(sin, cos))
    assert fused.dtype == ref.dtype == torch.float32
    assert_close(fused.cpu(), ref.cpu(), torch.bfloat16, what="block forward")


def test_block_forward_compacted_fused_rows_match_reference(vgo, device):
    print("[rows] block forward_compacted", flush=True)
    block = _block(vgo, device, 7)
    x = structured_tokens(9, 4, (16, 16), 5, 256).to(device)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        normalized, attn_input = block.norm1_for_plan(x)
        assert normalized.dtype == torch.float32 and attn_input.dtype == torch.bfloat16
        assert_close(normalized.cpu(), block.norm1.float()(x).cpu(), torch.float32, what="norm1 fp32")
        plan = vgo.build_sparse_convex_plan(normalized, threshold=0.9, **KW)
        fused = block.forward_compacted(x, plan, normalized=attn_input)
        _reference_rows(block)
        ref = block.forward_compacted(x, plan, normalized=block.norm1(x))
    assert_close(fused.cpu(), ref.cpu(), torch.bfloat16, what="forward_compacted")


def _restore_inputs(n, m, dim, table_dtype, mode, seed):
    g = torch.Generator().manual_seed(seed)
    table = (torch.randn(m, dim, generator=g) * 1.5).to(table_dtype)
    index = torch.randint(0, m, (n, 4), generator=g, dtype=torch.int32)
    if mode == "one_hot":
        weight = torch.zeros(n, 4)
        weight[:, 0] = 1.0
    else:
        weight = torch.rand(n, 4, generator=g)
        weight[torch.rand(n, 4, generator=g) < 0.3] = 0.0      # skipped corners
        weight[::7] = 0.0                                      # rows with no parent at all
        weight = weight / weight.sum(1, keepdim=True).clamp_min(1e-6)
        index[3, 2], weight[3, 2] = m + 5, 0.25                # out of range, used: NaN row
        index[5, 1], weight[5, 1] = -2, 0.0                    # out of range, unused: ignored
    return table, index, weight


@pytest.mark.parametrize("n,m,dim,table_dtype,norm_dtype,mode", [
    (1029, 517, 1024, torch.bfloat16, torch.bfloat16, "one_hot"),
    (1029, 517, 1024, torch.bfloat16, torch.bfloat16, "four"),
    (333, 1000, 260, torch.float16, torch.float16, "four"),
    (77, 40, 2048, torch.float32, torch.bfloat16, "four"),
    (5, 3, 1536, torch.bfloat16, torch.float16, "one_hot"),
])
def test_restore_residual_layer_norm_equals_projection_then_rows(kern, device, n, m, dim, table_dtype,
                                                                  norm_dtype, mode):
    print(f"[rows] restore+residual+LN n={n} m={m} dim={dim} {table_dtype} {mode}", flush=True)
    proj = import_package("projection")
    table, index, weight = _restore_inputs(n, m, dim, table_dtype, mode, n + m + dim)
    x, _, gamma, w, b = _inputs(n, dim, torch.float32, n * 3 + dim)
    x, gamma, w, b = x.to(device), gamma.to(device), w.to(device), b.to(device)
    table, index, weight = table.to(device), index.to(device), weight.to(device)
    for g_, aff in ((gamma, (w, b, 1e-5)), (None, (None, None, 1e-6))):
        restored = proj.top4_project(table, index, weight)
        ref_s, ref_n, _ = kern.residual_layer_norm(x, restored, g_, aff, norm_dtype=norm_dtype)
        s, nrm = kern.restore_residual_layer_norm(x, table, index, weight, g_, aff, norm_dtype=norm_dtype)
        torch.testing.assert_close(s, ref_s, rtol=0, atol=0, equal_nan=True)
        torch.testing.assert_close(nrm, ref_n, rtol=0, atol=0, equal_nan=True)
    if mode == "four":
        assert torch.isnan(s[3]).all() and not torch.isnan(s[5]).any()


@pytest.mark.parametrize("table_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_restore_residual_layer_norm_one_hot_index_equals_map(kern, device, table_dtype):
    """weight None: index is a one-hot [rows] map (a token plan's inverse); equal bit for
    bit to the map rows (k x 4, (1, 0, 0, 0)), with zero rows for k < 0 and NaN rows for
    k past the table."""
    print(f"[rows] one-hot restore {table_dtype}", flush=True)
    n, m, dim = 333, 120, 1024
    g = torch.Generator().manual_seed(21)
    table = (torch.randn(m, dim, generator=g) * 2).to(table_dtype).to(device)
    inv = torch.randint(0, m, (n,), generator=g, dtype=torch.int32)
    inv[7], inv[8], inv[40] = -1, m, m + 1000
    x, _, gamma, w, b = _inputs(n, dim, torch.float32, 22)
    x, gamma, w, b = x.to(device), gamma.to(device), w.to(device), b.to(device)
    index4 = inv.view(-1, 1).expand(n, 4).contiguous().to(device)
    weight4 = torch.zeros(n, 4)
    weight4[:, 0] = (inv >= 0).float()
    weight4 = weight4.to(device)
    for g_, aff in ((gamma, (w, b, 1e-5)), (None, (None, None, 1e-6))):
        ref_s, ref_n = kern.restore_residual_layer_norm(x, table, index4, weight4, g_, aff)
        s, nrm = kern.restore_residual_layer_norm(x, table, inv.to(device), None, g_, aff)
        torch.testing.assert_close(s, ref_s, rtol=0, atol=0, equal_nan=True)
        torch.testing.assert_close(nrm, ref_n, rtol=0, atol=0, equal_nan=True)
    assert torch.isnan(s[8]).all() and torch.isnan(s[40]).all() and not torch.isnan(s[7]).any()
    assert torch.equal(s[7], x[7])  # a zero branch row


def test_restore_residual_layer_norm_rejects_bad_arguments(kern, device):
    print("[rows] restore+residual argument checks", flush=True)
    x = torch.zeros(8, 64, device=device)
    table = torch.zeros(4, 64, device=device, dtype=torch.bfloat16)
    index = torch.zeros(8, 4, device=device, dtype=torch.int32)
    weight = torch.zeros(8, 4, device=device)
    with pytest.raises(ValueError):
        kern.restore_residual_layer_norm(x, table, index[:7], weight[:7], None, (None, None, 1e-5))
    with pytest.raises(ValueError):
        kern.restore_residual_layer_norm(x, table[:, :32], index, weight, None, (None, None, 1e-5))
    with pytest.raises(ValueError):
        kern.restore_residual_layer_norm(x, table, index.long(), weight, None, (None, None, 1e-5))
    with pytest.raises(ValueError):  # a one-hot map is [rows]
        kern.restore_residual_layer_norm(x, table, index, None, None, (None, None, 1e-5))
    with pytest.raises(ValueError):
        kern.restore_residual_layer_norm(x, table, index[:, 0].long(), None, None, (None, None, 1e-5))


@pytest.mark.parametrize("planner", ["fastvggt", "sparse_convex"])
def test_block_forward_compacted_fused_restore_equals_unfused(vgo, device, planner):
    """forward_compacted restores inside the first row pass; the result equals the plan's
    restore followed by the plain fused rows, bit for bit."""
    print(f"[rows] forward_compacted fused restore ({planner})", flush=True)
    block = _block(vgo, device, 17)
    x = structured_tokens(18, 4, (16, 16), 5, 256).to(device)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        normalized, attn_input = block.norm1_for_plan(x)
        if planner == "fastvggt":
            plan = vgo.build_fastvggt_plan(normalized, merge_ratio=0.5, protect_ratio=0.0,
                                           mass_bias=True, **KW)
        else:
            plan = vgo.build_sparse_convex_plan(normalized, threshold=0.9, **KW)
        y = block.attn._forward_merged(attn_input, None, None, plan)
        assert plan.restore_map_for(y) is not None
        unfused = block._fused_tail(x, plan.restore(y))
        fused = block.forward_compacted(x, plan, normalized=attn_input)
    assert torch.equal(fused, unfused)


def test_tuned_gemm_table_loads_and_matches_default(vgo, device):
    print("[rows] tuned GEMM table", flush=True)
    tuning = import_package("gemm_tuning")
    g = torch.Generator(device=device).manual_seed(4)
    x = torch.randn(32928, 1024, device=device, generator=g)
    lin = torch.nn.Linear(1024, 3072, device=device)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        default = lin(x)
        try:
            assert tuning.use_tuned_gemms()
            assert torch.cuda.tunable.is_enabled()
            tuned = lin(x)
        finally:
            tuning.default_gemms()
    assert tuned.dtype == torch.bfloat16
    assert_close(tuned.float().cpu(), default.float().cpu(), torch.bfloat16, what="tuned GEMM")


def test_aggregator_register_rows_in_place_match_concatenation(device):
    """A register block writes its special rows into the frame block's output when no
    cached layer keeps that tensor; the result equals the concatenating path."""
    print("[rows] aggregator register rows in place", flush=True)
    agg = import_package("aggregator")
    torch.manual_seed(0)
    model = agg.Aggregator(embed_dim=256, depth=3, num_heads=4, num_register_tokens=4,
                           register_attention_block_indices=(1,),
                           cached_layer_indices=(2,)).to(device).eval()
    patches = structured_tokens(2, 4, (16, 16), 5, 256)[0].view(4, 261, 256)[:, 5:].contiguous()
    model.set_input_patch_tokens_cache(patches.to(device))
    images = torch.zeros(1, 4, 3, 256, 256, device=device)
    model.set_fastvggt(True, merge_ratio=0.5, protect_ratio=0.0, mass_bias=True)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        in_place = model(images)[0][2]
        model.cached_layer_indices = {0, 1, 2}  # every frame output kept: concatenation
        concatenated = model(images)[0][2]
    assert torch.equal(in_place, concatenated)


@pytest.mark.parametrize("rows,dim", [(1029, 1024), (37, 256), (65, 1028)])
def test_unit_rows_equal_normalize_rows_of_the_fp32_norm(kern, device, rows, dim):
    """The fused pass's F.normalize output equals normalize_rows over its own fp32
    LayerNorm rows bit for bit (same values, same reduction order)."""
    print(f"[rows] unit rows rows={rows} dim={dim}", flush=True)
    x, _, _, w, b = _inputs(rows, dim, torch.bfloat16, rows + dim)
    _, n, n32, unit = kern.residual_layer_norm(x.to(device), norm=(w.to(device), b.to(device), 1e-5),
                                               norm_f32=True, unit_eps=1e-12)
    assert unit.dtype == torch.bfloat16 and n.dtype == torch.bfloat16
    assert torch.equal(unit, kern.normalize_rows(n32, None, 1e-12))
    ref = F.normalize(F.layer_norm(x.double(), (dim,), w.double(), b.double(), 1e-5), dim=-1)
    _rounded_close(unit, ref, torch.bfloat16, "unit rows")


def test_fastvggt_plan_from_fused_unit_rows_is_identical(vgo, device):
    """norm1_unit_rows + build_fastvggt_plan(prenormalized=True) gives the plan
    build_fastvggt_plan(norm1_for_plan fp32 rows) gives, bit for bit."""
    print("[rows] FastVGGT plan from unit rows", flush=True)
    block = _block(vgo, device, 11)
    x = structured_tokens(12, 4, (16, 16), 5, 256).to(device)
    kw = dict(KW, merge_ratio=0.5, protect_ratio=0.0, mass_bias=True)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        unit, attn_input = block.norm1_unit_rows(x)
        normalized, attn_input2 = block.norm1_for_plan(x)
    assert torch.equal(attn_input, attn_input2)
    fused = vgo.build_fastvggt_plan(unit, prenormalized=True, **kw)
    plain = vgo.build_fastvggt_plan(normalized, **kw)
    assert torch.equal(fused.keep, plain.keep) and torch.equal(fused.inverse, plain.inverse)
    assert torch.equal(fused.key_log_mass, plain.key_log_mass)
    with pytest.raises(ValueError, match="bf16 unit rows"):
        vgo.build_fastvggt_plan(normalized, prenormalized=True, **kw)


def test_block_forward_fp16_autocast_fused_rows(vgo, device):
    """fp16 autocast: the rows are cast to fp16, the matcher's unit rows stay with
    the reference path (they are bf16 by definition), and the block matches the
    reference op sequence."""
    print("[rows] block forward fp16 autocast", flush=True)
    layers = import_package("layers")
    block = _block(vgo, device, 13)
    x = structured_tokens(14, 3, (16, 16), 5, 256)[0].view(3, 261, 256).to(device)
    sin, cos = layers.rope_sincos(16, 16, 64, device=device)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
        assert block._fused_rows(x) and block.norm1_unit_rows(x) is None
        assert block.norm1_for_plan(x)[1].dtype == torch.float16
        fused = block(x, rope=(sin, cos))
        _reference_rows(block)
        ref = block(x, rope=(sin, cos))
    assert_close(fused.cpu(), ref.cpu(), torch.float16, what="fp16 block forward")
