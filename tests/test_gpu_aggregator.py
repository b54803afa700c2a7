"""Aggregator-level parity: this build's Aggregator against a reference run.

tests/golden/fixtures_agg.npz holds a reduced reference Aggregator forward
(vggt_omega/models/aggregator.py:721-808, global arm :841-1022, 1215-1216):
S=4 frames of 16x16 patches + 5 special tokens, dim 128, 2 heads of 64,
depth 3 with a register block at index 1 (merged global blocks at 0 and 2),
fp32 on the CPU, seeded weights from tests/golden/inputs.py
`aggregator_state` loaded into both models.  Three arms:

* fv  -- FastVGGT at ratio 0.5, protect 0 (two plans);
* sc  -- sparse-convex, threshold 0.9, global ordinal 0 compacts Q/K/V and
         ordinal 1 is KV-only (preserve_queries / preserve_destination_keys);
* scd -- as sc with ordinal 1 a dense bypass layer (dense_global_layers).

Checks: the plans this build's planners make at every global block against
the reference's (bit-exact indices; sparse-convex weights to the convex-fit
tolerance), the plan-stats lists (schema and values), and the last cached
output -- fp32 within 1e-5 where the plans are the reference's own bits, and
bf16 autocast within 2e-2 of the reference's fp32 output.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from tests._tol import assert_close, rel_error
from tests.conftest import import_package
from tests.golden.inputs import aggregator_state, structured_tokens

GOLDEN = Path(__file__).parent / "golden"
FRAMES, HW, SPECIALS = 4, (16, 16), 5
TPF = SPECIALS + HW[0] * HW[1]


@pytest.fixture(scope="module")
def afx():
    return np.load(GOLDEN / "fixtures_agg.npz")


@pytest.fixture(scope="module")
def manifest():
    return json.loads((GOLDEN / "fixtures_agg.json").read_text())


def _model(manifest, device):
    agg = import_package("aggregator")
    cfg = manifest["config"]
    model = agg.Aggregator(embed_dim=cfg["embed_dim"], depth=cfg["depth"], num_heads=cfg["num_heads"],
                           num_register_tokens=cfg["num_register_tokens"],
                           register_attention_block_indices=tuple(cfg["register_attention_block_indices"]),
                           cached_layer_indices=tuple(cfg["cached_layer_indices"])).eval()
    keys = [(k, tuple(s)) for k, s in manifest["state_keys"]]
    model.load_state_dict(aggregator_state(cfg["weight_seed"], keys, cfg["embed_dim"]))
    model = model.to(device)
    dim = cfg["embed_dim"]
    tokens = structured_tokens(cfg["patch_seed"], FRAMES, HW, SPECIALS, dim)[0]
    patches = tokens.view(FRAMES, TPF, dim)[:, SPECIALS:].contiguous()
    model.set_input_patch_tokens_cache(patches.to(device))
    images = torch.zeros(1, FRAMES, 3, HW[0] * 16, HW[1] * 16, device=device)
    return model, images


def _configure(model, tag: str) -> None:
    model.set_fastvggt(False)
    model.set_sparse_convex(False, qkv_global_blocks=0, qkv_global_layers=())
    if tag == "fv":
        model.set_fastvggt(True, merge_ratio=0.5, protect_ratio=0.0)
    else:
        model.set_sparse_convex(True, threshold=0.9, qkv_global_layers=(0,), qkv_global_blocks=1,
                                dense_global_layers=(1,) if tag == "scd" else ())


class _Recorder:
    """Records the plans the aggregator's planners return during one forward (built at
    once, or started and then waited for)."""

    def __init__(self, monkeypatch):
        self.plans = []
        self.inputs = []
        agg = import_package("aggregator")
        recorder = self

        class Pending:
            def __init__(self, pending, tokens):
                self.pending, self.tokens = pending, tokens

            def result(self):
                plan = self.pending.result()
                recorder.plans.append(plan)
                recorder.inputs.append(self.tokens)
                return plan

        for name in ("build_fastvggt_plan", "build_sparse_convex_plan", "start_sparse_convex_plan"):
            builder = getattr(agg, name)

            def wrapped(*args, _builder=builder, _name=name, **kwargs):
                out = _builder(*args, **kwargs)
                if _name.startswith("start_"):
                    return Pending(out, args[0])
                self.plans.append(out)
                self.inputs.append(args[0])
                return out

            monkeypatch.setattr(agg, name, wrapped)


def _reference_plan(vgo, afx, tag: str, i: int, device):
    """The reference's i-th plan of an arm as this build's WeightedBilinearTokenPlan."""
    t = lambda name: torch.from_numpy(afx[f"{tag}_plan{i}_{name}"]).to(device)  # noqa: E731
    mass = t("mass")
    special = (torch.arange(FRAMES)[:, None] * TPF + torch.arange(SPECIALS)[None]).flatten().to(device)
    w = t("weight")
    return vgo.WeightedBilinearTokenPlan(
        keep=t("keep")[None], source_original=t("source")[None], source_parent_compact=t("parent")[None],
        source_pool_weights=w[None], source_restore_weights=w[None], original_tokens=FRAMES * TPF,
        normalizer=mass.view(1, -1, 1), dense_special_queries=True, special_query_original=special,
        special_query_compact=t("special_compact"), key_log_mass=mass.log().view(1, -1))


def _ulp_bf16(x: np.ndarray) -> np.ndarray:
    return np.ldexp(1.0, np.frexp(np.maximum(np.abs(x), 1e-30))[1] - 8)


def _check_support_ties(afx, i: int, plan, differs: np.ndarray, first_differs: np.ndarray) -> None:
    """Rows whose top-4 support set, or first support, differs from the reference's
    differ inside a tie.

    With the reference's own bf16 scores S of the row (recorded from its matmul,
    sparse_convex.py:2402-2404, 2430) and t = the lowest score among its four
    supports, every support in one set but not the other scores within one bf16
    ulp of t; and two different first supports score within one ulp of each
    other.  Both choices are then equally valid up to the tie order (this build:
    lower dictionary position first, the Triton contract of
    sparse_convex_kernels.py:51-54; the reference's CPU torch.topk: another
    order) and the one-ulp rounding of the scores.  The first support matters
    beyond the set: the one-hot fit (sparse_convex.py:2300-2304) takes it."""
    if not (differs.any() or first_differs.any()):
        return
    from oracle import merging as om
    scores = afx[f"sc_plan{i}_local_scores"].view(np.uint16).astype(np.uint32) << 16
    scores = scores.view(np.float32)
    lay = om.sparse_convex_layout(FRAMES * TPF, FRAMES, TPF, SPECIALS, HW)
    row_of = {int(c): r for r, c in enumerate(lay["candidate"])}
    pos_of = {int(d): j for j, d in enumerate(lay["destination"])}
    keep = plan.keep[0].cpu().numpy()
    sources = plan.source_original[0].cpu().numpy()
    ours = keep[plan.source_parent_compact[0].cpu().numpy()]
    ref = keep[afx[f"sc_plan{i}_parent"]]
    for s in np.nonzero(differs)[0]:
        row = scores[row_of[int(sources[s])]]
        a, b = set(ours[s].tolist()), set(ref[s].tolist())
        t = min(row[pos_of[p]] for p in b)
        for p in a ^ b:
            assert abs(row[pos_of[p]] - t) <= 1.01 * _ulp_bf16(t), \
                f"source {sources[s]}: support {p} is not tied with the reference's top-4"
    for s in np.nonzero(first_differs)[0]:
        row = scores[row_of[int(sources[s])]]
        a, b = row[pos_of[int(ours[s, 0])]], row[pos_of[int(ref[s, 0])]]
        assert abs(a - b) <= 1.01 * _ulp_bf16(max(a, b)), \
            f"source {sources[s]}: first supports {ours[s, 0]} / {ref[s, 0]} are not tied"


def _fit_cosine(normalized, plan, parent, weight) -> torch.Tensor:
    """cos(source, sum_c w_c support_c) of every merged source, as `_convex_fit` scores
    it (sparse_convex.py:2297-2303), on the planner's fp32 input rows, in float64."""
    import torch.nn.functional as F
    x = F.normalize(normalized[0].double().cpu(), dim=-1, eps=1e-6)
    keep = plan.keep[0].cpu()
    src = F.normalize(x[plan.source_original[0].cpu()], dim=-1, eps=1e-6)
    sup = F.normalize(x[keep[parent.cpu()]], dim=-1, eps=1e-6)
    recon = (weight.cpu().double()[..., None] * sup).sum(1)
    return (recon * src).sum(-1) / recon.norm(dim=-1).clamp_min(1e-12)


def _compare_stats(ours: list[dict], ref: list[dict]) -> None:
    assert len(ours) == len(ref)
    for a, b in zip(ours, ref):
        assert set(a) == set(b), f"stats keys differ: {set(a) ^ set(b)}"
        for key, value in b.items():
            if isinstance(value, float) and key == "fit_mean":
                assert abs(a[key] - value) < 1e-4, key
            elif isinstance(value, float):
                assert abs(a[key] - value) < 1e-12, key
            else:
                assert a[key] == value, (key, a[key], value)


# ------------------------------------------------------------------ CPU ----
def test_aggregator_state_keys_match_reference(manifest):
    """The reference's block / token parameter names and shapes are this build's."""
    agg = import_package("aggregator")
    cfg = manifest["config"]
    model = agg.Aggregator(embed_dim=cfg["embed_dim"], depth=cfg["depth"], num_heads=cfg["num_heads"],
                           num_register_tokens=cfg["num_register_tokens"],
                           register_attention_block_indices=tuple(cfg["register_attention_block_indices"]))
    ours = {k: list(v.shape) for k, v in model.state_dict().items()}
    assert ours == {k: s for k, s in manifest["state_keys"]}
    state = aggregator_state(cfg["weight_seed"], [(k, tuple(s)) for k, s in manifest["state_keys"]],
                             cfg["embed_dim"])
    from tests.golden.inputs import sha256
    assert sha256(torch.cat([state[k].flatten() for k in sorted(state)])) == manifest["state_sha256"]


# ------------------------------------------------------------------ GPU ----
@pytest.mark.gpu
def test_aggregator_fastvggt_vs_reference_fp32(manifest, afx, device, monkeypatch):
    print("[aggregator] fastvggt fp32", flush=True)
    model, images = _model(manifest, device)
    _configure(model, "fv")
    rec = _Recorder(monkeypatch)
    with torch.no_grad():
        outputs, start = model(images)
    assert start == SPECIALS
    assert len(rec.plans) == manifest["fv_plans"] == 2
    for i, plan in enumerate(rec.plans):
        assert np.array_equal(plan.keep[0].cpu().numpy(), afx[f"fv_plan{i}_keep"]), f"plan {i} keep"
        assert np.array_equal(plan.inverse[0].cpu().numpy(), afx[f"fv_plan{i}_inverse"]), f"plan {i} inverse"
    _compare_stats(model.fastvggt_last_plan_stats, manifest["fv_stats"])
    err = assert_close(outputs[2].cpu(), torch.from_numpy(afx["fv_out2"]), torch.float32,
                       what="FastVGGT aggregator fp32")
    print(f"[aggregator] fastvggt fp32 rel err {err:.2e}", flush=True)


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["sc", "scd"])
def test_aggregator_sparse_convex_plans_and_stats(manifest, afx, device, monkeypatch, tag):
    """Live sparse-convex planning at both global ordinals: the reference's keep and
    source sets, weights within the convex-fit tolerance, the same stats list (incl.
    the dense bypass entry); the output within the error those weights allow."""
    print(f"[aggregator] sparse-convex live {tag}", flush=True)
    model, images = _model(manifest, device)
    _configure(model, tag)
    rec = _Recorder(monkeypatch)
    with torch.no_grad():
        outputs, _ = model(images)
    assert len(rec.plans) == manifest[f"{tag}_plans"]
    for i, plan in enumerate(rec.plans):
        assert np.array_equal(plan.keep[0].cpu().numpy(), afx[f"{tag}_plan{i}_keep"])
        assert np.array_equal(plan.source_original[0].cpu().numpy(), afx[f"{tag}_plan{i}_source"])
        assert np.array_equal(plan.special_query_compact.cpu().numpy(), afx[f"{tag}_plan{i}_special_compact"])
        # corners compared by parent id: exact bf16 ties in the top-4 go to the lower
        # dictionary position here and to torch.topk's order in the reference
        par, ref_par = plan.source_parent_compact[0].cpu().numpy(), afx[f"{tag}_plan{i}_parent"]
        order, ref_order = np.argsort(par, axis=1, kind="stable"), np.argsort(ref_par, axis=1, kind="stable")
        same = (np.take_along_axis(par, order, 1) == np.take_along_axis(ref_par, ref_order, 1)).all(1)
        same_first = par[:, 0] == ref_par[:, 0]
        _check_support_ties(afx, i, plan, ~same, ~same_first)
        # Where the supports agree, the simplex least-squares optimum (well conditioned
        # even where the weights are not: near-collinear supports) is the same fit.
        fit = _fit_cosine(rec.inputs[i], plan, plan.source_parent_compact[0], plan.source_pool_weights[0])
        ref_fit = _fit_cosine(rec.inputs[i], plan, torch.from_numpy(afx[f"{tag}_plan{i}_parent"]),
                              torch.from_numpy(afx[f"{tag}_plan{i}_weight"]))
        agree = torch.from_numpy(same & same_first)
        assert (fit - ref_fit)[agree].abs().max() < 1e-4
        w = np.take_along_axis(plan.source_pool_weights[0].cpu().numpy(), order, 1)
        ref_w = np.take_along_axis(afx[f"{tag}_plan{i}_weight"], ref_order, 1)
        close = (np.abs(w - ref_w) < 2e-3).all(1)
        print(f"[aggregator] {tag} plan {i}: of {same.size} sources {int((~same).sum())} pick another "
              f"top-4 set and {int((~same_first).sum())} another first support, all inside score ties; "
              f"the rest fit within {float((fit - ref_fit)[agree].abs().max()):.1e}, weights within 2e-3 on "
              f"{close[agree.numpy()].mean():.3f} of them", flush=True)
    _compare_stats(model.sparse_convex_last_plan_stats, manifest[f"{tag}_stats"])
    # A source restored from another, tied parent differs by that row's distance, so
    # the elementwise bound belongs to the replay test below; here the whole output
    # must agree in relative norm.
    out, ref = outputs[2].double().cpu(), torch.from_numpy(afx[f"{tag}_out2"]).double()
    norm_err = float((out - ref).norm() / ref.norm())
    print(f"[aggregator] sparse-convex live {tag}: relative norm error {norm_err:.2e}, "
          f"elementwise {rel_error(out, ref):.2e}", flush=True)
    assert norm_err < 5e-3


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["sc", "scd"])
@pytest.mark.parametrize("autocast", [False, True])
def test_aggregator_sparse_convex_replayed_plans(vgo, manifest, afx, device, tag, autocast):
    """The reference's own plans replayed: fp32 within 1e-5, bf16 autocast within 2e-2."""
    print(f"[aggregator] sparse-convex replay {tag} autocast={autocast}", flush=True)
    model, images = _model(manifest, device)
    _configure(model, tag)
    model.set_sparse_convex_plans([_reference_plan(vgo, afx, tag, i, device)
                                   for i in range(manifest[f"{tag}_plans"])])
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        outputs, _ = model(images)
    out = outputs[2].float().cpu()
    dtype = torch.bfloat16 if autocast else torch.float32
    err = assert_close(out, torch.from_numpy(afx[f"{tag}_out2"]), dtype,
                       what=f"sparse-convex aggregator {tag} {'bf16' if autocast else 'fp32'}")
    print(f"[aggregator] sparse-convex replay {tag} autocast={autocast} rel err {err:.2e}", flush=True)
    stats = model.sparse_convex_last_plan_stats
    assert [s["kept_tokens"] for s in stats] == [s["kept_tokens"] for s in manifest[f"{tag}_stats"]]


@pytest.mark.gpu
def test_aggregator_fastvggt_forward_replays_from_a_hip_graph(manifest, device):
    """The FastVGGT forward (bf16 autocast, mass bias) has no host synchronisation, so it
    captures into one HIP graph; three replays, with eager forwards between them, each give
    the eager output bit for bit."""
    print("[aggregator] FastVGGT forward in a HIP graph", flush=True)
    model, images = _model(manifest, device)
    _configure(model, "fv")
    model.set_fastvggt(True, merge_ratio=0.5, protect_ratio=0.0, mass_bias=True)

    def step():
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
            return [o for o in model(images)[0] if o is not None]

    eager = [o.clone() for o in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(static, eager))
        step()
        torch.cuda.synchronize()


@pytest.mark.gpu
def test_aggregator_side_stream_qkv_matches_in_block_projection(manifest, device, monkeypatch):
    """FastVGGT blocks project qkv on a side stream once the matcher is enqueued
    (`build_fastvggt_plan(after_match=...)`); the outputs equal, bit for bit, those of
    the same forward with the projection made inside the block."""
    print("[aggregator] side-stream qkv projection", flush=True)
    agg = import_package("aggregator")
    model, images = _model(manifest, device)
    _configure(model, "fv")
    model.set_fastvggt(True, merge_ratio=0.5, protect_ratio=0.0, mass_bias=True)

    def step():
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            return [o for o in model(images)[0] if o is not None]

    side = step()
    assert model.__dict__.get("_qkv_streams"), "the side stream was not used"
    monkeypatch.setattr(agg.Aggregator, "_side_qkv", lambda self, block, x: None)
    inline = step()
    torch.cuda.synchronize()
    assert len(side) == len(inline) > 0
    assert all(torch.equal(a, b) for a, b in zip(side, inline))
