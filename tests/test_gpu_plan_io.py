"""Plan files, TTT trace replay and plan reuse / replay in the aggregator, on the GPU.

* A trace record of the reference's own sparse-convex plan (C1 fixture) is
  rebuilt on the GPU exactly as the CPU oracle rebuilds it (keep, sources,
  parents, fp16 weights, special ids and the deterministic mass bit for bit).
* A plan built here and written as a trace file comes back with the same
  structure and its weights rounded to fp16, as the trace format stores them.
* Plan files round-trip every field bit for bit, and the merged layer gives
  bit-identical output with the loaded plan.
* The aggregator reuses one plan across a forward (reference
  aggregator.py:980-1006) and replays given plans, bit-identically.
"""
from __future__ import annotations

import dataclasses
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import plan_io as opi
from tests._tol import rel_error
from tests.conftest import import_package
from tests.golden.inputs import structured_tokens

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).parent / "golden"
LAYOUT = dict(tokens_per_frame=261, patch_token_start=5)
KW = dict(frames=4, patch_hw=(16, 16), **LAYOUT)


@pytest.fixture(scope="module")
def pio():
    return import_package("plan_io")


@pytest.fixture(scope="module")
def fx():
    return np.load(GOLDEN / "fixtures_c1.npz")


def _fixture_record(fx):
    return opi.ttt_record_from_plan(torch.from_numpy(fx["sc_keep"]), torch.from_numpy(fx["sc_source"]),
                                    torch.from_numpy(fx["sc_parent"]), torch.from_numpy(fx["sc_weight"]),
                                    frames=4, **LAYOUT)


def test_trace_record_of_reference_plan_matches_oracle(pio, fx, device):
    print("[plan_io] fixture record", flush=True)
    record = _fixture_record(fx)
    plan = pio.plan_from_ttt_record(record, device=device, **LAYOUT)
    ref = opi.plan_from_ttt_record(record, **LAYOUT)
    assert torch.equal(plan.keep.cpu(), ref["keep"])
    assert torch.equal(plan.source_original.cpu(), ref["source_original"])
    assert torch.equal(plan.source_parent_compact.cpu(), ref["parent_compact"])
    assert torch.equal(plan.source_pool_weights.cpu(), ref["weights"])
    assert torch.equal(plan.source_restore_weights.cpu(), ref["weights"])
    assert torch.equal(plan.special_query_compact.cpu(), ref["special_compact"])
    assert torch.equal(plan.special_query_original.cpu(), ref["special"])
    assert torch.equal(plan.normalizer.cpu(), ref["mass"])
    assert rel_error(plan.key_log_mass.cpu().reshape(-1), ref["log_mass"].reshape(-1)) < 1e-6
    assert plan.dense_special_queries and plan.original_tokens == 1044


def test_built_plan_round_trips_through_a_trace_file(vgo, pio, device, tmp_path):
    print("[plan_io] trace round trip", flush=True)
    tokens = structured_tokens(9, 4, (16, 16), 5, 256).to(device)
    plans = [vgo.build_sparse_convex_plan(tokens, threshold=t, **KW) for t in (0.9, 0.8)]
    records = [pio.ttt_record_from_plan(p, frames=4, layer=i, **LAYOUT) for i, p in enumerate(plans)]
    pio.save_ttt_trace(records, tmp_path / "trace.pt")
    back = pio.load_ttt_trace(tmp_path / "trace.pt", device=device, **LAYOUT)
    assert len(back) == 2
    for plan, again, record in zip(plans, back, records):
        assert torch.equal(again.keep, plan.keep)
        assert torch.equal(again.source_original, plan.source_original)
        assert torch.equal(again.source_parent_compact, plan.source_parent_compact)
        assert torch.equal(again.source_pool_weights, plan.source_pool_weights.half().float())
        assert torch.equal(again.special_query_compact, plan.special_query_compact)
        ref = opi.plan_from_ttt_record(record, **LAYOUT)
        assert torch.equal(again.normalizer.cpu(), ref["mass"])


def _layer_output(vgo, plan, device):
    layer = vgo.SelfAttention(256, num_heads=4, qkv_bias=True, mask_k_bias=True,
                              use_qk_norm=True).eval().to(device)
    torch.manual_seed(3)
    for p in layer.parameters():
        torch.nn.init.normal_(p, std=0.05)
    x = structured_tokens(5, 4, (16, 16), 5, 256).to(device)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        return layer(x, token_plan=plan)


@pytest.mark.parametrize("kind", ["fastvggt", "sparse_convex"])
def test_plan_files_round_trip_bit_exact(vgo, pio, device, tmp_path, kind):
    print(f"[plan_io] plan file {kind}", flush=True)
    tokens = structured_tokens(11, 4, (16, 16), 5, 256).to(device)
    if kind == "fastvggt":
        plan = vgo.build_fastvggt_plan(tokens, merge_ratio=0.5, protect_ratio=0.0, mass_bias=True, **KW)
    else:
        plan = vgo.build_sparse_convex_plan(tokens, threshold=0.9, **KW)
    path = tmp_path / f"{kind}.safetensors"
    pio.save_plan(plan, path)
    again = pio.load_plan(path, device=device)
    assert type(again) is type(plan)

    for f in dataclasses.fields(plan):
        if not f.init:
            continue
        a, b = getattr(plan, f.name), getattr(again, f.name)
        if f.name in ("precomputed_qkv", "source_attention_output"):
            assert b is None
        elif isinstance(a, torch.Tensor):
            assert isinstance(b, torch.Tensor) and a.dtype == b.dtype and torch.equal(a, b), f.name
        elif f.name == "metadata":
            assert json.loads(json.dumps(a)) == b
        else:
            assert a == b, f.name
    assert torch.equal(_layer_output(vgo, plan, device), _layer_output(vgo, again, device))


def test_load_plan_rejects_other_files(pio, tmp_path):
    from safetensors.torch import save_file
    save_file({"x": torch.zeros(3)}, str(tmp_path / "plain.safetensors"))
    with pytest.raises(ValueError, match="not a merge-plan file"):
        pio.load_plan(tmp_path / "plain.safetensors")
    header = {"format": "vgo-merge-plan", "version": 99, "kind": "TokenPlan"}
    save_file({"keep": torch.zeros(1, 2, dtype=torch.int64)}, str(tmp_path / "v99.safetensors"),
              metadata={"vgo_plan": json.dumps(header)})
    with pytest.raises(ValueError, match="version 99"):
        pio.load_plan(tmp_path / "v99.safetensors")


def test_aggregator_reuses_and_replays_plans(pio, device, tmp_path):
    print("[plan_io] aggregator reuse / replay", flush=True)
    agg = import_package("aggregator")
    torch.manual_seed(0)
    model = agg.Aggregator(embed_dim=256, depth=3, num_heads=4, num_register_tokens=4,
                           register_attention_block_indices=(1,),
                           cached_layer_indices=(2,)).to(device).eval()
    patches = structured_tokens(2, 4, (16, 16), 5, 256)[0].view(4, 261, 256)[:, 5:].contiguous()
    model.set_input_patch_tokens_cache(patches.to(device))
    images = torch.zeros(1, 4, 3, 256, 256, device=device)

    def run():
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            return model(images)[0][2]

    model.set_sparse_convex(True, threshold=0.9, qkv_global_blocks=1, qkv_global_layers=(0,), reuse_plan=True)
    reused = run()
    stats = model.sparse_convex_last_plan_stats
    assert [s["reused_plan"] for s in stats] == [False, True]
    assert stats[0]["kept_tokens"] == stats[1]["kept_tokens"]
    assert [s["compact_queries"] for s in stats] == [True, False]
    plan = model._sparse_convex_reuse_plan
    pio.save_plan(plan, tmp_path / "p.safetensors")
    loaded = pio.load_plan(tmp_path / "p.safetensors", device=device)
    # The same plan replayed: once with reuse, once per layer without.
    model.set_sparse_convex_plans([loaded])
    assert torch.equal(run(), reused)
    model.set_sparse_convex(True, threshold=0.9, qkv_global_blocks=1, qkv_global_layers=(0,), reuse_plan=False)
    model.set_sparse_convex_plans([loaded, loaded])
    assert torch.equal(run(), reused)
    assert [s["reused_plan"] for s in model.sparse_convex_last_plan_stats] == [False, False]
    model.set_sparse_convex_plans([loaded])
    with pytest.raises(RuntimeError, match="ran out"):
        run()
    # A TTT trace of the plan replays with its fp16 weights.
    pio.save_ttt_trace([pio.ttt_record_from_plan(plan, frames=4, **LAYOUT)], tmp_path / "t.pt")
    model.set_sparse_convex(True, threshold=0.9, qkv_global_blocks=1, qkv_global_layers=(0,), reuse_plan=True)
    model.set_sparse_convex_plans(pio.load_ttt_trace(tmp_path / "t.pt", device=device, **LAYOUT))
    replayed = run()
    assert rel_error(replayed.float(), reused.float()) < 2e-2
    # Refit: the cached plan is rebuilt (here: the next replayed plan) at ordinal 1.
    model.set_sparse_convex(True, threshold=0.9, qkv_global_blocks=1, qkv_global_layers=(0,), reuse_plan=True,
                            refit_ordinal=1)
    model.set_sparse_convex_plans([loaded, loaded])
    assert torch.equal(run(), reused)
    assert [s["refit_plan"] for s in model.sparse_convex_last_plan_stats] == [False, True]
    model.set_sparse_convex_plans(None)
