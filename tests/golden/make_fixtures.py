"""Write golden fixtures from the real reference (run once, in the build container).

The reference has no tests or stored vectors, and its planners' thresholded
and tie-dependent decisions (build_fastvggt_plan, build_sparse_convex_plan)
can only be pinned by running them.  This script imports the reference's
modules straight from their files under /root/reference (without executing the
package __init__, which would pull in the whole model), runs them on CPU on
the seeded inputs of tests/golden/inputs.py, and stores inputs' sha256 and all
outputs in tests/golden/fixtures_c1.npz plus a JSON manifest.  Only data is
stored; nothing of the reference is copied.  The GPU box never runs this.

A second file, tests/golden/fixtures_agg.npz (+ .json), holds a reduced
reference Aggregator run (S=4 frames of 16x16 patches + 5 special tokens, dim
128, 2 heads, depth 3 with one register block, so two merged global blocks),
fp32 on CPU, from the patch-token cache, with seeded weights
(tests/golden/inputs.py `aggregator_state`) loaded into the reference model:
the cached outputs, every plan the global blocks built and the plan stats,
for the FastVGGT arm and the sparse-convex arm (with and without a dense
bypass layer).  The reference Aggregator module is loaded by registering
`vggt_omega` and `vggt_omega.models` as bare package shells, so the package
__init__ (the whole VGGT-Omega model) never runs.

A third file, tests/golden/fixtures_c1w.npz (+ .json), holds the C1 merged layer at its
stated width (dim 1024, 16 heads): see `wide_layer_fixture`.

A fourth file, tests/golden/fixtures_enc.npz (+ .json), holds the reference's DINOv3 patch
encoder at reduced width: see `encoder_fixture`.

Usage:  PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_fixtures.py [c1|agg|c1w|enc|all]
"""
from __future__ import annotations

import importlib.util
import json
import sys
import types
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from tests.golden.inputs import (  # noqa: E402
    aggregator_state,
    attention_weights,
    encoder_state,
    seeded_values,
    sha256,
    structured_tokens,
)

REFERENCE_MODELS = Path("/root/reference/vggt_omega/models")
PKG = "_reference_models"

# C1 layout: 4 frames x (5 special + 16x16 patches) = 1044 tokens.
FRAMES, HW, SPECIALS = 4, (16, 16), 5
TPF = SPECIALS + HW[0] * HW[1]


def load_reference():
    sys.dont_write_bytecode = True
    pkg = types.ModuleType(PKG)
    pkg.__path__ = [str(REFERENCE_MODELS)]
    sys.modules[PKG] = pkg
    layers = types.ModuleType(PKG + ".layers")
    layers.__path__ = [str(REFERENCE_MODELS / "layers")]
    sys.modules[PKG + ".layers"] = layers

    def load(name: str, path: Path):
        spec = importlib.util.spec_from_file_location(f"{PKG}.{name}", path)
        module = importlib.util.module_from_spec(spec)
        sys.modules[spec.name] = module
        spec.loader.exec_module(module)
        return module

    tm = load("token_merging", REFERENCE_MODELS / "token_merging.py")
    load("sparse_convex_kernels", REFERENCE_MODELS / "sparse_convex_kernels.py")
    sc = load("sparse_convex", REFERENCE_MODELS / "sparse_convex.py")
    load("layers.utils", REFERENCE_MODELS / "layers" / "utils.py")
    attn = load("layers.attention", REFERENCE_MODELS / "layers" / "attention.py")
    return tm, sc, attn


class _RecordBf16Products:
    """Records the bf16 outputs of torch.bmm / Tensor.__matmul__ while active.

    The planners rank the bf16 products they compute (token_merging.py:1106-1111,
    sparse_convex.py:2402-2404, 2430); recording them keeps the reference's own
    score matrices, so tests can measure how often a score sits within one bf16
    ulp of a competitor (the tie band) instead of assuming it never does."""

    def __init__(self):
        self.products: list[torch.Tensor] = []

    def __enter__(self):
        self._bmm, self._matmul = torch.bmm, torch.Tensor.__matmul__
        record = self.products

        def bmm(a, b, *args, **kwargs):
            out = self._bmm(a, b, *args, **kwargs)
            if out.dtype == torch.bfloat16:
                record.append(out.detach().clone())
            return out

        def matmul(a, b):
            out = self._matmul(a, b)
            if out.dtype == torch.bfloat16:
                record.append(out.detach().clone())
            return out

        torch.bmm, torch.Tensor.__matmul__ = bmm, matmul
        return self

    def __exit__(self, *exc):
        torch.bmm, torch.Tensor.__matmul__ = self._bmm, self._matmul
        return False


def main() -> None:
    tm, sc, attn = load_reference()
    out: dict[str, np.ndarray] = {}
    manifest: dict[str, object] = {"layout": dict(frames=FRAMES, patch_hw=HW, specials=SPECIALS)}

    tokens = structured_tokens(1, FRAMES, HW, SPECIALS, 1024)
    manifest["tokens_sha256"] = sha256(tokens)
    kw = dict(frames=FRAMES, tokens_per_frame=TPF, patch_token_start=SPECIALS, patch_hw=HW)

    with torch.no_grad():
        # FastVGGT bipartite plans: the BASELINE ratio-0.5 case and the reference defaults.
        for tag, ratio, protect in (("fv50", 0.5, 0.0), ("fvdef", 0.9, 0.10)):
            with _RecordBf16Products() as rec:
                plan = tm.build_fastvggt_plan(tokens, merge_ratio=ratio, protect_ratio=protect, **kw)
            out[f"{tag}_keep"] = plan.keep[0].numpy()
            out[f"{tag}_inverse"] = plan.inverse[0].numpy()
            # the reference's bf16 score matrix [sources, destinations] (one chunk at C1)
            out[f"{tag}_scores"] = torch.cat([p[0] for p in rec.products]).view(torch.int16).numpy()

        # Sparse-convex fixed-topology plan.
        with _RecordBf16Products() as rec:
            plan = sc.build_sparse_convex_plan(tokens, threshold=0.90, **kw)
        # local-group scores [576 candidates, 448 dictionary] and the global fallback's
        out["sc_local_scores"] = rec.products[0].view(torch.int16).numpy()
        out["sc_fallback_scores"] = torch.cat(rec.products[1:]).view(torch.int16).numpy()
        out["sc_keep"] = plan.keep[0].numpy()
        out["sc_source"] = plan.source_original[0].numpy()
        out["sc_parent"] = plan.source_parent_compact[0].numpy()
        out["sc_weight"] = plan.source_pool_weights[0].numpy()
        out["sc_mass"] = plan.normalizer[0, :, 0].numpy()
        out["sc_log_mass"] = plan.key_log_mass[0].numpy()
        out["sc_special_compact"] = plan.special_query_compact.numpy()
        manifest["sc_metadata"] = {k: v for k, v in plan.metadata.items()}

        # Compaction / restore of seeded values on both plan types.
        fv = tm.build_fastvggt_plan(tokens, merge_ratio=0.5, protect_ratio=0.0, **kw)
        for dtype, dtag in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
            value = seeded_values(7, (1, tokens.shape[1], 32), dtype)
            out[f"sc_compact_{dtag}"] = plan.compact(value).float().numpy()[0]
            out[f"fv_compact_{dtag}"] = fv.compact(value).float().numpy()[0]
            small = seeded_values(8, (1, plan.kept_tokens, 32), dtype)
            out[f"sc_restore_{dtag}"] = plan.restore(small).float().numpy()[0]
            small_fv = seeded_values(8, (1, fv.kept_tokens, 32), dtype)
            out[f"fv_restore_{dtag}"] = fv.restore(small_fv).float().numpy()[0]

        # One merged global-attention layer (dim 128, 2 heads of 64), CPU fp32.
        x = structured_tokens(3, FRAMES, HW, SPECIALS, 128)
        manifest["attn_x_sha256"] = sha256(x)
        layer = attn.SelfAttention(128, num_heads=2, qkv_bias=True, mask_k_bias=True,
                                   use_qk_norm=True).eval()
        layer.load_state_dict(attention_weights(4, 128))
        for tag, preserve in (("attn_qkv", False), ("attn_kv", True)):
            p = sc.build_sparse_convex_plan(x, threshold=0.90, preserve_queries=preserve, **kw)
            out[f"{tag}_keep"] = p.keep[0].numpy()
            out[f"{tag}_source"] = p.source_original[0].numpy()
            out[f"{tag}_parent"] = p.source_parent_compact[0].numpy()
            out[f"{tag}_weight"] = p.source_pool_weights[0].numpy()
            out[f"{tag}_mass"] = p.normalizer[0, :, 0].numpy()
            out[f"{tag}_special_compact"] = p.special_query_compact.numpy()
            out[f"{tag}_out"] = layer(x, token_plan=p)[0].numpy()

    np.savez_compressed(HERE / "fixtures_c1.npz", **out)
    manifest["arrays"] = {k: [list(v.shape), str(v.dtype)] for k, v in out.items()}
    (HERE / "fixtures_c1.json").write_text(json.dumps(manifest, indent=1, default=str) + "\n")
    print(f"wrote {len(out)} arrays")


# Reduced aggregator: S=4 frames x (5 specials + 16x16 patches), dim 128, 2 heads of 64,
# depth 3 with a register block at index 1 -> merged global blocks at 0 and 2.
AGG = dict(embed_dim=128, depth=3, num_heads=2, num_register_tokens=4,
           register_attention_block_indices=[1], cached_layer_indices=(0, 2))
AGG_WEIGHT_SEED = 17
AGG_PATCH_SEED = 18


def load_reference_aggregator():
    """vggt_omega.models.aggregator without running the package __init__ files."""
    sys.dont_write_bytecode = True
    root = REFERENCE_MODELS.parent
    for name, path in (("vggt_omega", root), ("vggt_omega.models", REFERENCE_MODELS)):
        if name not in sys.modules:
            shell = types.ModuleType(name)
            shell.__path__ = [str(path)]
            sys.modules[name] = shell
    import importlib
    return importlib.import_module("vggt_omega.models.aggregator")


def aggregator_inputs(dim: int):
    """Patch-token cache [frames, 256, dim] (the patches of structured tokens)."""
    tokens = structured_tokens(AGG_PATCH_SEED, FRAMES, HW, SPECIALS, dim)[0]
    return tokens.view(FRAMES, TPF, dim)[:, SPECIALS:].contiguous()


def aggregator_fixture() -> None:
    agg_mod = load_reference_aggregator()
    torch.manual_seed(0)
    model = agg_mod.Aggregator(**AGG).eval()
    names = [(k, tuple(v.shape)) for k, v in model.state_dict().items()
             if k.startswith(("frame_blocks.", "inter_frame_blocks.", "camera_token", "register_token"))]
    state = aggregator_state(AGG_WEIGHT_SEED, names, AGG["embed_dim"])
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert not unexpected and all(not m.startswith(("frame_blocks", "inter_frame_blocks")) for m in missing)
    patches = aggregator_inputs(AGG["embed_dim"])
    images = torch.zeros(1, FRAMES, 3, HW[0] * 16, HW[1] * 16)
    model.set_input_patch_tokens_cache(patches)

    # Record every plan the global blocks build (the builders are module globals).
    built = []
    originals = (agg_mod.build_fastvggt_plan, agg_mod.build_sparse_convex_plan)

    def recording(builder):
        def wrapped(*args, **kwargs):
            with _RecordBf16Products() as rec:
                plan = builder(*args, **kwargs)
            built.append((plan, rec.products))
            return plan
        return wrapped

    agg_mod.build_fastvggt_plan = recording(originals[0])
    agg_mod.build_sparse_convex_plan = recording(originals[1])
    out: dict[str, np.ndarray] = {}
    manifest: dict[str, object] = {
        "config": dict(AGG, frames=FRAMES, patch_hw=HW, weight_seed=AGG_WEIGHT_SEED,
                       patch_seed=AGG_PATCH_SEED),
        "patches_sha256": sha256(patches),
        "state_sha256": sha256(torch.cat([state[k].flatten() for k in sorted(state)])),
        "state_keys": [[k, list(shape)] for k, shape in names],
    }
    runs = {
        "fv": lambda: model.set_fastvggt(True, merge_ratio=0.5, protect_ratio=0.0),
        "sc": lambda: model.set_sparse_convex(True, threshold=0.9, qkv_global_layers=(0,),
                                              qkv_global_blocks=1),
        "scd": lambda: model.set_sparse_convex(True, threshold=0.9, qkv_global_layers=(0,),
                                               qkv_global_blocks=1, dense_global_layers=(1,)),
    }
    try:
        for tag, configure in runs.items():
            model.set_fastvggt(False)
            model.set_sparse_convex(False, qkv_global_blocks=0, qkv_global_layers=())
            configure()
            built.clear()
            with torch.no_grad():
                outputs, start = model(images)
            assert start == SPECIALS
            # the last cached output (frame and global tokens of block 2) depends on every block
            last = max(AGG["cached_layer_indices"])
            out[f"{tag}_out{last}"] = outputs[last].numpy()
            stats = model.fastvggt_last_plan_stats if tag == "fv" else model.sparse_convex_last_plan_stats
            manifest[f"{tag}_stats"] = stats
            for i, (plan, products) in enumerate(built):
                out[f"{tag}_plan{i}_keep"] = plan.keep[0].numpy()
                if tag == "fv":
                    out[f"{tag}_plan{i}_inverse"] = plan.inverse[0].numpy()
                else:
                    if tag == "sc":
                        # The planner's bf16 scores, so tests can tell a top-4 tie from a
                        # different support choice.  At this layout the single local group's
                        # dictionary is the global one, and every global-fallback row equals
                        # its candidate's local row, so the local matrix covers both.
                        local = products[0]
                        rows = {bytes(r.view(torch.int16).numpy()) for r in local}
                        assert all(bytes(r.view(torch.int16).numpy()) in rows for r in torch.cat(products[1:]))
                        out[f"{tag}_plan{i}_local_scores"] = local.view(torch.int16).numpy()
                    out[f"{tag}_plan{i}_source"] = plan.source_original[0].numpy()
                    out[f"{tag}_plan{i}_parent"] = plan.source_parent_compact[0].numpy()
                    out[f"{tag}_plan{i}_weight"] = plan.source_pool_weights[0].numpy()
                    out[f"{tag}_plan{i}_mass"] = plan.normalizer[0, :, 0].numpy()
                    out[f"{tag}_plan{i}_special_compact"] = plan.special_query_compact.numpy()
            manifest[f"{tag}_plans"] = len(built)
    finally:
        agg_mod.build_fastvggt_plan, agg_mod.build_sparse_convex_plan = originals
    np.savez_compressed(HERE / "fixtures_agg.npz", **out)
    manifest["arrays"] = {k: [list(v.shape), str(v.dtype)] for k, v in out.items()}
    (HERE / "fixtures_agg.json").write_text(json.dumps(manifest, indent=1, default=str) + "\n")
    print(f"wrote {len(out)} aggregator arrays")


WIDE_DIM, WIDE_HEADS = 1024, 16


def wide_layer_fixture() -> None:
    """BASELINE configs[0] at its stated width: one merged global-attention layer, dim 1024,
    16 heads of 64, on the C1 tokens (structured_tokens seed 1, the tokens the C1 plans of
    fixtures_c1.npz were built from), CPU fp32, weights attention_weights(4, 1024).

    Two arms, each the reference's own SelfAttention.forward with a plan its planners build
    from the same tokens (so the plans are the ones fixtures_c1.npz already holds):
    * fv  -- FastVGGT ratio 0.5 / protect 0 with integer cluster masses as the key bias:
             the reference's TokenPlan given key_log_mass = log(bincount(inverse)), which
             compute_attention reads by getattr (layers/attention.py:384-388) and, on CPU,
             applies through SDPA with the float mask (:400);
    * sc  -- the sparse-convex plan (threshold 0.9, Q/K/V compacted, dense special
             queries), whose key_log_mass is log(normalizer).
    Stores the two [1044, 1024] outputs in tests/golden/fixtures_c1w.npz (+ .json)."""
    tm, sc, attn = load_reference()
    kw = dict(frames=FRAMES, tokens_per_frame=TPF, patch_token_start=SPECIALS, patch_hw=HW)
    c1 = np.load(HERE / "fixtures_c1.npz")
    tokens = structured_tokens(1, FRAMES, HW, SPECIALS, WIDE_DIM)
    manifest: dict[str, object] = {
        "layout": dict(frames=FRAMES, patch_hw=HW, specials=SPECIALS),
        "dim": WIDE_DIM, "heads": WIDE_HEADS, "weight_seed": 4, "tokens_seed": 1,
        "tokens_sha256": sha256(tokens),
    }
    out: dict[str, np.ndarray] = {}
    layer = attn.SelfAttention(WIDE_DIM, num_heads=WIDE_HEADS, qkv_bias=True, mask_k_bias=True,
                               use_qk_norm=True).eval()
    layer.load_state_dict(attention_weights(4, WIDE_DIM))
    with torch.no_grad():
        fv = tm.build_fastvggt_plan(tokens, merge_ratio=0.5, protect_ratio=0.0, **kw)
        assert np.array_equal(fv.keep[0].numpy(), c1["fv50_keep"])
        assert np.array_equal(fv.inverse[0].numpy(), c1["fv50_inverse"])
        counts = torch.bincount(fv.inverse[0], minlength=fv.kept_tokens).float()
        fv.key_log_mass = counts.log().view(1, -1)
        manifest["fv_mass_max"] = float(counts.max())
        out["fv_out"] = layer(tokens, token_plan=fv)[0].numpy()
        plan = sc.build_sparse_convex_plan(tokens, threshold=0.90, **kw)
        for name in ("keep", "source_original", "source_parent_compact", "source_pool_weights"):
            key = {"keep": "sc_keep", "source_original": "sc_source",
                   "source_parent_compact": "sc_parent", "source_pool_weights": "sc_weight"}[name]
            assert np.array_equal(getattr(plan, name)[0].numpy(), c1[key]), name
        assert plan.dense_special_queries
        out["sc_out"] = layer(tokens, token_plan=plan)[0].numpy()
    np.savez_compressed(HERE / "fixtures_c1w.npz", **out)
    manifest["arrays"] = {k: [list(v.shape), str(v.dtype)] for k, v in out.items()}
    manifest["arrays_sha256"] = {k: sha256(torch.from_numpy(v)) for k, v in out.items()}
    (HERE / "fixtures_c1w.json").write_text(json.dumps(manifest, indent=1, default=str) + "\n")
    print(f"wrote {len(out)} wide-layer arrays")


# A reduced DINOv3 patch encoder: the arguments of aggregator.py:1296-1320 at dim 128,
# 2 heads, depth 2, on two 64x64 images (4x4 patches after the 16x16 projection).
ENC = dict(embed_dim=128, depth=2, num_heads=2)
ENC_IMAGES = (2, 3, 64, 64)
ENC_WEIGHT_SEED, ENC_IMAGE_SEED = 23, 24


def encoder_fixture() -> None:
    """forward_features of the reference DinoVisionTransformer built as the aggregator's
    _build_patch_embed builds it (reduced width), fp32 on CPU, seeded parameters
    (tests/golden/inputs.py `encoder_state`), on seeded already-normalised images."""
    load_reference_aggregator()
    import importlib
    vit = importlib.import_module("vggt_omega.models.layers.vision_transformer")
    torch.manual_seed(0)
    model = vit.DinoVisionTransformer(
        img_size=224, patch_size=16, in_chans=3, pos_embed_rope_base=100,
        pos_embed_rope_normalize_coords="max", pos_embed_rope_dtype="fp32", ffn_ratio=4,
        qkv_bias=True, drop_path_rate=0.0, layerscale_init=1.0e-5, norm_layer="layernormbf16",
        ffn_layer="mlp", ffn_bias=True, proj_bias=True, n_storage_tokens=4, mask_k_bias=True, **ENC)
    model.init_weights()
    model.eval()
    # every parameter and the qkv bias masks; the RoPE periods keep their init
    names = [(k, tuple(v.shape)) for k, v in model.state_dict().items() if not k.startswith("rope_embed.")]
    state = encoder_state(ENC_WEIGHT_SEED, names)
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert not unexpected and all(m.startswith("rope_embed.") for m in missing), missing
    images = seeded_values(ENC_IMAGE_SEED, ENC_IMAGES)
    with torch.no_grad():
        feats = model.forward_features(images)
    out = {k: feats[k].numpy() for k in ("x_norm_clstoken", "x_storage_tokens", "x_norm_patchtokens")}
    manifest = {
        "config": dict(ENC, images=list(ENC_IMAGES), weight_seed=ENC_WEIGHT_SEED, image_seed=ENC_IMAGE_SEED,
                       patch_size=16, n_storage_tokens=4, rope_base=100, normalize_coords="max"),
        "images_sha256": sha256(images),
        "state_sha256": sha256(torch.cat([state[k].flatten() for k in sorted(state)])),
        "state_keys": [[k, list(shape)] for k, shape in names],
        "arrays": {k: [list(v.shape), str(v.dtype)] for k, v in out.items()},
        "arrays_sha256": {k: sha256(torch.from_numpy(v)) for k, v in out.items()},
    }
    np.savez_compressed(HERE / "fixtures_enc.npz", **out)
    (HERE / "fixtures_enc.json").write_text(json.dumps(manifest, indent=1, default=str) + "\n")
    print(f"wrote {len(out)} encoder arrays")


if __name__ == "__main__":
    which = sys.argv[1] if len(sys.argv) > 1 else "all"
    if which in ("c1", "all"):
        main()
    if which in ("agg", "all"):
        aggregator_fixture()
    if which in ("c1w", "all"):
        wide_layer_fixture()
    if which in ("enc", "all"):
        encoder_fixture()
