"""Write golden fixtures from the real reference (run once, in the build container).

The reference has no tests or stored vectors, and its planners' thresholded
and tie-dependent decisions (build_fastvggt_plan, build_sparse_convex_plan)
can only be pinned by running them.  This script imports the reference's
modules straight from their files under /root/reference (without executing the
package __init__, which would pull in the whole model), runs them on CPU on
the seeded inputs of tests/golden/inputs.py, and stores inputs' sha256 and all
outputs in tests/golden/fixtures_c1.npz plus a JSON manifest.  Only data is
stored; nothing of the reference is copied.  The GPU box never runs this.

Usage:  PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_fixtures.py
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
from tests.golden.inputs import attention_weights, seeded_values, sha256, structured_tokens  # noqa: E402

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
            plan = tm.build_fastvggt_plan(tokens, merge_ratio=ratio, protect_ratio=protect, **kw)
            out[f"{tag}_keep"] = plan.keep[0].numpy()
            out[f"{tag}_inverse"] = plan.inverse[0].numpy()

        # Sparse-convex fixed-topology plan.
        plan = sc.build_sparse_convex_plan(tokens, threshold=0.90, **kw)
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


if __name__ == "__main__":
    main()
