"""BASELINE configs[0] at its stated width: one merged global-attention layer, dim 1024,
16 heads of 64, S=4 frames x (5 specials + 16x16 patches) = 1,044 tokens.

tests/golden/fixtures_c1w.npz holds the reference's own SelfAttention.forward
(vggt_omega/models/layers/attention.py:264-439) on the C1 tokens with two plans the
reference's planners built from those tokens (the plans of fixtures_c1.npz):

* fv -- FastVGGT ratio 0.5 / protect 0 (token_merging.py:1044-1122), integer
        cluster masses as the log-mass key bias: the C1 configuration itself;
* sc -- the sparse-convex plan (sparse_convex.py:2343-2481), Q/K/V compacted,
        dense special queries, log(normalizer) key bias.

CPU: the oracle layer against the fixture (fp32, 1e-5).  GPU: this build's
SelfAttention (qkv GEMM, fused LayerNorm64 compaction, mass-bias attention kernel,
output projection, restore) against the fixture in fp32 (1e-5) and against the
oracle's bf16-autocast semantics under bf16 autocast (2e-2); the measured margins
are printed.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import layer as oracle_layer
from tests._tol import assert_close, rel_error
from tests.golden.inputs import attention_weights, sha256, structured_tokens

GOLDEN = Path(__file__).parent / "golden"
FRAMES, HW, SPECIALS, DIM, HEADS = 4, (16, 16), 5, 1024, 16
TPF = SPECIALS + HW[0] * HW[1]


@pytest.fixture(scope="module")
def wide():
    return np.load(GOLDEN / "fixtures_c1w.npz")


@pytest.fixture(scope="module")
def c1():
    return np.load(GOLDEN / "fixtures_c1.npz")


@pytest.fixture(scope="module")
def tokens():
    x = structured_tokens(1, FRAMES, HW, SPECIALS, DIM)
    manifest = json.loads((GOLDEN / "fixtures_c1w.json").read_text())
    assert sha256(x) == manifest["tokens_sha256"]
    return x


def _oracle_plan(c1, tag: str) -> dict:
    if tag == "fv":
        return {"inverse": torch.from_numpy(c1["fv50_inverse"])}
    return dict(keep=torch.from_numpy(c1["sc_keep"]), source_original=torch.from_numpy(c1["sc_source"]),
                parent_compact=torch.from_numpy(c1["sc_parent"]), weights=torch.from_numpy(c1["sc_weight"]),
                mass=torch.from_numpy(c1["sc_mass"]),
                special_original=(torch.arange(FRAMES)[:, None] * TPF + torch.arange(SPECIALS)[None]).flatten(),
                special_compact=torch.from_numpy(c1["sc_special_compact"]))


@pytest.mark.parametrize("tag", ["fv", "sc"])
def test_oracle_wide_layer_matches_reference(wide, c1, tokens, tag):
    out = oracle_layer.self_attention(tokens[0], attention_weights(4, DIM), HEADS, _oracle_plan(c1, tag), False)
    err = rel_error(out, torch.from_numpy(wide[f"{tag}_out"]))
    print(f"[c1 wide] oracle {tag} fp32 rel err {err:.2e}")
    assert err < 1e-5


def test_oracle_wide_layer_checks_have_teeth(wide, c1, tokens):
    """A dropped mass bias or a transposed restore corner order fails the comparison."""
    state = attention_weights(4, DIM)
    # every token its own cluster: no merging, mass 1, no bias
    unmerged = oracle_layer.self_attention(tokens[0], state, HEADS,
                                           {"inverse": torch.arange(FRAMES * TPF)}, False)
    assert rel_error(unmerged, torch.from_numpy(wide["fv_out"])) > 1e-2
    sc = _oracle_plan(c1, "sc")
    sc_bad = dict(sc, parent_compact=sc["parent_compact"].flip(1))
    bad = oracle_layer.self_attention(tokens[0], state, HEADS, sc_bad, False)
    assert rel_error(bad, torch.from_numpy(wide["sc_out"])) > 1e-3


def _plan(vgo, c1, tag: str, device):
    t = lambda name: torch.from_numpy(c1[name]).to(device)  # noqa: E731
    if tag == "fv":
        inverse = t("fv50_inverse")
        counts = torch.bincount(inverse, minlength=int(c1["fv50_keep"].size)).float()
        return vgo.TokenPlan(keep=t("fv50_keep")[None], inverse=inverse[None], original_tokens=FRAMES * TPF,
                             key_log_mass=counts.log().view(1, -1))
    special = (torch.arange(FRAMES)[:, None] * TPF + torch.arange(SPECIALS)[None]).flatten().to(device)
    w = t("sc_weight")
    mass = t("sc_mass")
    return vgo.WeightedBilinearTokenPlan(
        keep=t("sc_keep")[None], source_original=t("sc_source")[None], source_parent_compact=t("sc_parent")[None],
        source_pool_weights=w[None], source_restore_weights=w[None], original_tokens=FRAMES * TPF,
        normalizer=mass.view(1, -1, 1), dense_special_queries=True, special_query_original=special,
        special_query_compact=t("sc_special_compact"), key_log_mass=mass.log().view(1, -1))


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["fv", "sc"])
def test_wide_layer_vs_reference(vgo, device, wide, c1, tokens, tag):
    print(f"[c1 wide] layer {tag}: dim 1024, 16 heads, 1,044 tokens", flush=True)
    layer = vgo.SelfAttention(DIM, num_heads=HEADS, qkv_bias=True, mask_k_bias=True,
                              use_qk_norm=True).eval().to(device)
    layer.load_state_dict(attention_weights(4, DIM))
    plan = _plan(vgo, c1, tag, device)
    x = tokens.to(device)
    with torch.no_grad():
        out = layer(x, token_plan=plan)
    err32 = assert_close(out[0].cpu(), torch.from_numpy(wide[f"{tag}_out"]), torch.float32,
                         what=f"C1 wide {tag} fp32 layer")
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        out16 = layer(x, token_plan=plan)
    assert out16.dtype == torch.bfloat16
    ref16 = oracle_layer.self_attention(tokens[0], attention_weights(4, DIM), HEADS, _oracle_plan(c1, tag),
                                        False, autocast_bf16=True)
    err16 = assert_close(out16[0].float().cpu(), ref16.float(), torch.bfloat16,
                         what=f"C1 wide {tag} bf16 layer")
    print(f"[c1 wide] layer {tag}: fp32 rel err {err32:.2e} (bar 1e-5), bf16 autocast rel err "
          f"{err16:.2e} (bar 2e-2)", flush=True)
