"""The aggregator's DINOv3 patch encoder (4d_ttt_merging_amd/patch_encoder.py) against the
reference.

tests/golden/fixtures_enc.npz holds `DinoVisionTransformer.forward_features` of the
reference encoder built with the arguments of vggt_omega/models/aggregator.py:1296-1320
at reduced width (dim 128, 2 heads, depth 2), fp32 on the CPU, seeded parameters
(tests/golden/inputs.py `encoder_state`), on two seeded 64x64 images: the class token,
the 4 storage tokens and the 16 normalised patch rows of each image.

Checks: the parameter names and shapes equal the reference's (CPU); fp32 outputs within
1e-5 and bf16 autocast outputs within 2e-2 of the reference's (GPU); and an aggregator
built with the encoder runs it on the normalised images, giving the same outputs bit for
bit as the same aggregator fed the encoder's patch rows as its patch-token cache (GPU).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from tests._tol import assert_close
from tests.conftest import import_package
from tests.golden.inputs import encoder_state, seeded_values, sha256

GOLDEN = Path(__file__).parent / "golden"
OUTPUTS = ("x_norm_clstoken", "x_storage_tokens", "x_norm_patchtokens")


@pytest.fixture(scope="module")
def manifest():
    return json.loads((GOLDEN / "fixtures_enc.json").read_text())


@pytest.fixture(scope="module")
def efx():
    return np.load(GOLDEN / "fixtures_enc.npz")


def _ours(name: str) -> str:
    """This build's parameter name of the reference's `name`."""
    return name[len("patch_embed."):] if name.startswith("patch_embed.") else name


def _encoder(manifest, device=None):
    pe = import_package("patch_encoder")
    cfg = manifest["config"]
    enc = pe.PatchEncoder(patch_size=cfg["patch_size"], embed_dim=cfg["embed_dim"], depth=cfg["depth"],
                          num_heads=cfg["num_heads"], n_storage_tokens=cfg["n_storage_tokens"]).eval()
    state = encoder_state(cfg["weight_seed"], [(k, tuple(s)) for k, s in manifest["state_keys"]])
    enc.load_state_dict({_ours(k): v for k, v in state.items()})
    images = seeded_values(cfg["image_seed"], tuple(cfg["images"]))
    return (enc if device is None else enc.to(device)), images


# ------------------------------------------------------------------ CPU ----
def test_encoder_state_keys_match_reference(manifest):
    """Every reference parameter (less the `patch_embed.` prefix) is this build's, same shape,
    and the seeded state and images are the fixture's bits."""
    enc, images = _encoder(manifest)
    ours = {k: list(v.shape) for k, v in enc.state_dict().items()}
    assert ours == {_ours(k): s for k, s in manifest["state_keys"]}
    cfg = manifest["config"]
    state = encoder_state(cfg["weight_seed"], [(k, tuple(s)) for k, s in manifest["state_keys"]])
    assert sha256(torch.cat([state[k].flatten() for k in sorted(state)])) == manifest["state_sha256"]
    assert sha256(images) == manifest["images_sha256"]


# ------------------------------------------------------------------ GPU ----
@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_encoder_vs_reference(manifest, efx, device, dtype):
    print(f"[patch encoder] dtype={dtype}", flush=True)
    enc, images = _encoder(manifest, device)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=dtype != torch.float32):
        out = enc(images.to(device))
    torch.cuda.synchronize()
    for name in OUTPUTS:
        ref = torch.from_numpy(efx[name])
        err = assert_close(out[name].float().cpu(), ref, dtype, what=f"encoder {name}")
        print(f"[patch encoder] {name} relative error {err:.3e}", flush=True)


@pytest.mark.gpu
def test_aggregator_runs_its_encoder(manifest, device):
    """Aggregator(patch_encoder=...) without a cache equals the same aggregator fed the
    encoder's patch rows (of the mean/std-normalised images) as cached patch tokens."""
    print("[patch encoder] aggregator", flush=True)
    agg = import_package("aggregator")
    enc, _ = _encoder(manifest)
    cfg = manifest["config"]
    torch.manual_seed(3)
    model = agg.Aggregator(embed_dim=cfg["embed_dim"], depth=2, num_heads=cfg["num_heads"], num_register_tokens=4,
                           register_attention_block_indices=(1,), cached_layer_indices=(0, 1),
                           patch_encoder=enc).to(device).eval()
    model.set_fastvggt(True, merge_ratio=0.5, protect_ratio=0.0)
    g = torch.Generator().manual_seed(5)
    images = torch.rand(1, 3, 3, 64, 64, generator=g).to(device)
    mean = torch.tensor([0.485, 0.456, 0.406], device=device).view(1, 1, 3, 1, 1)
    std = torch.tensor([0.229, 0.224, 0.225], device=device).view(1, 1, 3, 1, 1)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        outputs, start = model(images)
        patches = enc(((images - mean) / std).view(3, 3, 64, 64))["x_norm_patchtokens"]
        model.set_input_patch_tokens_cache(patches.float())
        cached, _ = model(images)
    torch.cuda.synchronize()
    assert start == 5 and patches.shape == (3, 16, cfg["embed_dim"])
    for a, b in zip(outputs, cached):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(a, b)
