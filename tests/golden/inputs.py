"""Seeded synthetic inputs shared by the fixture script and the tests.

`structured_tokens` builds a VGGT-Omega token layout [1, frames * (specials +
H*W), dim] whose later frames are shifted, noisy copies of a latent scene, so
merge planners find real matches, near-ties, hard cases and rejects:
  frame f, patch (r, c) = scene[(r + f) % H, (c + 2f) % W] + sigma * noise,
with sigma drawn per patch from {0.05, 0.3, 0.6, 1.5}; special tokens ~ N(0,1).
Everything comes from torch's CPU generator, so every machine regenerates the
same bits (the fixture manifest records a sha256 of each input).
"""
from __future__ import annotations

import hashlib

import torch

NOISE_LEVELS = torch.tensor([0.05, 0.3, 0.6, 1.5])


def structured_tokens(seed: int, frames: int, patch_hw: tuple[int, int], specials: int,
                      dim: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    height, width = patch_hw
    scene = torch.randn(height, width, dim, generator=g)
    out = []
    for f in range(frames):
        rows = (torch.arange(height) + f) % height
        cols = (torch.arange(width) + 2 * f) % width
        patches = scene[rows][:, cols].reshape(height * width, dim)
        sigma = NOISE_LEVELS[torch.randint(0, 4, (height * width,), generator=g)]
        patches = patches + sigma[:, None] * torch.randn(height * width, dim, generator=g)
        special = torch.randn(specials, dim, generator=g)
        out.append(torch.cat((special, patches)))
    return torch.cat(out)[None]


def seeded_values(seed: int, shape: tuple[int, ...], dtype=torch.float32) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def attention_weights(seed: int, dim: int) -> dict[str, torch.Tensor]:
    """State dict of SelfAttention(dim, qkv_bias=True, mask_k_bias=True, use_qk_norm=True).

    Non-trivial values everywhere (biases, LayerNorm affine) so that a dropped
    term shows up in the output.
    """
    g = torch.Generator().manual_seed(seed)
    head = 64

    def r(*shape, s=0.02):
        return torch.randn(*shape, generator=g) * s

    bias_mask = torch.ones(3 * dim)
    bias_mask[dim:2 * dim] = 0
    return {
        "qkv.weight": r(3 * dim, dim, s=dim ** -0.5),
        "qkv.bias": r(3 * dim, s=0.1),
        "qkv.bias_mask": bias_mask,
        "proj.weight": r(dim, dim, s=dim ** -0.5),
        "proj.bias": r(dim, s=0.1),
        "q_norm.weight": 1.0 + r(head, s=0.1),
        "q_norm.bias": r(head, s=0.1),
        "k_norm.weight": 1.0 + r(head, s=0.1),
        "k_norm.bias": r(head, s=0.1),
    }


def aggregator_state(seed: int, keys_and_shapes: list[tuple[str, tuple[int, ...]]],
                     dim: int) -> dict[str, torch.Tensor]:
    """Seeded values for the aggregator's block parameters and camera/register tokens.

    `keys_and_shapes` lists state-dict entries (names as in the reference's
    Aggregator: frame_blocks.i.*, inter_frame_blocks.i.*, camera_token,
    register_token); the values depend only on the seed and each entry's name
    and shape, so the reference model and this build load identical weights.
    LayerScale gammas are large (0.2-0.6, not the 1e-5 init) so that every
    block moves the residual stream and a dropped term shows in the output.
    """
    out = {}
    for key, shape in sorted(keys_and_shapes):
        g = torch.Generator().manual_seed(seed * 1_000_003 + int(hashlib.sha256(key.encode()).hexdigest()[:8], 16))
        leaf = key.rsplit(".", 1)[-1]
        if leaf == "bias_mask":
            value = torch.ones(shape)
            value[shape[0] // 3:2 * shape[0] // 3] = 0
        elif leaf == "gamma":
            value = 0.2 + 0.4 * torch.rand(shape, generator=g)
        elif key in ("camera_token", "register_token"):
            value = torch.randn(shape, generator=g)
        elif "norm" in key and leaf == "weight":
            value = 1.0 + 0.1 * torch.randn(shape, generator=g)
        elif leaf == "bias":
            value = 0.05 * torch.randn(shape, generator=g)
        elif leaf == "weight":
            value = torch.randn(shape, generator=g) * shape[-1] ** -0.5
        else:
            raise KeyError(f"aggregator_state: no rule for {key}")
        out[key] = value
    return out


def encoder_state(seed: int, keys_and_shapes: list[tuple[str, tuple[int, ...]]]) -> dict[str, torch.Tensor]:
    """Seeded values for the patch encoder's parameters (names as in the reference's
    DinoVisionTransformer: patch_embed.proj.*, cls_token, storage_tokens, mask_token,
    blocks.i.*, norm.*).  Block entries follow `aggregator_state`; the class and
    storage tokens are N(0,1), the mask token zero (the reference adds 0 times it to
    the class token), and the patch projection is scaled by its fan-in."""
    out, blocks = {}, []
    for key, shape in sorted(keys_and_shapes):
        g = torch.Generator().manual_seed(seed * 1_000_003 + int(hashlib.sha256(key.encode()).hexdigest()[:8], 16))
        if key in ("cls_token", "storage_tokens"):
            out[key] = torch.randn(shape, generator=g)
        elif key == "mask_token":
            out[key] = torch.zeros(shape)
        elif key == "patch_embed.proj.weight":
            fan_in = shape[1] * shape[2] * shape[3]
            out[key] = torch.randn(shape, generator=g) * fan_in ** -0.5
        else:
            blocks.append((key, shape))
    out.update(aggregator_state(seed, blocks, 0))
    return out


def sha256(tensor: torch.Tensor) -> str:
    return hashlib.sha256(tensor.detach().cpu().contiguous().numpy().tobytes()).hexdigest()
