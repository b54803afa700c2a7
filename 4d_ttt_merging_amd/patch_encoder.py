"""The aggregator's DINOv3 ViT-L/16 patch encoder (`Aggregator.patch_embed`).

Structure of vggt_omega/models/aggregator.py:1296-1320 (`_build_patch_embed`)
and of the inference path of `DinoVisionTransformer.forward_features`
(vggt_omega/models/layers/vision_transformer.py:66-110, 196-270):

* a 16x16, stride-16 convolution of the normalised image to `embed_dim`
  channels (layers/patch_embed.py:55-74), flattened row-major into patch rows;
* a class token and 4 storage tokens in front of them (:210-235);
* `depth` SelfAttentionBlocks (16 heads, MLP ratio 4, qkv bias with the K third
  masked, LayerScale, LayerNorm eps 1e-5: the "layernormbf16" norm) with axial
  RoPE on the patch rows (base 100, coordinates normalised by max(H, W), fp32
  tables);
* a final LayerNorm over every row; `x_norm_patchtokens` are its patch rows.

The blocks are this package's SelfAttentionBlock, the class of the aggregator's
frame blocks (which add a q/k LayerNorm), so under bf16/f16 autocast the encoder
runs the same HIP row passes, QKV epilogue (LayerNorm-free, with RoPE) and
attention kernels.  The encoder is not part of the merged path: the aggregator
runs it only when no patch-token cache is installed, which lets the C4 forward
be timed with its encoder as well as from cached patch tokens.
"""
from __future__ import annotations

import math

import torch
from torch import Tensor, nn

from .layers import Mlp, SelfAttentionBlock, init_weights_vit, rope_sincos


class PatchEncoder(nn.Module):
    def __init__(self, patch_size: int = 16, embed_dim: int = 1024, depth: int = 24,
                 num_heads: int = 16, ffn_ratio: float = 4.0, n_storage_tokens: int = 4,
                 layerscale_init: float = 1.0e-5, device=None) -> None:
        super().__init__()
        self.patch_size = patch_size
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.n_storage_tokens = n_storage_tokens
        self.proj = nn.Conv2d(3, embed_dim, kernel_size=patch_size, stride=patch_size, device=device)
        self.cls_token = nn.Parameter(torch.empty(1, 1, embed_dim, device=device))
        self.storage_tokens = nn.Parameter(torch.empty(1, n_storage_tokens, embed_dim, device=device))
        self.mask_token = nn.Parameter(torch.empty(1, embed_dim, device=device))
        self.blocks = nn.ModuleList([
            SelfAttentionBlock(dim=embed_dim, num_heads=num_heads, ffn_ratio=ffn_ratio, qkv_bias=True,
                               proj_bias=True, ffn_bias=True, ffn_layer=Mlp, init_values=layerscale_init,
                               norm_layer=_layer_norm, mask_k_bias=True, use_qk_norm=False, device=device)
            for _ in range(depth)])
        self.norm = _layer_norm(embed_dim, device=device)
        self.init_weights()

    def init_weights(self) -> None:
        """`DinoVisionTransformer.init_weights` (vision_transformer.py:196-201) and the
        patch projection's `reset_parameters` (patch_embed.py:91-95)."""
        nn.init.normal_(self.cls_token, std=0.02)
        nn.init.normal_(self.storage_tokens, std=0.02)
        nn.init.zeros_(self.mask_token)
        bound = math.sqrt(1.0 / (3 * self.patch_size ** 2))
        nn.init.uniform_(self.proj.weight, -bound, bound)
        nn.init.uniform_(self.proj.bias, -bound, bound)
        for module in self.blocks.modules():
            init_weights_vit(module)
        self.norm.reset_parameters()

    def forward(self, images: Tensor) -> dict[str, Tensor]:
        """[B, 3, H, W] normalised images -> the `forward_features` dict of one crop:
        x_norm_clstoken [B, D], x_storage_tokens [B, n, D], x_norm_patchtokens [B, HW, D]."""
        x = self.proj(images)
        B, D, H, W = x.shape
        x = x.flatten(2).transpose(1, 2)
        cls = self.cls_token + 0 * self.mask_token  # the reference's unmasked class token
        x = torch.cat([cls.expand(B, -1, -1).to(x.dtype), self.storage_tokens.expand(B, -1, -1).to(x.dtype), x],
                      dim=1)
        with torch.no_grad():
            rope = rope_sincos(H, W, D // self.num_heads, device=x.device)
        for blk in self.blocks:
            x = blk(x, rope)
        x = self.norm(x)
        n = self.n_storage_tokens
        return {"x_norm_clstoken": x[:, 0], "x_storage_tokens": x[:, 1:n + 1],
                "x_norm_patchtokens": x[:, n + 1:]}


def _layer_norm(dim: int, device=None) -> nn.LayerNorm:
    """The encoder's "layernormbf16" norm: torch LayerNorm with eps 1e-5
    (vision_transformer.py:34-38)."""
    return nn.LayerNorm(dim, eps=1e-5, device=device)
