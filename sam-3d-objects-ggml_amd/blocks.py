"""The SLAT flow model's sparse residual block on the fused kernels.

SparseResBlock3d (sam3d_objects/model/backbone/tdfy_dit/models/
structured_latent_flow.py:15-74; native graph SRC/slat_flow_graph.cpp:
284-380) computes

    x = updown(x)
    h = conv1(silu(norm1(x)))                              norm1: LayerNorm32, affine
    h = conv2(silu(norm2(h) * (1 + scale) + shift))        norm2: LayerNorm32, no affine
    out = h + skip(x)                                      skip: SparseLinear or identity

with (scale, shift) = chunk(emb_layers(emb)).  Here it runs as three
kernels: spc_layernorm_silu (norm1 + SiLU), conv1 with the norm2 /
modulation / SiLU epilogue (whole output rows in one tile, Cout <= 128) and
conv2 with the residual epilogue.  Every intermediate is rounded to the
feature dtype where the reference's tensors are (LayerNorm32 casts back,
bf16 / f16 elementwise ops round per op).  Parameters and state-dict keys
are the reference's.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from . import _native as nat
from .sparse import SparseConv3d, SparseDownsample, SparseLinear, SparseTensor, SparseUpsample

__all__ = ["LayerNorm32", "SparseResBlock3d"]


class LayerNorm32(nn.LayerNorm):
    """LayerNorm computed in F32, cast back to the input dtype
    (modules/norm.py:6-8)."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return super().forward(x.float()).type(x.dtype)


class SparseResBlock3d(nn.Module):
    def __init__(self, channels: int, emb_channels: int, out_channels: Optional[int] = None,
                 downsample: bool = False, upsample: bool = False):
        super().__init__()
        self.channels = channels
        self.emb_channels = emb_channels
        self.out_channels = out_channels or channels
        self.downsample = downsample
        self.upsample = upsample
        assert not (downsample and upsample), "Cannot downsample and upsample at the same time"
        self.norm1 = LayerNorm32(channels, elementwise_affine=True, eps=1e-6)
        self.norm2 = LayerNorm32(self.out_channels, elementwise_affine=False, eps=1e-6)
        self.conv1 = SparseConv3d(channels, self.out_channels, 3)
        self.conv2 = SparseConv3d(self.out_channels, self.out_channels, 3)
        for p in self.conv2.parameters():  # zero_module (modules/utils.py)
            p.detach().zero_()
        self.emb_layers = nn.Sequential(nn.SiLU(), nn.Linear(emb_channels, 2 * self.out_channels,
                                                             bias=True))
        self.skip_connection = (SparseLinear(channels, self.out_channels)
                                if channels != self.out_channels else nn.Identity())
        self.updown = None
        if self.downsample:
            self.updown = SparseDownsample(2)
        elif self.upsample:
            self.updown = SparseUpsample(2)

    def _updown(self, x: SparseTensor) -> SparseTensor:
        if self.updown is not None:
            x = self.updown(x)
        return x

    def forward(self, x: SparseTensor, emb: torch.Tensor) -> SparseTensor:
        emb_out = self.emb_layers(emb).type(x.dtype)
        scale, shift = torch.chunk(emb_out, 2, dim=1)
        x = self._updown(x)
        h = x.replace(nat.layernorm_silu(x.feats, self.norm1.weight, self.norm1.bias,
                                         eps=self.norm1.eps))
        if self.out_channels <= 128 and self.out_channels % 32 == 0:
            h = self.conv1.forward_fused(h, norm_mod=(scale.float(), shift.float(),
                                                      self.norm2.eps))
        else:
            h = self.conv1(h)
            h = h.replace(nat.layernorm_silu(h.feats, eps=self.norm2.eps, silu=False))
            h = h * (1 + scale) + shift
            h = h.replace(torch.nn.functional.silu(h.feats))
        skip = self.skip_connection(x)
        if self.out_channels % 32 == 0:
            return self.conv2.forward_fused(h, residual=skip.feats)
        return self.conv2(h) + skip
