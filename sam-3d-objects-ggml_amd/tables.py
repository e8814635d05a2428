"""GPU builders of the reference's host index-table structs.

SlatTables   cpp_ggml/src/sparse_ops.hpp:11-50, built by sparse_ops.cpp:23-186
MeshTables   cpp_ggml/src/sparse_ops.hpp:84-102, built by sparse_ops.cpp:375-391

Same field names and contents (bit-exact), as int32 / float32 device
tensors, produced by the library's map kernels instead of std::map loops.
Left out: the absolute-position embeddings (`ape`) and the Swin window
tables of the Gaussian/mesh decoders' attention torso, which are not part of
the sparse convolution path.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import torch

from . import _native as nat


@dataclass
class SlatTables:
    nf: int
    nc: int
    fine_to_coarse: torch.Tensor       # [nf]
    coarse_children: torch.Tensor      # [8*nc], padded with nf
    coarse_count: torch.Tensor         # [nc] float32, |children| + 1
    conv_fine: torch.Tensor            # [nf*27] token-major, sentinel nf
    conv_coarse: torch.Tensor          # [nc*27] token-major, sentinel nc
    conv_fine_spconv: torch.Tensor     # [27*nf] offset-major, -1 missing
    conv_coarse_spconv: torch.Tensor   # [27*nc]
    conv_fine_mask: torch.Tensor       # [nf] masks, stable ascending
    conv_coarse_mask: torch.Tensor     # [nc]
    conv_fine_argsort: torch.Tensor    # [nf]
    conv_coarse_argsort: torch.Tensor  # [nc]
    coarse_coords: torch.Tensor        # [nc, 4] (b, x/2, y/2, z/2)

    @classmethod
    def build(cls, coords: torch.Tensor, resolution: int = 64) -> "SlatTables":
        """coords: int32 [nf, 4] (b, x, y, z) on the GPU, 0 <= x,y,z <
        resolution.  Raises SparseConvError where SlatTables::build returns
        false (no rows; coordinates the coarse key cannot hold)."""
        coords = coords.contiguous()
        nf = coords.shape[0]
        if nf <= 0:
            raise nat.SparseConvError("SlatTables.build", nat.BAD_SHAPE, "no tokens")
        n_batch = int(coords[:, 0].max().item()) + 1
        d = nat.downsample_map(coords, n_batch, resolution, with_taps=False)
        fine = nat.map_build(coords)
        coarse = nat.map_build(d.coarse_coords.contiguous())
        return cls(nf, d.nc, d.fine_to_coarse, d.children, d.counts, fine.token_major,
                   coarse.token_major, fine.offset_major, coarse.offset_major,
                   fine.mask_sorted, coarse.mask_sorted, fine.argsort, coarse.argsort,
                   d.coarse_coords)


@dataclass
class MeshConvLevel:
    n: int
    resolution: int
    coords: torch.Tensor               # [n, 4]
    conv: torch.Tensor                 # [n*27] token-major, sentinel n
    parent: Optional[torch.Tensor] = None  # [n] row of the parent level (levels 1, 2)


@dataclass
class MeshTables:
    levels: List[MeshConvLevel] = field(default_factory=list)

    @classmethod
    def build(cls, coords: torch.Tensor, base_resolution: int = 64,
              keep: Optional[List[Optional[torch.Tensor]]] = None) -> "MeshTables":
        """levels[0] is the input support, levels[1] and [2] the two
        SparseSubdivide expansions (child c = dx*4 + dy*2 + dz at row
        parent*8 + c).  Each level's conv table has the build_mesh_conv_table
        checks: coordinates in [0, resolution) and unique, else
        SparseConvError (BAD_COORD / DUP_COORD).  `keep` optionally prunes
        the children of level 1 and 2 ([8n] masks, survivors kept in
        parent-major order) -- an extension, the reference keeps all."""
        coords = coords.contiguous()
        if coords.shape[0] <= 0 or base_resolution <= 0:
            raise nat.SparseConvError("MeshTables.build", nat.BAD_SHAPE, "empty input")
        keep = keep or [None, None]
        res = base_resolution
        m = nat.map_build(coords, mesh_resolution=res, outputs="token")
        levels = [MeshConvLevel(coords.shape[0], res, coords, m.token_major)]
        for k in keep[:2]:
            prev = levels[-1]
            c, par = nat.subdivide_map(prev.coords, k)
            res *= 2
            m = nat.map_build(c, mesh_resolution=res, outputs="token")
            levels.append(MeshConvLevel(c.shape[0], res, c, m.token_major, par))
        return cls(levels)
