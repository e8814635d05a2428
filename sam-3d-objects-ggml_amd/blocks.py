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
modulation / SiLU epilogue (whole output rows in one tile: Cout 32, 64 or
128; other widths run conv1 and then one spc_layernorm_mod_silu row pass)
and conv2 with the residual epilogue.  Every intermediate is rounded to the
feature dtype where the reference's tensors are (LayerNorm32 casts back,
bf16 / f16 elementwise ops round per op).  Parameters and state-dict keys
are the reference's.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from . import _native as nat
from .sparse import (SparseConv3d, SparseDownsample, SparseGroupNorm32, SparseLinear, SparseSiLU,
                     SparseSubdivide, SparseTensor, SparseUpsample, _pad32, _run, _subm_map,
                     batch_offsets, max_item_rows)

__all__ = ["LayerNorm32", "SparseResBlock3d", "SparseSubdivideBlock3d"]


def _tap_merge_matrix() -> torch.Tensor:
    """[64, 27] 0/1 (F64): row d*8 + t (child class d = dx*4 + dy*2 + dz,
    parent tap t = ix*4 + iy*2 + iz at offset j_a = d_a - 1 + i_a) has a 1 at
    child tap o (offset k = (o//9 - 1, (o//3)%3 - 1, o%3 - 1)) when
    floor((d_a + k_a) / 2) = j_a on every axis."""
    m = torch.zeros(64, 27, dtype=torch.float64)
    for d in range(8):
        da = (d >> 2, (d >> 1) & 1, d & 1)
        for t in range(8):
            ja = tuple(da[a] - 1 + ((t >> (2 - a)) & 1) for a in range(3))
            for o in range(27):
                ka = (o // 9 - 1, (o // 3) % 3 - 1, o % 3 - 1)
                if all((da[a] + ka[a]) // 2 == ja[a] for a in range(3)):
                    m[d * 8 + t, o] = 1.0
    return m


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
        # upsample: norm1 / SiLU and the skip on the coarse rows (see
        # _forward_upsample); False runs the reference's order over the
        # upsampled copies
        self.coarse_rows = True

    def _updown(self, x: SparseTensor) -> SparseTensor:
        if self.updown is not None:
            x = self.updown(x)
        return x

    def forward(self, x: SparseTensor, emb: torch.Tensor) -> SparseTensor:
        emb_out = self.emb_layers(emb).type(x.dtype)
        scale, shift = torch.chunk(emb_out, 2, dim=1)
        if self.upsample and self.coarse_rows:
            return self._forward_upsample(x, scale, shift)
        x = self._updown(x)
        h = x.replace(nat.layernorm_silu(x.feats, self.norm1.weight, self.norm1.bias,
                                         eps=self.norm1.eps))
        if self.out_channels in (32, 64, 128):
            # one conv tile holds whole output rows: norm2 / modulation / SiLU
            # in the conv's epilogue
            h = self.conv1.forward_fused(h, norm_mod=(scale.float(), shift.float(),
                                                      self.norm2.eps))
        else:
            # wider rows: the conv, then one row pass for norm2 / modulation / SiLU
            h = self.conv1(h)
            h = h.replace(nat.layernorm_mod_silu(h.feats, scale.float(), shift.float(), h.coords,
                                                 eps=self.norm2.eps))
        skip = self.skip_connection(x)
        if self.out_channels % 32 == 0:
            return self.conv2.forward_fused(h, residual=skip.feats)
        return self.conv2(h) + skip


    def _forward_upsample(self, x: SparseTensor, scale: torch.Tensor,
                          shift: torch.Tensor) -> SparseTensor:
        """forward() with upsampling.  The reference upsamples first (fine
        row f is a copy of coarse row up[f]) and normalises the copies; norm1,
        SiLU and the skip Linear are row-wise, so they run on the coarse rows
        (2048 channels over 11,774 instead of 62,710 rows in the SLAT output
        block), conv1 reads them through the fine neighbour table composed
        with up[] (the same values per row and tap, so the same sums, without
        writing the copies), and conv2 adds the skip from row up[f] in its
        epilogue."""
        up = self.updown
        rows = up.fine_rows(x)
        n_f, n_c = rows.shape[0], x.feats.shape[0]
        h_c = nat.layernorm_silu(x.feats, self.norm1.weight, self.norm1.bias, eps=self.norm1.eps)
        # the fine level (coordinates, layout and cached maps of the paired
        # downsample's input); its features are conv1's output
        fine = up.fine_tensor(x, h_c.new_empty((n_f, 0)))
        m = _subm_map(fine)
        c1 = self.conv1.conv
        comp = fine.data.cached("subm3_from_coarse", lambda c: nat.compose_rows(m.token_major, rows))
        plan = fine.data.cached(("plan", "subm3_from_coarse"), lambda c: nat.conv_plan(
            comp, ntaps=27, n_out=n_f, n_in=n_c, device=c.device, sections=nat.plan_section(
                h_c.dtype, ntaps=27, n_out=n_f, cin=_pad32(c1.in_channels),
                cout=_pad32(c1.out_channels),
                epi_mode=nat.EPI_NORM_MOD_SILU if self.out_channels in (32, 64, 128) else 0)))
        if self.out_channels in (32, 64, 128):
            y1 = self.conv1._conv(h_c, comp, n_f, plan,
                                  norm_mod=(scale.float(), shift.float(), fine.coords,
                                            self.norm2.eps))
        else:
            y1 = self.conv1._conv(h_c, comp, n_f, plan)
            y1 = nat.layernorm_mod_silu(y1, scale.float(), shift.float(), fine.coords,
                                        eps=self.norm2.eps)
        h = fine.replace(y1)
        skip = self.skip_connection(x).feats
        if self.out_channels % 32 == 0:
            return self.conv2.forward_fused(h, residual=skip, residual_rows=rows)
        return self.conv2(h) + h.replace(nat.gather_rows(skip, rows))


class SparseSubdivideBlock3d(nn.Module):
    """The mesh decoder's upsampling block (decoder_mesh.py:17-83;
    SRC/mesh_decoder_graph.cpp:399-437):

        h = out_layers(subdivide(silu(groupnorm(x))))
        out = h + skip(subdivide(x))

    with out_layers = [conv 3x3x3, GroupNorm32, SiLU, conv 3x3x3] and skip a
    1x1x1 conv when the channel count changes.  Runs as: GroupNorm
    statistics + norm / SiLU on the parent rows, conv1 on the parents' rows
    (the children's features are copies of them), GroupNorm statistics +
    norm / SiLU, conv2 with the skip (computed on the parent rows) added in
    its epilogue.  conv1 runs in merged-tap form by default (`merged_taps`):
    a child's 27 taps land on 8 parent rows, so it runs as 8 taps with
    summed weights per child class (spc_subdivide_tap_classes) -- 8 / 27 of
    the MFMA work; the summed weights are rounded once to the feature
    dtype, so the result agrees with the 27-tap conv to that rounding.
    `merged_taps = False` runs the 27 taps over the composed child table
    (bit-identical to the conv over the copied rows).  State-dict keys are
    the reference's (act_layers.0.*, out_layers.0.conv.*, out_layers.1.*,
    out_layers.3.conv.*, skip_connection.conv.*)."""

    def __init__(self, channels: int, resolution: int, out_channels: Optional[int] = None,
                 num_groups: int = 32):
        super().__init__()
        self.channels = channels
        self.resolution = resolution
        self.out_resolution = resolution * 2
        self.out_channels = out_channels or channels
        self.act_layers = nn.Sequential(SparseGroupNorm32(num_groups, channels), SparseSiLU())
        self.sub = SparseSubdivide()
        conv2 = SparseConv3d(self.out_channels, self.out_channels, 3,
                             indice_key=f"res_{self.out_resolution}")
        for p in conv2.parameters():  # zero_module (modules/utils.py)
            p.detach().zero_()
        self.out_layers = nn.Sequential(
            SparseConv3d(channels, self.out_channels, 3, indice_key=f"res_{self.out_resolution}"),
            SparseGroupNorm32(num_groups, self.out_channels),
            SparseSiLU(),
            conv2,
        )
        if self.out_channels == channels:
            self.skip_connection = nn.Identity()
        else:
            self.skip_connection = SparseConv3d(channels, self.out_channels, 1,
                                                indice_key=f"res_{self.out_resolution}")
        self.merged_taps = True
        self._merged = None
        self._merged_key = None

    def _merged_weights(self, dtype: torch.dtype, device) -> nat.PackedWeights:
        """conv1's weights summed per (child class d, parent tap t): W'[d*8 + t]
        = sum of W_k over the child taps k with floor((d + k) / 2) = j(d, t),
        formed in F64 and rounded once to the feature dtype; packed as 64
        taps (cached per weight version)."""
        conv1 = self.out_layers[0]
        c = conv1.conv
        key = (dtype, device, c.weight.data_ptr(), c.weight._version,
               None if conv1._q8 is None else conv1._q8[0].data_ptr())
        if self._merged is not None and self._merged_key == key:
            return self._merged
        cin, cout = c.in_channels, c.out_channels
        if conv1._q8 is not None:
            blocks, layout = conv1._q8
            w = nat.q8_0_dequant(blocks.to(device), torch.float32)
            w = (w.view(27, cout, cin).permute(1, 0, 2) if layout == "mesh"
                 else w.view(cout, 27, cin))
        else:
            w = c.weight.detach().to(device=device).reshape(cout, 27, cin)
        w = w.to(torch.float64).permute(1, 0, 2).reshape(27, cout * cin)
        wm = torch.matmul(_tap_merge_matrix().to(device), w).reshape(64, cout, cin)
        self._merged = nat.pack_weights(wm.to(dtype).contiguous(), layout=nat.W_TCK)
        self._merged_key = key
        return self._merged

    def forward(self, x: SparseTensor) -> SparseTensor:
        gn0, gn1 = self.act_layers[0], self.out_layers[1]
        conv1, conv2 = self.out_layers[0], self.out_layers[3]
        coords, parent = self.sub.map(x)
        nc = coords.shape[0]
        offs, rows_max = batch_offsets(x), max_item_rows(x)
        # silu(GroupNorm(x)) on the parent rows only: the children's features
        # are copies of them, so conv1 reads the parents through the child
        # neighbour table composed with the parent rows (bit-identical to the
        # conv over the copies, without writing 8x the rows)
        h_par = nat.group_norm_silu(x.feats, offs, gn0.num_groups, gn0.weight, gn0.bias, gn0.eps,
                                    silu=True, max_rows=rows_max)
        # the child table follows from the parents' one (no hash build)
        n_par = x.feats.shape[0]
        pm = _subm_map(x).token_major
        cm = nat.subdivide_neighbors(pm, n_par)
        c1, c2 = conv1.conv, conv2.conv
        dt = x.feats.dtype
        # the plans are rebuilt per call: only the tile geometry each conv runs
        if self.merged_taps and c1.in_channels % 32 == 0 and c1.out_channels % 32 == 0:
            idx8, perm, crows = nat.subdivide_tap_classes(pm, n_par)
            plan8 = nat.conv_plan(idx8, ntaps=8, n_out=8 * crows, n_in=n_par, row_perm=perm,
                                  sections=nat.plan_section(
                                      dt, ntaps=8, n_out=8 * crows, cin=c1.in_channels,
                                      cout=c1.out_channels, class_rows=crows))
            hp = h_par.detach()
            y1 = _run(lambda: nat.sparse_conv(
                hp, self._merged_weights(hp.dtype, hp.device), conv1._bias_operand(hp.dtype, hp.device),
                idx8, ntaps=8, n_out=8 * crows, row_perm=perm, plan=plan8, class_rows=crows,
                n_classes=8)[:nc], h_par, c1.weight, c1.bias)
        else:
            composed = nat.compose_rows(cm.token_major, parent)
            plan1 = nat.conv_plan(composed, ntaps=27, n_out=nc, n_in=n_par,
                                  sections=nat.plan_section(dt, ntaps=27, n_out=nc,
                                                            cin=_pad32(c1.in_channels),
                                                            cout=_pad32(c1.out_channels)))
            y1 = conv1._conv(h_par, composed, nc, plan1)
        h = self.sub.assemble(x, coords, y1)
        h.data.cached("subm3", lambda c: cm)  # conv2's map: the same child coordinates
        h.data.cached(("plan", "subm3"), lambda c: nat.conv_plan(
            cm.token_major, ntaps=27, n_out=nc, device=c.device, sections=nat.plan_section(
                dt, ntaps=27, n_out=nc, cin=_pad32(c2.in_channels), cout=_pad32(c2.out_channels),
                epi_mode=nat.EPI_RESIDUAL)))
        h = h.replace(nat.group_norm_silu(h.feats, 8 * offs, gn1.num_groups, gn1.weight, gn1.bias,
                                          gn1.eps, silu=True, max_rows=8 * rows_max))
        # the skip on the parent rows (a 1x1x1 conv is row-wise), added to
        # child t from row parent[t] in conv2's epilogue
        skip = x.feats if isinstance(self.skip_connection, nn.Identity) \
            else self.skip_connection(x).feats
        if self.out_channels % 32 == 0:
            return conv2.forward_fused(h, residual=skip, residual_rows=parent)
        return conv2(h) + h.replace(nat.gather_rows(skip, parent))
