"""Sparse operator surface: SparseTensor, SparseConv3d, SparseInverseConv3d,
SparseDownsample, SparseUpsample, SparseSubdivide.

Same names, constructor arguments, state-dict keys and bookkeeping (shape,
layout, scale, spatial cache) as the reference's
sam3d_objects/model/backbone/tdfy_dit/modules/sparse (SP below):
  SparseTensor            SP/basic.py:20-453
  SparseConv3d            SP/conv/conv_spconv.py:9-89
  SparseInverseConv3d     SP/conv/conv_spconv.py:92-139
  SparseDownsample        SP/spatial.py:10-72
  SparseUpsample          SP/spatial.py:75-105
  SparseSubdivide         SP/spatial.py:108-130
The reference delegates the maps and convolutions to spconv; here every map
(neighbour tables, stride-2 and subdivide maps) and every feature op (conv,
scatter-mean, row gather) is a HIP kernel of libsam3d_spconv_amd.so.  There
is no CPU path: feature tensors must live on the GPU.

Supported convolutions (what the SAM 3D models instantiate):
  kernel 3, stride 1, padding None   submanifold 3x3x3 (27 taps)
  kernel 1, stride 1, padding None   submanifold 1x1x1; its weight is read the
                                     way spconv's Conv1x1 path reads it (the
                                     saved [Cout,1,1,1,Cin] buffer viewed as
                                     (Cin, Cout)), as the reference's decoder
                                     does (SRC/mesh_decoder_graph.cpp:349-376)
  kernel 2, stride 2                 2x2x2 downsampling conv, output rows in
                                     lexicographic (b, x/2, y/2, z/2) order
                                     (SRC/sparse_ops.cpp:27-81)
Anything else raises NotImplementedError.  Channel counts that are not
multiples of 32 are zero-padded around the kernel.  The modules are
forward-only (inference): the conv's backward raises.
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple, Union

import torch
import torch.nn as nn

from . import _native as nat

__all__ = [
    "SparseTensor", "SparseTensorData", "sparse_batch_broadcast", "sparse_batch_op",
    "sparse_cat", "sparse_unbind", "SparseConv3d", "SparseInverseConv3d",
    "SparseDownsample", "SparseUpsample", "SparseSubdivide", "SparseLinear",
    "SparseGroupNorm32", "SparseSiLU",
]

BACKEND = "hip"
DEBUG = False


# ---------------------------------------------------------------------------
# storage
# ---------------------------------------------------------------------------
class SparseTensorData:
    """Features, coordinates and the kernel maps built for those coordinates
    (the role spconv's SparseConvTensor plays for the reference)."""

    def __init__(self, features: torch.Tensor, indices: torch.Tensor,
                 spatial_shape: Sequence[int], batch_size: int,
                 indice_dict: Optional[dict] = None):
        self.features = features
        self.indices = indices
        self.spatial_shape = [int(s) for s in spatial_shape]
        self.batch_size = int(batch_size)
        # maps keyed by kind; each entry remembers the coordinate tensor (and
        # its version counter) it was built from
        self.indice_dict = {} if indice_dict is None else indice_dict

    def replace_feature(self, features: torch.Tensor) -> "SparseTensorData":
        return SparseTensorData(features, self.indices, self.spatial_shape, self.batch_size,
                                self.indice_dict)

    def dense(self, channels_first: bool = True) -> torch.Tensor:
        f = self.features.reshape(self.features.shape[0], -1)
        out = torch.zeros((self.batch_size, *self.spatial_shape, f.shape[1]), dtype=f.dtype,
                          device=f.device)
        idx = self.indices.long()
        out[idx[:, 0], idx[:, 1], idx[:, 2], idx[:, 3]] = f
        if channels_first:
            out = out.permute(0, 4, 1, 2, 3).contiguous()
        return out

    def cached(self, key, build):
        """Returns the map `key` for the current coordinates, building it on
        first use (or when the coordinates changed)."""
        ent = self.indice_dict.get(key)
        c = self.indices
        if ent is not None and ent[0] is c and ent[1] == c._version:
            return ent[2]
        val = build(c)
        self.indice_dict[key] = (c, c._version, val)
        return val


# ---------------------------------------------------------------------------
# SparseTensor (SP/basic.py:20-453)
# ---------------------------------------------------------------------------
class SparseTensor:
    """Sparse tensor: feats [N, C...] and int32 coords [N, 4] (b, x, y, z),
    rows of one batch contiguous, coordinates in [0, 1023].

    SparseTensor(feats, coords, shape=None, layout=None, **kwargs) or
    SparseTensor(data, shape=None, layout=None, **kwargs); kwargs `scale`
    and `spatial_cache` as in SP/basic.py:55-137."""

    # the two constructor forms: a leading tensor selects the first, a
    # leading SparseTensorData (or, with no positional argument, a `data`
    # keyword) the second
    _FORMS = (("feats", "coords", "shape", "layout"), ("data", "shape", "layout"))

    def __init__(self, *args, **kwargs):
        if args:
            names = self._FORMS[0 if isinstance(args[0], torch.Tensor) else 1]
        else:
            names = self._FORMS[1 if "data" in kwargs else 0]
        if len(args) > len(names):
            raise TypeError(f"SparseTensor takes at most {len(names)} positional arguments")
        given = dict(zip(names, args))
        for name in names:
            if name in kwargs:
                given[name] = kwargs[name]  # a keyword wins over the positional slot
        if "data" in names:
            self.data = given.get("data")
        else:
            coords = given.get("coords")
            shape0 = given.get("shape")
            n_b = shape0[0] if shape0 is not None else self._batch_count(coords)
            extent = [0, 0, 0]
            if coords.shape[0]:
                extent = [int(v) + 1 for v in coords[:, 1:].amax(0).tolist()]
            self.data = SparseTensorData(given.get("feats"), coords, extent, n_b)
        shape = given.get("shape")
        if shape is None:
            shape = torch.Size([self._batch_count(self.coords), *self.feats.shape[1:]])
        layout = given.get("layout")
        if layout is None:
            layout = self._batch_slices(self.coords, shape[0])
        self._shape = torch.Size(shape)
        self._layout = layout
        self._scale = kwargs.get("scale", (1, 1, 1))
        self._spatial_cache = kwargs.get("spatial_cache", {})
        if DEBUG:
            assert self.feats.shape[0] == self.coords.shape[0]
            for i in range(self.shape[0]):
                assert torch.all(self.coords[self.layout[i], 0] == i), \
                    f"the rows of batch {i} are not contiguous"

    @staticmethod
    def _batch_count(coords) -> int:
        """Batch items: one past the largest batch index."""
        return int(coords[:, 0].max().item()) + 1

    @staticmethod
    def _batch_slices(coords, batch_size) -> List[slice]:
        """Row range of each batch item (rows of an item are contiguous)."""
        sizes = torch.bincount(coords[:, 0], minlength=batch_size)[:batch_size]
        ends = torch.cumsum(sizes, 0).tolist()
        return [slice(e - int(c), e) for e, c in zip(ends, sizes.tolist())]

    # -- accessors ----------------------------------------------------------
    @property
    def shape(self) -> torch.Size:
        return self._shape

    def dim(self) -> int:
        return len(self.shape)

    @property
    def layout(self) -> List[slice]:
        return self._layout

    @property
    def feats(self) -> torch.Tensor:
        return self.data.features

    @feats.setter
    def feats(self, value: torch.Tensor):
        self.data.features = value

    @property
    def coords(self) -> torch.Tensor:
        return self.data.indices

    @coords.setter
    def coords(self, value: torch.Tensor):
        self.data.indices = value

    @property
    def dtype(self):
        return self.feats.dtype

    @property
    def device(self):
        return self.feats.device

    # -- conversions --------------------------------------------------------
    def to(self, *args, **kwargs) -> "SparseTensor":
        """to(device), to(dtype), to(device, dtype) or the keywords; the
        coordinates follow the device only."""
        target = {"device": None, "dtype": None}
        if len(args) == 2:
            target["device"], target["dtype"] = args
        elif len(args) == 1:
            target["dtype" if isinstance(args[0], torch.dtype) else "device"] = args[0]
        for k in ("device", "dtype"):
            if k in kwargs:
                assert target[k] is None, f"to() received multiple values for argument '{k}'"
                target[k] = kwargs[k]
        return self.replace(self.feats.to(**target), self.coords.to(device=target["device"]))

    def type(self, dtype) -> "SparseTensor":
        return self.replace(self.feats.type(dtype))

    def cpu(self) -> "SparseTensor":
        return self.replace(self.feats.cpu(), self.coords.cpu())

    def cuda(self) -> "SparseTensor":
        return self.replace(self.feats.cuda(), self.coords.cuda())

    def half(self) -> "SparseTensor":
        return self.replace(self.feats.half())

    def float(self) -> "SparseTensor":
        return self.replace(self.feats.float())

    def detach(self) -> "SparseTensor":
        return self.replace(self.feats.detach(), self.coords.detach())

    def dense(self) -> torch.Tensor:
        return self.data.dense()

    def reshape(self, *shape) -> "SparseTensor":
        return self.replace(self.feats.reshape(self.feats.shape[0], *shape))

    def unbind(self, dim: int) -> List["SparseTensor"]:
        return sparse_unbind(self, dim)

    def replace(self, feats: torch.Tensor, coords: Optional[torch.Tensor] = None
                ) -> "SparseTensor":
        """Same coordinates (or `coords`), layout, scale and spatial cache;
        new features.  Kernel maps built for the coordinates are shared."""
        new_shape = [self.shape[0], *feats.shape[1:]]
        data = SparseTensorData(feats, self.data.indices if coords is None else coords,
                                self.data.spatial_shape, self.data.batch_size,
                                self.data.indice_dict)
        return SparseTensor(data, shape=torch.Size(new_shape), layout=self.layout,
                            scale=self._scale, spatial_cache=self._spatial_cache)

    @staticmethod
    def full(aabb, dim, value, dtype=torch.float32, device=None) -> "SparseTensor":
        """Every voxel of the inclusive box aabb = (x0, y0, z0, x1, y1, z1)
        in each of dim[0] batch items, dim[1] channels of `value`; rows in
        (b, x, y, z) lexicographic order."""
        n_b, c = dim
        lo = torch.tensor(aabb[:3], dtype=torch.int64)
        ext = torch.tensor(aabb[3:], dtype=torch.int64) - lo + 1
        cells = int(ext.prod())
        r = torch.arange(n_b * cells, dtype=torch.int64)
        local = r % cells
        coords = torch.stack([r // cells, lo[0] + local // (ext[1] * ext[2]),
                              lo[1] + (local // ext[2]) % ext[1], lo[2] + local % ext[2]], 1)
        coords = coords.to(dtype=torch.int32, device=device)
        feats = torch.full((coords.shape[0], c), value, dtype=dtype, device=device)
        return SparseTensor(feats=feats, coords=coords)

    # -- arithmetic ---------------------------------------------------------
    def __neg__(self) -> "SparseTensor":
        return self.replace(-self.feats)

    def _elemwise(self, other, op) -> "SparseTensor":
        # SP/basic.py:349-364: a SparseTensor operand is replaced by its feats
        # before the cache check there, so the result keeps self's spatial
        # cache only (replace) and the operands' caches are never merged
        if isinstance(other, torch.Tensor):
            try:
                other = sparse_batch_broadcast(self, torch.broadcast_to(other, self.shape))
            except (RuntimeError, ValueError):
                pass
        if isinstance(other, SparseTensor):
            other = other.feats
        return self.replace(op(self.feats, other))

    def __add__(self, other):
        return self._elemwise(other, torch.add)

    __radd__ = __add__

    def __sub__(self, other):
        return self._elemwise(other, torch.sub)

    def __rsub__(self, other):
        return self._elemwise(other, lambda x, y: torch.sub(y, x))

    def __mul__(self, other):
        return self._elemwise(other, torch.mul)

    __rmul__ = __mul__

    def __truediv__(self, other):
        return self._elemwise(other, torch.div)

    def __rtruediv__(self, other):
        return self._elemwise(other, lambda x, y: torch.div(y, x))

    def _batch_ids(self, idx) -> List[int]:
        """Batch items an index selects: an int, a slice, a bool mask over
        the items or an int32 / int64 vector of item indices."""
        if isinstance(idx, int):
            return [idx]
        if isinstance(idx, slice):
            return list(range(self.shape[0]))[idx]
        if not isinstance(idx, torch.Tensor):
            raise ValueError(f"Unknown index type: {type(idx)}")
        if idx.dtype == torch.bool:
            assert idx.shape == (self.shape[0],), f"Invalid index shape: {idx.shape}"
            return torch.nonzero(idx).flatten().tolist()
        if idx.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"Unknown index type: {idx.dtype}")
        assert idx.dim() == 1, f"Invalid index shape: {idx.shape}"
        return idx.tolist()

    def __getitem__(self, idx) -> "SparseTensor":
        """The selected batch items, renumbered 0.. in selection order."""
        rows = [self.layout[b] for b in self._batch_ids(idx)]
        coords = torch.cat([self.coords[r] for r in rows], 0)
        coords[:, 0] = torch.repeat_interleave(
            torch.arange(len(rows), dtype=coords.dtype, device=coords.device),
            torch.tensor([r.stop - r.start for r in rows], device=coords.device))
        feats = torch.cat([self.feats[r] for r in rows], 0)
        return SparseTensor(feats=feats.contiguous(), coords=coords.contiguous())

    # -- spatial cache (keyed by the current scale) -------------------------
    def register_spatial_cache(self, key, value) -> None:
        scale_key = str(self._scale)
        self._spatial_cache.setdefault(scale_key, {})[key] = value

    def get_spatial_cache(self, key=None):
        cur = self._spatial_cache.get(str(self._scale), {})
        return cur if key is None else cur.get(key, None)


def sparse_batch_broadcast(input: SparseTensor, other: torch.Tensor) -> torch.Tensor:
    """Row-wise copy of other[b] into every row of batch b."""
    out = torch.zeros_like(input.feats)
    for k in range(input.shape[0]):
        out[input.layout[k]] = other[k]
    return out


def sparse_batch_op(input: SparseTensor, other: torch.Tensor, op=torch.add) -> SparseTensor:
    return input.replace(op(input.feats, sparse_batch_broadcast(input, other)))


def sparse_cat(inputs: List[SparseTensor], dim: int = 0) -> SparseTensor:
    if dim == 0:
        start, coords = 0, []
        for t in inputs:
            c = t.coords.clone()
            c[:, 0] += start
            coords.append(c)
            start += t.shape[0]
        return SparseTensor(coords=torch.cat(coords, 0),
                            feats=torch.cat([t.feats for t in inputs], 0))
    return inputs[0].replace(torch.cat([t.feats for t in inputs], dim=dim))


def sparse_unbind(input: SparseTensor, dim: int) -> List[SparseTensor]:
    if dim == 0:
        return [input[i] for i in range(input.shape[0])]
    return [input.replace(f) for f in input.feats.unbind(dim)]


# ---------------------------------------------------------------------------
# maps (cached on the coordinates)
# ---------------------------------------------------------------------------
def _subm_map(x: SparseTensor) -> nat.SubmMap:
    """The submanifold table of x's coordinates, cached on them: over a dense
    grid when the batch count and spatial shape bound it within
    nat.DENSE_MAX_CELLS cells, else over the hash table."""
    def build(c):
        nb, shape = x.data.batch_size, x.data.spatial_shape
        if nb and shape and min(shape) > 0:
            res = max(int(v) for v in shape)
            if nb * res ** 3 <= nat.DENSE_MAX_CELLS:
                return nat.map_build(c.contiguous(), outputs="token", dense=(nb, res))
        return nat.map_build(c.contiguous(), outputs="token")

    return x.data.cached("subm3", build)


def _resolution(x: SparseTensor) -> int:
    return max(2, max(x.data.spatial_shape) if x.data.spatial_shape else 2)


def _plan(x: SparseTensor, key, idx, ntaps: int, n_out: int, n_in: int):
    """Tile plan of an index table, cached with the coordinates like the maps."""
    return x.data.cached(("plan", key), lambda c: nat.conv_plan(
        idx, ntaps=ntaps, n_out=n_out, n_in=n_in, device=c.device))


def _downsample_map(x: SparseTensor) -> nat.DownsampleMap:
    return x.data.cached(
        "down2", lambda c: nat.downsample_map(c.contiguous(), x.data.batch_size,
                                              _resolution(x), with_taps=True))


# ---------------------------------------------------------------------------
# convolution
# ---------------------------------------------------------------------------
def _triple(v) -> Tuple[int, int, int]:
    if isinstance(v, (list, tuple)):
        assert len(v) == 3
        return tuple(int(a) for a in v)
    return (int(v),) * 3


def _pad32(n: int) -> int:
    return (n + 31) // 32 * 32


class _ForwardOnly(torch.autograd.Function):
    """Runs a kernel closure; gradients are not implemented."""

    @staticmethod
    def forward(ctx, run, *tensors):
        return run()

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError("the HIP sparse convolution is forward-only")


def _run(run, *tensors):
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        return _ForwardOnly.apply(run, *tensors)
    return run()


class _ConvParams(nn.Module):
    """Parameters of one sparse conv, laid out as spconv's module holds them
    (weight [Cout, k, k, k, Cin], bias [Cout]) so that the reference's state
    dicts load unchanged (keys `conv.weight`, `conv.bias`)."""

    def __init__(self, in_channels, out_channels, kernel_size, stride, dilation, padding, bias,
                 indice_key, subm):
        super().__init__()
        self.in_channels = int(in_channels)
        self.out_channels = int(out_channels)
        self.kernel_size = kernel_size
        self.stride = stride
        self.dilation = dilation
        self.padding = padding
        self.indice_key = indice_key
        self.subm = subm
        self.weight = nn.Parameter(torch.empty(out_channels, *kernel_size, in_channels))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_channels))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()

    def reset_parameters(self):
        fan_in = self.in_channels * math.prod(self.kernel_size)
        bound = 1.0 / math.sqrt(fan_in)
        nn.init.uniform_(self.weight, -bound, bound)
        if self.bias is not None:
            nn.init.uniform_(self.bias, -bound, bound)


# Q8_0 convs over at least this many output rows expand the packed quants
# to packed bf16 once per forward (one HBM pass over the weights) and run
# the bf16 kernel; smaller ones dequantise in registers, once per row tile.
# Both give the same bits.  (With q8_operands = "f16", the default, bf16
# features take the f16-operand path instead, at every size.)
Q8_EXPAND_MIN_ROWS = 2048


class _ConvCore:
    """Weight packing (cached per weight version and dtype), Q8_0 weights
    and the kernel call shared by SparseConv3d and SparseInverseConv3d."""

    def _init_core(self, ntaps: int, raw_view: bool):
        self._ntaps = ntaps
        self._raw_view = raw_view  # 1x1x1: the (Cin, Cout) view of the buffer
        self._packed = None
        self._packed_key = None
        self._q8 = None            # (blocks uint8 tensor, layout) or None
        # Q8_0 weights under bf16 features: "f16" runs the reference's GEMM
        # operands -- features cast to f16 (exact inside f16's range) and
        # f16(f32(d) * q) weights (as_f16, SRC/slat_flow_graph.cpp:24-27) --
        # through the f16 kernel, the output cast back to bf16; "bf16" feeds
        # bf16(f32(d) * q) to the bf16 kernel (no feature casts, weights
        # rounded to 8 significant bits instead of 11).  Fused epilogues
        # always take "bf16", whose rounding steps they are defined in.
        self.q8_operands = "f16"

    # ---- Q8_0 -------------------------------------------------------------
    def load_q8_0(self, blocks: torch.Tensor, layout: str = "slat") -> None:
        """Uses ggml Q8_0 blocks (uint8, 34 bytes each) as the weight.
        layout "slat": rows [Cout, ntaps*Cin] (cpp_ggml/scripts/
        gguf_schema.py:330-338); "mesh": rows [ntaps, Cout*Cin]
        (convert_sam3d_to_gguf.py:508-511).  The float parameter is left as
        is; bf16 features dequantise in the GEMM, other dtypes dequantise
        once to the feature dtype (SRC/slat_flow_graph.cpp:24-27)."""
        if layout not in ("slat", "mesh"):
            raise ValueError("layout must be 'slat' or 'mesh'")
        c = self.conv
        n = self._ntaps * c.in_channels * c.out_channels
        if blocks.dtype != torch.uint8 or blocks.numel() != n // 32 * 34 or n % 32:
            raise ValueError(f"expected {n // 32 * 34} Q8_0 bytes for this conv")
        self._q8 = (blocks.contiguous(), layout)
        self._packed_key = None

    def quantize_q8_0(self, layout: str = "slat") -> torch.Tensor:
        """Quantises the current weight with the converter's Q8_0 recipe
        (gguf_schema.py:14-24) on the GPU, uses it, and returns the blocks."""
        c = self.conv
        w = c.weight.detach().float().reshape(c.out_channels, self._ntaps, c.in_channels)
        if layout == "mesh":
            w = w.permute(1, 0, 2)
        blocks = nat.q8_0_quantize(w.contiguous())
        self.load_q8_0(blocks, layout)
        return blocks

    # ---- packing ----------------------------------------------------------
    def _weight_operand(self, dtype: torch.dtype, device) -> nat.PackedWeights:
        c = self.conv
        cin, cout, t = c.in_channels, c.out_channels, self._ntaps
        cin_p, cout_p = _pad32(cin), _pad32(cout)
        key = (dtype, device, c.weight.data_ptr(), c.weight._version,
               None if self._q8 is None else self._q8[0].data_ptr())
        if self._packed is not None and self._packed_key == key:
            return self._packed
        q8_direct = (self._q8 is not None and dtype == torch.bfloat16 and not self._raw_view
                     and cout_p == cout and cin_p == cin)
        if q8_direct:
            blocks, layout = self._q8
            qs, d = nat.q8_0_repack(blocks.to(device))
            lay = nat.W_KRSC if layout == "slat" else nat.W_TCK
            packed = nat.pack_weights(qs, d, cin=cin, cout=cout, ntaps=t, layout=lay)
        else:
            if self._q8 is not None:
                blocks, layout = self._q8
                w = nat.q8_0_dequant(blocks.to(device), torch.float32)
                if layout == "mesh":
                    w = w.view(t, cout, cin).permute(1, 0, 2)
                w = w.reshape(-1)
            else:
                w = c.weight.detach().to(device=device, dtype=torch.float32).reshape(-1)
            if self._raw_view:
                # (Cin, Cout) view of the saved buffer: w[ci][co]
                wm = w.view(cin, cout)
                if cin_p != cin or cout_p != cout:
                    wm = torch.nn.functional.pad(wm, (0, cout_p - cout, 0, cin_p - cin))
                packed = nat.pack_weights(wm.to(dtype).reshape(1, cin_p, cout_p).contiguous(),
                                          layout=nat.W_TKC)
            else:
                wm = w.view(cout, t, cin)
                if cin_p != cin or cout_p != cout:
                    wm = torch.nn.functional.pad(wm, (0, cin_p - cin, 0, 0, 0, cout_p - cout))
                packed = nat.pack_weights(wm.to(dtype).contiguous(), layout=nat.W_KRSC)
        self._packed, self._packed_key = packed, key
        return packed

    def _bias_operand(self, dtype, device):
        b = self.conv.bias
        if b is None:
            return None
        b = b.detach().to(device=device, dtype=dtype)
        cout_p = _pad32(self.conv.out_channels)
        if cout_p != b.shape[0]:
            b = torch.nn.functional.pad(b, (0, cout_p - b.shape[0]))
        return b.contiguous()

    def _conv(self, feats: torch.Tensor, idx: Optional[torch.Tensor], n_out: int,
              plan: Optional[torch.Tensor] = None, residual: Optional[torch.Tensor] = None,
              norm_mod: Optional[tuple] = None,
              residual_rows: Optional[torch.Tensor] = None) -> torch.Tensor:
        c = self.conv
        if feats.dim() != 2 or feats.shape[1] != c.in_channels:
            raise ValueError(f"expected feats [N, {c.in_channels}], got {tuple(feats.shape)}")
        nat._need_gpu(feats)
        if (residual is not None or norm_mod is not None) and c.out_channels % 32:
            raise ValueError("fused epilogues need out_channels a multiple of 32")

        def run():
            x = feats.detach().contiguous()
            cin_p = _pad32(c.in_channels)
            if cin_p != c.in_channels:
                x = torch.nn.functional.pad(x, (0, cin_p - c.in_channels))
            w = self._weight_operand(x.dtype, x.device)
            if (w.w_dtype == nat.Q8_0 and self.q8_operands == "f16" and residual is None
                    and norm_mod is None):
                # the reference's operands: f16 features, f16(f32(d) * q)
                # weights (the per-forward dequant cast before the GEMM,
                # SRC/slat_flow_graph.cpp:24-27, as one HBM pass), f16 conv
                w16 = nat.expand_q8_0(w, dtype=torch.float16)
                y16 = nat.sparse_conv(nat.convert(x, torch.float16), w16,
                                      self._bias_operand(torch.float16, x.device), idx,
                                      ntaps=self._ntaps, n_out=n_out, plan=plan)
                y = nat.convert(y16, x.dtype)
                if y.shape[1] != c.out_channels:
                    y = y[:, : c.out_channels].contiguous()
                return y
            if w.w_dtype == nat.Q8_0 and n_out >= Q8_EXPAND_MIN_ROWS:
                # the per-forward dequant cast before the GEMM
                # (SRC/slat_flow_graph.cpp:24-27) as one HBM pass
                w = nat.expand_q8_0(w)
            b = self._bias_operand(x.dtype, x.device)
            r = None if residual is None else residual.detach().to(x.dtype)
            y = nat.sparse_conv(x, w, b, idx, ntaps=self._ntaps, n_out=n_out, plan=plan,
                                residual=r, norm_mod=norm_mod, residual_rows=residual_rows)
            if y.shape[1] != c.out_channels:
                y = y[:, : c.out_channels].contiguous()
            return y

        return _run(run, feats, c.weight, c.bias)


class SparseConv3d(nn.Module, _ConvCore):
    """SparseConv3d(in_channels, out_channels, kernel_size, stride=1,
    dilation=1, padding=None, bias=True, indice_key=None)
    (SP/conv/conv_spconv.py:9-89).  Submanifold iff stride == 1 and padding
    is None."""

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, dilation=1,
                 padding=None, bias=True, indice_key=None):
        super().__init__()
        ks, st, dl = _triple(kernel_size), _triple(stride), _triple(dilation)
        subm = all(s == 1 for s in st) and padding is None
        if dl != (1, 1, 1):
            raise NotImplementedError("dilated sparse conv is not supported")
        if subm and ks == (3, 3, 3):
            kind, ntaps = "subm3", 27
        elif subm and ks == (1, 1, 1):
            kind, ntaps = "subm1", 1
        elif ks == (2, 2, 2) and st == (2, 2, 2) and padding in (None, 0, (0, 0, 0)):
            kind, ntaps = "down2", 8
        else:
            raise NotImplementedError(
                f"sparse conv kernel_size={ks} stride={st} padding={padding} is not supported "
                "(3x3x3 / 1x1x1 submanifold, 2x2x2 stride 2)")
        self.conv = _ConvParams(in_channels, out_channels, ks, st, dl, padding, bias,
                                indice_key, subm)
        self.stride = st
        self.padding = padding
        self._kind = kind
        self._init_core(ntaps, raw_view=(kind == "subm1"))

    def forward(self, x: SparseTensor) -> SparseTensor:
        return self.forward_fused(x)

    def forward_fused(self, x: SparseTensor, residual: Optional[torch.Tensor] = None,
                      norm_mod: Optional[tuple] = None,
                      residual_rows: Optional[torch.Tensor] = None) -> SparseTensor:
        """forward() with a fused epilogue on the output rows (submanifold
        convs only): `residual` [N, Cout] is added to the rounded output
        (`h = conv2(h); h = h + skip`) -- or, with `residual_rows` [N],
        residual[residual_rows[t]] from a [R, Cout] residual --
        `norm_mod` = (scale, shift, eps) with
        per-batch [B, Cout] scale / shift gives silu(norm(y) * (1 + scale)
        + shift) (structured_latent_flow.py:69-71; Cout 32, 64 or 128)."""
        spatial_changed = any(s != 1 for s in self.stride) or (self.padding is not None)
        new_shape = torch.Size([x.shape[0], self.conv.out_channels])
        scale = tuple(s * k for s, k in zip(x._scale, self.stride))
        nm = None
        if norm_mod is not None:
            sc, sh, eps = norm_mod
            nm = (sc, sh, x.coords, eps)
        if (residual is not None or nm is not None) and self._kind not in ("subm3", "subm1"):
            raise ValueError("fused epilogues apply to submanifold convs")
        if self._kind == "subm3":
            m = _subm_map(x)
            n = x.feats.shape[0]
            feats = self._conv(x.feats, m.token_major, n, _plan(x, "subm3", m.token_major, 27, n, n),
                               residual=residual, norm_mod=nm, residual_rows=residual_rows)
            data = x.data.replace_feature(feats)
        elif self._kind == "subm1":
            n = x.feats.shape[0]
            feats = self._conv(x.feats, None, n, _plan(x, "dense1", None, 1, n, n),
                               residual=residual, norm_mod=nm, residual_rows=residual_rows)
            data = x.data.replace_feature(feats)
        else:
            d = _downsample_map(x)
            feats = self._conv(x.feats, d.stride2_taps, d.nc,
                               _plan(x, "down2", d.stride2_taps, 8, d.nc, d.nf))
            spatial = [(s + 1) // 2 for s in x.data.spatial_shape]
            data = SparseTensorData(feats, d.coarse_coords, spatial, x.data.batch_size)
        out = SparseTensor(data, shape=new_shape, layout=None if spatial_changed else x.layout,
                           scale=scale, spatial_cache=x._spatial_cache)
        if self._kind == "down2":
            # what SparseInverseConv3d needs to map back to the fine rows
            out.register_spatial_cache(f"conv_{self.stride}_fine_data", x.data)
            out.register_spatial_cache(f"conv_{self.stride}_fine_layout", x.layout)
            out.register_spatial_cache(f"conv_{self.stride}_downsample_map", d)
        return out


class SparseInverseConv3d(nn.Module, _ConvCore):
    """SparseInverseConv3d(in_channels, out_channels, kernel_size, stride=1,
    dilation=1, bias=True, indice_key=None) (SP/conv/conv_spconv.py:92-139):
    the transposed 2x2x2 stride-2 conv back onto the fine rows of the
    matching SparseConv3d, y[f] = bias + W[:, k(f), :] x[coarse(f)] with
    k(f) = (x&1)*4 + (y&1)*2 + (z&1) -- spconv's inverse conv reuses the
    forward pairs and weight offsets; its own kernel was not available to
    compare against."""

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, dilation=1, bias=True,
                 indice_key=None):
        super().__init__()
        ks, st = _triple(kernel_size), _triple(stride)
        if not (ks == (2, 2, 2) and st == (2, 2, 2)):
            raise NotImplementedError("inverse sparse conv supports kernel_size 2, stride 2")
        self.conv = _ConvParams(in_channels, out_channels, ks, st, _triple(dilation), None, bias,
                                indice_key, False)
        self.stride = st
        self._init_core(8, raw_view=False)

    def forward(self, x: SparseTensor) -> SparseTensor:
        fine = x.get_spatial_cache(f"conv_{self.stride}_fine_data")
        layout = x.get_spatial_cache(f"conv_{self.stride}_fine_layout")
        d = x.get_spatial_cache(f"conv_{self.stride}_downsample_map")
        if fine is None or d is None:
            raise ValueError("SparseInverseConv3d needs the spatial cache of a stride-2 "
                             "SparseConv3d at this scale")
        taps = fine.cached(("inverse2", d.nc), lambda c: nat.stride2_inverse_taps(
            c.contiguous(), d.fine_to_coarse, d.nc))
        plan = fine.cached(("inverse2_plan", d.nc), lambda c: nat.conv_plan(
            taps, ntaps=8, n_out=d.nf, n_in=d.nc))
        feats = self._conv(x.feats, taps, d.nf, plan)
        data = SparseTensorData(feats, fine.indices, fine.spatial_shape, fine.batch_size,
                                fine.indice_dict)
        return SparseTensor(data, shape=torch.Size([x.shape[0], self.conv.out_channels]),
                            layout=layout,
                            scale=tuple(s // k for s, k in zip(x._scale, self.stride)),
                            spatial_cache=x._spatial_cache)


# ---------------------------------------------------------------------------
# spatial ops (SP/spatial.py)
# ---------------------------------------------------------------------------
class SparseLinear(nn.Linear):
    """nn.Linear over the feats of a SparseTensor (SP/linear.py:9-15)."""

    def forward(self, input: SparseTensor) -> SparseTensor:
        return input.replace(super().forward(input.feats))


def batch_offsets(x: SparseTensor) -> torch.Tensor:
    """Row offsets [B + 1] (int64, on the feature device) of the batch
    items' contiguous row ranges (the tensor's layout)."""
    lay = x.layout
    offs = [lay[0].start] + [sl.stop for sl in lay]
    for a, sl in zip(offs, lay):
        if sl.start != a:
            raise ValueError("batch items must occupy contiguous, ascending row ranges")
    return torch.tensor(offs, dtype=torch.int64).to(x.feats.device, non_blocking=True)


def max_item_rows(x: SparseTensor) -> int:
    """Rows of the largest batch item (from the layout, no device sync)."""
    return max((sl.stop - sl.start for sl in x.layout), default=0)


class SparseGroupNorm32(nn.GroupNorm):
    """GroupNorm over each batch item's rows, computed in F32 and cast back
    (SP/norm.py:15-55), on spc_group_norm_stats / spc_group_norm_silu."""

    def __init__(self, num_groups, num_channels, eps=1e-5, affine=True):
        super().__init__(num_groups, num_channels, eps, affine)

    def forward(self, input: SparseTensor) -> SparseTensor:
        return input.replace(nat.group_norm_silu(input.feats, batch_offsets(input), self.num_groups,
                                                 self.weight, self.bias, self.eps, silu=False,
                                                 max_rows=max_item_rows(input)))


class SparseSiLU(nn.SiLU):
    """SiLU on the feats (SP/nonlinearity.py:14-16)."""

    def forward(self, input: SparseTensor) -> SparseTensor:
        return input.replace(super().forward(input.feats))


def _factor3(f) -> Tuple[int, int, int]:
    return tuple(f) if isinstance(f, (list, tuple)) else (f,) * 3


class SparseDownsample(nn.Module):
    """2x mean-pool (SP/spatial.py:10-72): coarse rows in lexicographic
    (b, x/2, y/2, z/2) order; each coarse feature is the F32-divided
    deterministic sum of its children over |children| + 1 (torch
    scatter_reduce 'mean' counts the zero initial value)."""

    def __init__(self, factor: Union[int, Tuple[int, ...], List[int]]):
        super().__init__()
        self.factor = tuple(factor) if isinstance(factor, (list, tuple)) else factor

    def forward(self, input: SparseTensor) -> SparseTensor:
        factor = _factor3(self.factor)
        if factor != (2, 2, 2):
            raise NotImplementedError("SparseDownsample supports factor 2")
        d = _downsample_map(input)
        # the map's children lists give scatter_mean's values without its sort
        feats = nat.children_mean(input.feats, d.children, d.counts, d.nc)
        # The coarse level's maps are kept with the fine coordinates (a
        # block's downsample yields the same coarse coordinates every call,
        # so its convs' maps and plans are built once), and the coarse maps
        # keep the fine level's for the paired upsample.  Maps depend on the
        # coordinates only, so reusing them changes no result.
        data = SparseTensorData(feats, d.coarse_coords,
                                [(s + 1) // 2 for s in input.data.spatial_shape],
                                input.data.batch_size, input.data.cached("down2_maps", lambda c: {}))
        fine = input.data
        data.cached("up2_maps", lambda c: (fine.indice_dict, fine.spatial_shape, fine.batch_size))
        # the coarse rows' batch slices, cached like the maps (computing them
        # reads the coordinates back to the host)
        layout = data.cached("layout", lambda c: SparseTensor._batch_slices(c, input.shape[0]))
        out = SparseTensor(data, shape=input.shape, layout=layout)
        out._scale = tuple(s // f for s, f in zip(input._scale, factor))
        out._spatial_cache = input._spatial_cache
        out.register_spatial_cache(f"upsample_{factor}_coords", input.coords)
        out.register_spatial_cache(f"upsample_{factor}_layout", input.layout)
        out.register_spatial_cache(f"upsample_{factor}_idx", d.fine_to_coarse)
        return out


class SparseUpsample(nn.Module):
    """Nearest-neighbour upsample paired with SparseDownsample
    (SP/spatial.py:75-105): fine feats = coarse feats[fine_to_coarse]."""

    def __init__(self, factor: Union[int, Tuple[int, int, int], List[int]]):
        super().__init__()
        self.factor = tuple(factor) if isinstance(factor, (list, tuple)) else factor

    def forward(self, input: SparseTensor) -> SparseTensor:
        return self.fine_tensor(input, nat.gather_rows(input.feats, self.fine_rows(input)))

    def fine_rows(self, input: SparseTensor) -> torch.Tensor:
        """int32 [N_fine]: the coarse row each fine row copies."""
        idx = input.get_spatial_cache(f"upsample_{_factor3(self.factor)}_idx")
        if idx is None:
            raise ValueError("Upsample cache not found. SparseUpsample must be paired with "
                             "SparseDownsample.")
        return idx

    def fine_tensor(self, input: SparseTensor, feats: torch.Tensor) -> SparseTensor:
        """The fine-level tensor (coordinates, layout, scale and kernel maps
        of the paired downsample's input) carrying `feats` [N_fine, C]."""
        factor = _factor3(self.factor)
        coords = input.get_spatial_cache(f"upsample_{factor}_coords")
        layout = input.get_spatial_cache(f"upsample_{factor}_layout")
        if coords is None or layout is None:
            raise ValueError("Upsample cache not found. SparseUpsample must be paired with "
                             "SparseDownsample.")
        # the fine level's maps and extent, kept by the paired downsample
        # (the maps' entries check that they were built from these
        # coordinates); without them the extent is read from the coordinates
        ent = input.data.indice_dict.get("up2_maps")
        c = input.data.indices
        if ent is not None and ent[0] is c and ent[1] == c._version:
            maps, extent, n_b = ent[2]
            out = SparseTensor(SparseTensorData(feats, coords, extent, n_b, maps),
                               shape=input.shape, layout=layout)
        else:
            out = SparseTensor(feats, coords, input.shape, layout)
        out._scale = tuple(s * f for s, f in zip(input._scale, factor))
        out._spatial_cache = input._spatial_cache
        return out


class SparseSubdivide(nn.Module):
    """Every voxel -> its 8 children in torch.nonzero order, child c = dx*4 +
    dy*2 + dz at row parent*8 + c, each carrying its parent's features
    (SP/spatial.py:108-130; SRC/sparse_ops.cpp:348-371).  The output scale
    is `input._scale * 2` exactly as the reference writes it (tuple
    repetition), so spatial-cache keys match the reference's."""

    def forward(self, input: SparseTensor) -> SparseTensor:
        coords, parent = self.map(input)
        return self.assemble(input, coords, nat.gather_rows(input.feats, parent))

    @staticmethod
    def map(input: SparseTensor):
        """(child coords, parent row of every child).  Queued without a host
        synchronisation: like the reference's `coords * 2 + offset`
        (SP/spatial.py:120-124) it reports no out-of-range coordinate here;
        a map built over the children (spc_map_build, synchronous) does."""
        return nat.subdivide_map(input.coords.contiguous(), sync=False)

    @staticmethod
    def assemble(input: SparseTensor, coords: torch.Tensor, feats: torch.Tensor) -> SparseTensor:
        """The subdivided tensor with the given child features."""
        data = SparseTensorData(feats, coords, [2 * s for s in input.data.spatial_shape],
                                input.data.batch_size)
        layout = None
        if coords.shape[0] == 8 * input.coords.shape[0]:
            # no pruning: item b's children are rows 8 * (its parent rows)
            layout = [slice(8 * sl.start, 8 * sl.stop) for sl in input.layout]
        out = SparseTensor(data, shape=input.shape, layout=layout)
        out._scale = input._scale * 2
        out._spatial_cache = input._spatial_cache
        return out
