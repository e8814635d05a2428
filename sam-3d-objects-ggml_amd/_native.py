"""ctypes binding of libsam3d_spconv_amd.so (the C ABI in include/).

torch supplies device memory and the current HIP stream; every compute call
goes to a hand-written HIP kernel in the library.  There is no CPU or
PyTorch fallback: if the library is missing or the tensors are not on a GPU
the call raises.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path

import torch

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libsam3d_spconv_amd.so"

F32, F16, BF16, Q8_0 = 0, 1, 2, 3
OK, BAD_SHAPE, BAD_COORD, DUP_COORD, OOM, HIP_ERROR, BAD_ARG = range(7)
MAP_MESH, MAP_SYNC = 1, 2
IDX_TOKEN_MAJOR, IDX_OFFSET_MAJOR = 0, 1
W_KRSC, W_PACKED, W_TCK, W_TKC = 0, 1, 2, 3

_STATUS_NAMES = {BAD_SHAPE: "BAD_SHAPE", BAD_COORD: "BAD_COORD", DUP_COORD: "DUP_COORD",
                 OOM: "OOM", HIP_ERROR: "HIP_ERROR", BAD_ARG: "BAD_ARG"}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_U32 = ctypes.c_uint32
_INT = ctypes.c_int
_SZ = ctypes.c_size_t

_lib = None


class SparseConvError(RuntimeError):
    """A library call returned a non-OK status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn}: {_STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


def lib() -> ctypes.CDLL:
    """Loads the HIP library (after torch, so both share torch's HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
    L = ctypes.CDLL(str(LIB_PATH))
    L.spc_last_error.restype = ctypes.c_char_p
    L.spc_status_string.restype = ctypes.c_char_p
    L.spc_status_string.argtypes = [_INT]
    L.spc_version.restype = _INT
    L.spc_map_workspace_bytes.restype = _SZ
    L.spc_map_workspace_bytes.argtypes = [_I64]
    L.spc_map_build.argtypes = [_P, _P, _I64, _I32, _U32, _P, _P, _P, _P, _P, _P, _SZ]
    L.spc_read_status.argtypes = [_P, _P]
    L.spc_downsample_workspace_bytes.restype = _SZ
    L.spc_downsample_workspace_bytes.argtypes = [_I64]
    L.spc_downsample_map.argtypes = [_P, _P, _I64, _I64, _I32, _P, _P, _P, _P, _P, _P, _P, _SZ]
    L.spc_stride2_inverse_taps.argtypes = [_P, _P, _P, _I64, _I64, _P]
    L.spc_compose_rows.argtypes = [_P, _P, _I64, _P, _I64, _P]
    L.spc_map_dense_workspace_bytes.restype = _SZ
    L.spc_map_dense_workspace_bytes.argtypes = [_I64, _I64, _I32]
    L.spc_map_build_dense.argtypes = [_P, _P, _I64, _I64, _I32, _U32, _P, _P, _P, _P, _P, _P, _SZ]
    L.spc_subdivide_neighbors.argtypes = [_P, _P, _I64, _P]
    L.spc_subdivide_tap_classes.argtypes = [_P, _P, _I64, _I64, _P, _P]
    L.spc_sparse_conv_classes.argtypes = [_P, _INT, _P, _P, _P, _P, _P, _INT, _P, _P, _I64, _I64,
                                          _I64, _I64, _I64, _I64, _I64, _P]
    L.spc_subdivide_workspace_bytes.restype = _SZ
    L.spc_subdivide_workspace_bytes.argtypes = [_I64]
    L.spc_subdivide_map.argtypes = [_P, _P, _I64, _P, _U32, _P, _P, _P, _P, _SZ]
    L.spc_sparse_conv.argtypes = [_P, _INT, _P, _INT, _INT, _P, _P, _P, _P, _P, _INT, _P, _I64,
                                  _I64, _I64, _I64, _I64]
    L.spc_sparse_conv_plan.argtypes = [_P, _INT, _P, _INT, _INT, _P, _P, _P, _P, _P, _INT, _P,
                                       _P, _I64, _I64, _I64, _I64, _I64]
    L.spc_conv_plan_bytes.restype = _SZ
    L.spc_conv_plan_bytes.argtypes = [_I64, _I64]
    L.spc_conv_plan.argtypes = [_P, _P, _INT, _P, _I64, _I64, _I64, _P, _SZ]
    L.spc_conv_plan_sections.argtypes = [_P, _P, _INT, _P, _I64, _I64, _I64, _U32, _P, _SZ]
    L.spc_conv_packed_bytes.restype = _SZ
    L.spc_conv_packed_bytes.argtypes = [_INT, _I64, _I64, _I64]
    L.spc_conv_pack_weights.argtypes = [_P, _INT, _INT, _P, _P, _I64, _I64, _I64, _P]
    L.spc_conv_expand_q8_0.argtypes = [_P, _P, _I64, _I64, _I64, _P]
    L.sam3d_spconv_f16_forward.argtypes = [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64]
    L.sam3d_spconv_f16_forward.restype = None
    L.spc_q8_0_repack.argtypes = [_P, _P, _I64, _P, _P]
    L.spc_conv_expand_q8_0_to.argtypes = [_P, _P, _I64, _I64, _I64, _INT, _P]
    L.spc_convert.argtypes = [_P, _INT, _P, _INT, _P, _I64]
    L.spc_q8_0_quantize.argtypes = [_P, _P, _I64, _P]
    L.spc_q8_0_dequant.argtypes = [_P, _P, _I64, _INT, _P]
    L.spc_scatter_mean_workspace_bytes.restype = _SZ
    L.spc_scatter_mean_workspace_bytes.argtypes = [_I64, _I64]
    L.spc_scatter_mean.argtypes = [_P, _INT, _P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ]
    L.spc_children_mean.argtypes = [_P, _INT, _P, _P, _P, _P, _I64, _I64, _I64]
    L.spc_gather_rows.argtypes = [_P, _INT, _P, _P, _P, _I64, _I64, _I64]
    L.spc_layernorm_silu.argtypes = [_P, _INT, _P, _I64, _I64, _P, _P, ctypes.c_float, _INT, _P]
    L.spc_conv_set_tile_geometry.argtypes = [_INT]
    L.spc_conv_tile_geometry.argtypes = [_INT, _INT, _I64, _I64, _I64, _I64, _I64, _INT]
    L.spc_map_build_noalloc.argtypes = [_P, _P, _I64, _I32, _U32, _P, _P, _P, _P, _P]
    L.spc_layernorm_mod_silu.argtypes = [_P, _INT, _P, _I64, _I64, ctypes.c_float, _P, _P, _P,
                                         _I64, _P]
    L.spc_group_norm_workspace_bytes.restype = _SZ
    L.spc_group_norm_workspace_bytes.argtypes = [_I64, _I64, _I64]
    L.spc_group_norm_stats.argtypes = [_P, _INT, _P, _I64, _I64, _P, _I64, _I64, ctypes.c_float,
                                       _P, _P, _SZ]
    L.spc_group_norm_silu.argtypes = [_P, _INT, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _INT,
                                      _P, _I64, _P]
    L.spc_sparse_conv_fused.argtypes = [_P, _INT, _P, _INT, _INT, _P, _P, _P, _P, _P, _INT, _P,
                                        _P, _I64, _I64, _I64, _I64, _I64,
                                        ctypes.POINTER(ConvEpilogue)]
    _lib = L
    return L


EPI_NONE, EPI_RESIDUAL, EPI_NORM_MOD_SILU = 0, 1, 2


class ConvEpilogue(ctypes.Structure):
    """spc_conv_epilogue (include/sam3d_spconv_amd.h)."""
    _fields_ = [("mode", ctypes.c_int32), ("eps", ctypes.c_float), ("residual", ctypes.c_void_p),
                ("scale", ctypes.c_void_p), ("shift", ctypes.c_void_p),
                ("coords", ctypes.c_void_p), ("n_batch", ctypes.c_int64),
                ("residual_rows", ctypes.c_void_p), ("n_residual", ctypes.c_int64)]


def _check(fn: str, status: int) -> None:
    if status != OK:
        raise SparseConvError(fn, status, lib().spc_last_error().decode(errors="replace"))


def _stream(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _need_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("sparse-conv kernels run on the GPU only; got a CPU tensor")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.float16:
        return F16
    if dt == torch.bfloat16:
        return BF16
    raise TypeError(f"unsupported feature dtype {dt}")


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------
# kernel maps
# ---------------------------------------------------------------------------
@dataclass
class SubmMap:
    """Submanifold 3x3x3 map of one coordinate set (all device tensors)."""

    n: int
    token_major: torch.Tensor   # [n*27] int32, sentinel n
    offset_major: torch.Tensor | None  # [27*n] int32, -1 missing (outputs "all")
    mask_sorted: torch.Tensor | None   # [n] int32 (outputs "all")
    argsort: torch.Tensor | None       # [n] int32 (outputs "all")
    mask_natural: torch.Tensor | None  # [n] int32 (outputs "all")
    _plan: torch.Tensor | None = None

    @property
    def pairs(self) -> int:
        return int((self.token_major < self.n).sum().item())

    def plan(self) -> torch.Tensor:
        """The conv kernel's tile plan for the token-major table (built once)."""
        if self._plan is None:
            self._plan = conv_plan(self.token_major, ntaps=27, n_out=self.n)
        return self._plan


# dense-grid map builds up to this many cells (4 bytes each)
DENSE_MAX_CELLS = 1 << 26


def map_build(coords: torch.Tensor, *, mesh_resolution: int | None = None,
              outputs: str = "all", sync: bool = True, workspace: torch.Tensor | None = None,
              dense: tuple | None = None):
    """spc_map_build on int32 [N,4] device coords.  mesh_resolution selects the
    build_mesh_conv_table semantics (range + uniqueness checks).  outputs
    "token" builds the token-major table only (no mask sort).  dense =
    (n_batch, resolution) bounds the coordinates (b < n_batch, x, y, z <
    resolution) and builds over a dense grid (spc_map_build_dense)."""
    _need_gpu(coords)
    coords = coords.contiguous()
    if coords.dtype != torch.int32 or coords.dim() != 2 or coords.shape[1] != 4:
        raise ValueError("coords must be int32 [N, 4]")
    n = coords.shape[0]
    dev = coords.device
    L = lib()
    if dense is not None:
        nb, res = int(dense[0]), int(dense[1])
        if mesh_resolution is not None and mesh_resolution != res:
            raise ValueError("dense resolution must equal mesh_resolution")
        wsb = L.spc_map_dense_workspace_bytes(n, nb, res)
    else:
        wsb = L.spc_map_workspace_bytes(n)
    ws = workspace if workspace is not None else _workspace(wsb, dev)
    e = lambda k: torch.empty(k, dtype=torch.int32, device=dev)  # noqa: E731
    tm = e(27 * n)
    full = outputs == "all"
    om = e(27 * n) if full else None
    # the mask sort runs only when its outputs are asked for
    ms, ar, mn = (e(n), e(n), e(n)) if full else (None, None, None)
    flags = (MAP_MESH if mesh_resolution is not None else 0) | (MAP_SYNC if sync else 0)
    if dense is not None:
        st = L.spc_map_build_dense(_stream(dev), _ptr(coords), n, nb, res, flags, _ptr(tm),
                                   _ptr(om), _ptr(ms), _ptr(ar), _ptr(mn), _ptr(ws), ws.numel())
        _check("spc_map_build_dense", st)
        return SubmMap(n, tm, om, ms, ar, mn)
    st = L.spc_map_build(_stream(dev), _ptr(coords), n, int(mesh_resolution or 0), flags,
                         _ptr(tm), _ptr(om), _ptr(ms), _ptr(ar), _ptr(mn), _ptr(ws), ws.numel())
    _check("spc_map_build", st)
    return SubmMap(n, tm, om, ms, ar, mn)


@dataclass
class DownsampleMap:
    nf: int
    nc: int
    fine_to_coarse: torch.Tensor  # [nf]
    coarse_coords: torch.Tensor   # [nc, 4]
    children: torch.Tensor        # [8*nc]
    counts: torch.Tensor          # [nc] float32
    stride2_taps: torch.Tensor | None  # [nc*8]


def downsample_map(coords: torch.Tensor, n_batch: int, resolution: int,
                   with_taps: bool = True) -> DownsampleMap:
    _need_gpu(coords)
    coords = coords.contiguous()
    nf = coords.shape[0]
    dev = coords.device
    L = lib()
    ws = _workspace(L.spc_downsample_workspace_bytes(nf), dev)
    f2c = torch.empty(nf, dtype=torch.int32, device=dev)
    cc = torch.empty((nf, 4), dtype=torch.int32, device=dev)
    ch = torch.empty(8 * nf, dtype=torch.int32, device=dev)
    cnt = torch.empty(nf, dtype=torch.float32, device=dev)
    taps = torch.empty(8 * nf, dtype=torch.int32, device=dev) if with_taps else None
    nc = ctypes.c_int64(0)
    st = L.spc_downsample_map(_stream(dev), _ptr(coords), nf, int(n_batch), int(resolution),
                              _ptr(f2c), _ptr(cc), _ptr(ch), _ptr(cnt), _ptr(taps),
                              ctypes.byref(nc), _ptr(ws), ws.numel())
    _check("spc_downsample_map", st)
    k = nc.value
    return DownsampleMap(nf, k, f2c, cc[:k], ch[: 8 * k], cnt[:k],
                         None if taps is None else taps[: 8 * k])


def subdivide_neighbors(parent_token_major: torch.Tensor, n_parent: int) -> SubmMap:
    """Token-major map of the children of a subdivision without pruning,
    derived from the parents' token-major table (spc_subdivide_neighbors);
    equal to map_build(child coords, outputs="token")."""
    _need_gpu(parent_token_major)
    ptm = parent_token_major.to(torch.int32).contiguous()
    if ptm.numel() != 27 * n_parent:
        raise ValueError("parent table must hold 27 * n_parent entries")
    nc = 8 * n_parent
    ctm = torch.empty(27 * nc, dtype=torch.int32, device=ptm.device)
    st = lib().spc_subdivide_neighbors(_stream(ptm.device), _ptr(ptm), n_parent, _ptr(ctm))
    _check("spc_subdivide_neighbors", st)
    return SubmMap(nc, ctm, None, None, None, None)


def subdivide_tap_classes(parent_token_major: torch.Tensor, n_parent: int):
    """(idx [64 n_parent], row_perm [8 class_rows], class_rows) of the
    merged-tap child conv (spc_subdivide_tap_classes), class_rows = n_parent
    rounded up to 256."""
    _need_gpu(parent_token_major)
    ptm = parent_token_major.to(torch.int32).contiguous()
    if ptm.numel() != 27 * n_parent:
        raise ValueError("parent table must hold 27 * n_parent entries")
    class_rows = (n_parent + 255) // 256 * 256
    idx = torch.empty(64 * n_parent, dtype=torch.int32, device=ptm.device)
    perm = torch.empty(8 * class_rows, dtype=torch.int32, device=ptm.device)
    st = lib().spc_subdivide_tap_classes(_stream(ptm.device), _ptr(ptm), n_parent, class_rows,
                                         _ptr(idx), _ptr(perm))
    _check("spc_subdivide_tap_classes", st)
    return idx, perm, class_rows


def compose_rows(idx: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    """out[i] = rows[idx[i]] for idx[i] in [0, len(rows)), else -1
    (spc_compose_rows): a neighbour table over subdivided children composed
    with their parent rows."""
    _need_gpu(idx, rows)
    idx = idx.to(torch.int32).contiguous()
    rows = rows.to(torch.int32).contiguous()
    out = torch.empty_like(idx)
    st = lib().spc_compose_rows(_stream(idx.device), _ptr(idx), idx.numel(), _ptr(rows),
                                rows.numel(), _ptr(out))
    _check("spc_compose_rows", st)
    return out


def stride2_inverse_taps(fine_coords: torch.Tensor, fine_to_coarse: torch.Tensor,
                         nc: int) -> torch.Tensor:
    """Token-major [nf*8] map of the transposed stride-2 conv (coarse -> fine)."""
    _need_gpu(fine_coords, fine_to_coarse)
    fine_coords = fine_coords.contiguous()
    f2c = fine_to_coarse.to(torch.int32).contiguous()
    nf = fine_coords.shape[0]
    taps = torch.empty(8 * nf, dtype=torch.int32, device=fine_coords.device)
    st = lib().spc_stride2_inverse_taps(_stream(fine_coords.device), _ptr(fine_coords), _ptr(f2c),
                                        nf, int(nc), _ptr(taps))
    _check("spc_stride2_inverse_taps", st)
    return taps


def subdivide_map(coords: torch.Tensor, keep: torch.Tensor | None = None, sync: bool = True):
    """Returns (child coords [m,4], parent [m]) in parent-major order.  With
    `keep` the call synchronises (the survivor count comes back) and raises
    on out-of-range coordinates; without it only when `sync` is set --
    otherwise it returns once the kernels are queued (m = 8n) and the range
    check is not reported."""
    _need_gpu(coords, keep)
    coords = coords.contiguous()
    n = coords.shape[0]
    dev = coords.device
    L = lib()
    ws = _workspace(L.spc_subdivide_workspace_bytes(n), dev)
    oc = torch.empty((8 * n, 4), dtype=torch.int32, device=dev)
    par = torch.empty(8 * n, dtype=torch.int32, device=dev)
    if keep is not None:
        keep = keep.to(torch.uint8).contiguous()
        if keep.numel() != 8 * n:
            raise ValueError("keep must have 8*n entries")
    m = ctypes.c_int64(0)
    st = L.spc_subdivide_map(_stream(dev), _ptr(coords), n, _ptr(keep), MAP_SYNC if sync else 0,
                             _ptr(oc), _ptr(par), ctypes.byref(m), _ptr(ws), ws.numel())
    _check("spc_subdivide_map", st)
    return oc[: m.value], par[: m.value]


# ---------------------------------------------------------------------------
# feature ops
# ---------------------------------------------------------------------------
@dataclass
class PackedWeights:
    """Weights in the kernel's MFMA fragment order (spc_conv_pack_weights)."""

    data: torch.Tensor  # uint8
    w_dtype: int
    ntaps: int
    cin: int
    cout: int


def pack_weights(weight: torch.Tensor, w_scale: torch.Tensor | None = None, *,
                 cin: int | None = None, cout: int | None = None, ntaps: int | None = None,
                 layout: int = W_KRSC) -> PackedWeights:
    """Weights -> the kernel's packed operand layout.  `layout` says how
    `weight` is stored: W_KRSC [Cout, ntaps, Cin], W_TCK [ntaps, Cout, Cin]
    or W_TKC [ntaps, Cin, Cout].  int8 weights are Q8_0 quants with fp16
    block scales `w_scale` (blocks along Cin)."""
    _need_gpu(weight, w_scale)
    weight = weight.contiguous()
    if weight.dtype == torch.int8:
        wdt = Q8_0
        if w_scale is None:
            raise ValueError("Q8_0 weights need w_scale")
        w_scale = w_scale.contiguous()
    else:
        wdt = dtype_code(weight.dtype)
    if weight.dim() == 3:
        a, b, c = weight.shape
        if layout == W_KRSC:
            cout, ntaps, cin = a, b, c
        elif layout == W_TCK:
            ntaps, cout, cin = a, b, c
        elif layout == W_TKC:
            ntaps, cin, cout = a, b, c
        else:
            raise ValueError(f"unknown weight layout {layout}")
    else:
        known = [v for v in (cin, cout, ntaps) if v is not None]
        if len(known) < 2:
            raise ValueError("a flat weight needs two of cin, cout, ntaps")
        if ntaps is None:
            ntaps = weight.numel() // (cin * cout)
        elif cin is None:
            cin = weight.numel() // (ntaps * cout)
        elif cout is None:
            cout = weight.numel() // (ntaps * cin)
        if ntaps * cin * cout != weight.numel():
            raise ValueError("weight size does not match ntaps * cin * cout")
    L = lib()
    nbytes = L.spc_conv_packed_bytes(wdt, ntaps, cin, cout)
    out = torch.empty(nbytes, dtype=torch.uint8, device=weight.device)
    st = L.spc_conv_pack_weights(_stream(weight.device), wdt, int(layout), _ptr(weight),
                                 _ptr(w_scale), ntaps, cin, cout, _ptr(out))
    _check("spc_conv_pack_weights", st)
    return PackedWeights(out, wdt, ntaps, cin, cout)


def expand_q8_0(packed: PackedWeights, out: torch.Tensor | None = None,
                dtype: torch.dtype = torch.bfloat16) -> PackedWeights:
    """Packed Q8_0 weights -> packed 16-bit weights (spc_conv_expand_q8_0_to):
    bf16(f32(d) * q) for dtype bfloat16 -- a bf16 conv on them is
    bit-identical to the Q8_0 conv, and faster over many row tiles (each
    weight dequantised once instead of once per tile) -- or f16(f32(d) * q)
    for float16, the reference's f16 GEMM operand.  `out` (uint8, the
    packed 16-bit size) is reused when given."""
    if packed.w_dtype != Q8_0:
        raise ValueError("expand_q8_0 takes packed Q8_0 weights")
    if dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("expand_q8_0 expands to bfloat16 or float16")
    _need_gpu(packed.data, out)
    L = lib()
    dt = dtype_code(dtype)
    nbytes = L.spc_conv_packed_bytes(dt, packed.ntaps, packed.cin, packed.cout)
    if out is None:
        out = torch.empty(nbytes, dtype=torch.uint8, device=packed.data.device)
    elif out.dtype != torch.uint8 or out.numel() < nbytes or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous uint8 tensor of >= {nbytes} bytes")
    st = L.spc_conv_expand_q8_0_to(_stream(out.device), _ptr(packed.data), packed.ntaps,
                                   packed.cin, packed.cout, dt, _ptr(out))
    _check("spc_conv_expand_q8_0_to", st)
    return PackedWeights(out, dt, packed.ntaps, packed.cin, packed.cout)


def convert(x: torch.Tensor, dtype: torch.dtype, out: torch.Tensor | None = None) -> torch.Tensor:
    """Element conversion between float32 / float16 / bfloat16 (spc_convert,
    round to nearest even)."""
    _need_gpu(x, out)
    x = x.contiguous()
    if out is None:
        out = torch.empty(x.shape, dtype=dtype, device=x.device)
    elif out.dtype != dtype or out.shape != x.shape or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of x's shape and the target dtype")
    st = lib().spc_convert(_stream(x.device), dtype_code(x.dtype), _ptr(x), dtype_code(dtype),
                           _ptr(out), x.numel())
    _check("spc_convert", st)
    return out


TILES_AUTO, TILES_WIDE, TILES_SMALL, TILES_TALL = 0, 1, 2, 3
PLAN_WIDE, PLAN_SMALL = 1, 2


def tile_geometry(dtype: torch.dtype, *, ntaps: int, n_out: int, cin: int, cout: int,
                  q8: bool = False, class_rows: int = 0, epi_mode: int = 0) -> int:
    """spc_conv_tile_geometry: the geometry (TILES_WIDE / TILES_SMALL /
    TILES_TALL) a packed-weight conv with these arguments runs now."""
    dt = dtype_code(dtype)
    return lib().spc_conv_tile_geometry(dt, Q8_0 if q8 else dt, ntaps, n_out, cin, cout,
                                        class_rows, epi_mode)


def plan_section(dtype: torch.dtype, *, ntaps: int, n_out: int, cin: int, cout: int,
                 q8: bool = False, class_rows: int = 0, epi_mode: int = 0) -> int:
    """The plan section (PLAN_WIDE / PLAN_SMALL) a packed-weight conv with
    these arguments reads: the small tiles read the small section, the wide
    and the tall tiles the wide one."""
    g = tile_geometry(dtype, ntaps=ntaps, n_out=n_out, cin=cin, cout=cout, q8=q8,
                      class_rows=class_rows, epi_mode=epi_mode)
    return PLAN_SMALL if g == TILES_SMALL else PLAN_WIDE


def set_tile_geometry(geometry: int) -> None:
    """spc_conv_set_tile_geometry: TILES_WIDE / TILES_SMALL / TILES_TALL
    force the conv kernel's tile geometry for every later conv of the
    process (where it applies); TILES_AUTO (the default) lets each conv pick
    by shape.  Results are the same."""
    _check("spc_conv_set_tile_geometry", lib().spc_conv_set_tile_geometry(int(geometry)))


def conv_plan(idx: torch.Tensor | None, *, ntaps: int, n_out: int, n_in: int | None = None,
              idx_layout: int = IDX_TOKEN_MAJOR,
              row_perm: torch.Tensor | None = None, device=None,
              sections: int = PLAN_WIDE | PLAN_SMALL) -> torch.Tensor:
    """spc_conv_plan_sections: the conv kernel's per-tile setup for this
    index table (reusable by every conv over it), for the tile geometries in
    `sections` (a conv whose geometry finds no plan sets its tiles up)."""
    _need_gpu(idx, row_perm)
    dev = idx.device if idx is not None else device
    if dev is None or torch.device(dev).type != "cuda":
        raise RuntimeError("sparse-conv kernels run on the GPU only; got a CPU tensor")
    n_in = n_out if n_in is None else n_in
    L = lib()
    nbytes = L.spc_conv_plan_bytes(n_out, ntaps)
    plan = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    st = L.spc_conv_plan_sections(_stream(dev), _ptr(idx), idx_layout, _ptr(row_perm), ntaps,
                                  n_out, n_in, int(sections), _ptr(plan), nbytes)
    _check("spc_conv_plan", st)
    return plan


def sparse_conv(x: torch.Tensor, weight, bias: torch.Tensor | None,
                idx: torch.Tensor | None, *, ntaps: int, n_out: int,
                idx_layout: int = IDX_TOKEN_MAJOR, row_perm: torch.Tensor | None = None,
                w_scale: torch.Tensor | None = None, out: torch.Tensor | None = None,
                cout: int | None = None, plan: torch.Tensor | None = None,
                residual: torch.Tensor | None = None,
                norm_mod: tuple | None = None,
                residual_rows: torch.Tensor | None = None,
                class_rows: int = 0, n_classes: int = 1) -> torch.Tensor:
    """y = conv(x) through spc_sparse_conv_fused.  `weight` is a
    PackedWeights, a [Cout, ntaps, Cin] tensor in the feature dtype, or int8
    Q8_0 quants with w_scale (fp16 block scales).  idx None with ntaps 1 is
    the identity map (the dense 1x1x1 conv).  Epilogues: `residual`
    ([n_out, Cout], feature dtype) is added to the rounded output -- with
    `residual_rows` (int32 [n_out]) residual is [R, Cout] and output row t
    adds residual[residual_rows[t]];
    `norm_mod` = (scale, shift, coords, eps) with f32 [n_batch, Cout] scale
    and shift gives silu(norm(y) * (1 + scale[b]) + shift[b]).  class_rows >
    0 selects weight classes (spc_sparse_conv_classes): `weight` is then a
    PackedWeights of n_classes * ntaps taps."""
    _need_gpu(x, bias, idx, row_perm, w_scale, residual, residual_rows)
    x = x.contiguous()
    dt = dtype_code(x.dtype)
    cin = x.shape[1]
    if isinstance(weight, PackedWeights):
        _need_gpu(weight.data)
        wdt, layout, wptr, sptr = weight.w_dtype, W_PACKED, _ptr(weight.data), None
        cout = weight.cout
        if weight.ntaps != ntaps * (n_classes if class_rows else 1) or weight.cin != cin:
            raise ValueError("packed weights do not match ntaps / cin")
    else:
        _need_gpu(weight)
        weight = weight.contiguous()
        layout = W_KRSC
        if weight.dtype == torch.int8:
            wdt = Q8_0
            if w_scale is None:
                raise ValueError("Q8_0 weights need w_scale")
            w_scale = w_scale.contiguous()
        else:
            wdt = dtype_code(weight.dtype)
        wptr, sptr = _ptr(weight), _ptr(w_scale)
        if cout is None:
            cout = weight.numel() // (ntaps * cin)
    if bias is not None:
        bias = bias.contiguous()
    if out is None:
        out = torch.empty((n_out, cout), dtype=x.dtype, device=x.device)
    epi = ConvEpilogue(EPI_NONE, 0.0, None, None, None, None, 0, None, 0)
    keep = []
    if residual is not None and norm_mod is not None:
        raise ValueError("one epilogue at a time")
    if residual is not None:
        residual = residual.contiguous()
        if residual_rows is not None:
            residual_rows = residual_rows.to(torch.int32).contiguous()
            if residual_rows.shape != (n_out,) or residual.dim() != 2 or residual.shape[1] != cout \
                    or residual.shape[0] < 1 or residual.dtype != x.dtype:
                raise ValueError("residual_rows must be int32 [n_out] and residual [R >= 1, cout] "
                                 "in the feature dtype")
            epi.residual_rows, epi.n_residual = _ptr(residual_rows), residual.shape[0]
            keep.append(residual_rows)
        elif residual.shape != (n_out, cout) or residual.dtype != x.dtype:
            raise ValueError("residual must be [n_out, cout] in the feature dtype")
        epi.mode, epi.residual = EPI_RESIDUAL, _ptr(residual)
        keep.append(residual)
    if norm_mod is not None:
        scale, shift, coords, eps = norm_mod
        _need_gpu(scale, shift, coords)
        scale = scale.to(torch.float32).contiguous()
        shift = shift.to(torch.float32).contiguous()
        coords = coords.contiguous()
        if scale.shape != shift.shape or scale.dim() != 2 or scale.shape[1] != cout:
            raise ValueError("scale / shift must be [n_batch, cout]")
        if coords.dtype != torch.int32 or coords.shape != (n_out, 4):
            raise ValueError("coords must be int32 [n_out, 4]")
        epi.mode, epi.eps = EPI_NORM_MOD_SILU, float(eps)
        epi.scale, epi.shift, epi.coords = _ptr(scale), _ptr(shift), _ptr(coords)
        epi.n_batch = scale.shape[0]
        keep += [scale, shift, coords]
    if class_rows:
        if not isinstance(weight, PackedWeights):
            raise ValueError("weight classes need PackedWeights")
        st = lib().spc_sparse_conv_classes(_stream(x.device), dt, _ptr(x), wptr, _ptr(bias),
                                           _ptr(out), _ptr(idx), idx_layout, _ptr(row_perm),
                                           _ptr(plan), ntaps, n_out, x.shape[0], cin, cout,
                                           int(class_rows), int(n_classes), ctypes.byref(epi))
        _check("spc_sparse_conv_classes", st)
        return out
    st = lib().spc_sparse_conv_fused(_stream(x.device), dt, _ptr(x), wdt, layout, wptr, sptr,
                                     _ptr(bias), _ptr(out), _ptr(idx), idx_layout, _ptr(row_perm),
                                     _ptr(plan), ntaps, n_out, x.shape[0], cin, cout,
                                     ctypes.byref(epi))
    _check("spc_sparse_conv", st)
    return out


def layernorm_silu(x: torch.Tensor, weight: torch.Tensor | None = None,
                   bias: torch.Tensor | None = None, eps: float = 1e-6, silu: bool = True,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """silu(LayerNorm32(x)) over the rows of x [n, c] (spc_layernorm_silu);
    weight / bias the optional affine parameters."""
    _need_gpu(x, weight, bias)
    x = x.contiguous()
    n, c = x.shape
    w = None if weight is None else weight.detach().to(torch.float32).contiguous()
    b = None if bias is None else bias.detach().to(torch.float32).contiguous()
    if out is None:
        out = torch.empty_like(x)
    st = lib().spc_layernorm_silu(_stream(x.device), dtype_code(x.dtype), _ptr(x), n, c, _ptr(w),
                                  _ptr(b), float(eps), int(bool(silu)), _ptr(out))
    _check("spc_layernorm_silu", st)
    return out


def layernorm_mod_silu(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                       coords: torch.Tensor, eps: float = 1e-6,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """silu(LayerNorm32(x) * (1 + scale[b]) + shift[b]) over the rows of x
    [n, c], b = coords[:, 0] (spc_layernorm_mod_silu); scale / shift
    [n_batch, c] holding feature-dtype values."""
    _need_gpu(x, scale, shift, coords)
    x = x.contiguous()
    n, c = x.shape
    scale = scale.to(torch.float32).contiguous()
    shift = shift.to(torch.float32).contiguous()
    coords = coords.contiguous()
    if scale.shape != shift.shape or scale.dim() != 2 or scale.shape[1] != c:
        raise ValueError("scale / shift must be [n_batch, c]")
    if coords.dtype != torch.int32 or coords.shape != (n, 4):
        raise ValueError("coords must be int32 [n, 4]")
    if out is None:
        out = torch.empty_like(x)
    st = lib().spc_layernorm_mod_silu(_stream(x.device), dtype_code(x.dtype), _ptr(x), n, c,
                                      float(eps), _ptr(scale), _ptr(shift), _ptr(coords),
                                      scale.shape[0], _ptr(out))
    _check("spc_layernorm_mod_silu", st)
    return out


def spconv_f16_forward(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                       indices: torch.Tensor, mask: torch.Tensor, argsort: torch.Tensor,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """The reference bridge signature sam3d_spconv_f16_forward."""
    _need_gpu(x, weight, bias, indices, mask, argsort)
    n, c = x.shape
    cout = bias.shape[0]
    if out is None:
        out = torch.empty((n, cout), dtype=torch.float16, device=x.device)
    L = lib()
    L.sam3d_spconv_f16_forward(_stream(x.device), _ptr(x), _ptr(weight), _ptr(bias), _ptr(out),
                               _ptr(indices), _ptr(mask), _ptr(argsort), n, c, cout)
    msg = L.spc_last_error().decode(errors="replace")
    return out, msg


def q8_0_repack(blocks: torch.Tensor):
    """ggml Q8_0 blocks (uint8, 34 bytes each) -> (int8 quants, fp16 scales)."""
    _need_gpu(blocks)
    blocks = blocks.contiguous()
    nb = blocks.numel() // 34
    qs = torch.empty(nb * 32, dtype=torch.int8, device=blocks.device)
    d = torch.empty(nb, dtype=torch.float16, device=blocks.device)
    st = lib().spc_q8_0_repack(_stream(blocks.device), _ptr(blocks), nb, _ptr(qs), _ptr(d))
    _check("spc_q8_0_repack", st)
    return qs, d


def q8_0_quantize(w: torch.Tensor) -> torch.Tensor:
    """float32 weights (numel % 32 == 0, blocks along the last, contiguous
    dimension) -> ggml Q8_0 blocks (uint8, 34 bytes per block)."""
    _need_gpu(w)
    w = w.to(torch.float32).contiguous()
    n = w.numel()
    out = torch.empty(n // 32 * 34, dtype=torch.uint8, device=w.device)
    st = lib().spc_q8_0_quantize(_stream(w.device), _ptr(w), n, _ptr(out))
    _check("spc_q8_0_quantize", st)
    return out


def q8_0_dequant(blocks: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """ggml Q8_0 blocks -> f32(d) * q as a flat tensor of `dtype`."""
    _need_gpu(blocks)
    blocks = blocks.contiguous()
    nb = blocks.numel() // 34
    out = torch.empty(nb * 32, dtype=dtype, device=blocks.device)
    st = lib().spc_q8_0_dequant(_stream(blocks.device), _ptr(blocks), nb, dtype_code(dtype),
                                _ptr(out))
    _check("spc_q8_0_dequant", st)
    return out


def scatter_mean(features: torch.Tensor, rows: torch.Tensor, counts: torch.Tensor,
                 nc: int) -> torch.Tensor:
    _need_gpu(features, rows, counts)
    features = features.contiguous()
    rows = rows.to(torch.int32).contiguous()
    counts = counts.to(torch.float32).contiguous()
    nf, c = features.shape
    dev = features.device
    L = lib()
    ws = _workspace(L.spc_scatter_mean_workspace_bytes(nf, nc), dev)
    out = torch.empty((nc, c), dtype=features.dtype, device=dev)
    st = L.spc_scatter_mean(_stream(dev), dtype_code(features.dtype), _ptr(features), _ptr(rows),
                            _ptr(counts), _ptr(out), c, nf, nc, _ptr(ws), ws.numel())
    _check("spc_scatter_mean", st)
    return out


def children_mean(features: torch.Tensor, children: torch.Tensor, counts: torch.Tensor,
                  nc: int) -> torch.Tensor:
    """spc_children_mean: scatter_mean's values from a downsample map's
    children lists (no sort)."""
    _need_gpu(features, children, counts)
    features = features.contiguous()
    children = children.to(torch.int32).contiguous()
    counts = counts.to(torch.float32).contiguous()
    nf, c = features.shape
    if children.numel() < 8 * nc or counts.numel() < nc:
        raise ValueError("children must hold 8 * nc entries and counts nc")
    out = torch.empty((nc, c), dtype=features.dtype, device=features.device)
    st = lib().spc_children_mean(_stream(features.device), dtype_code(features.dtype),
                                 _ptr(features), _ptr(children), _ptr(counts), _ptr(out), c, nf,
                                 nc)
    _check("spc_children_mean", st)
    return out


def gather_rows(src: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    _need_gpu(src, idx)
    src = src.contiguous()
    idx = idx.to(torch.int32).contiguous()
    n_src = src.shape[0]
    channels = 1
    for s in src.shape[1:]:
        channels *= int(s)
    out = torch.empty((idx.numel(),) + tuple(src.shape[1:]), dtype=src.dtype, device=src.device)
    st = lib().spc_gather_rows(_stream(src.device), dtype_code(src.dtype), _ptr(src), _ptr(idx),
                               _ptr(out), idx.numel(), n_src, channels)
    _check("spc_gather_rows", st)
    return out


def group_norm_silu(x: torch.Tensor, offsets: torch.Tensor, groups: int, weight=None, bias=None,
                    eps: float = 1e-5, silu: bool = True, rows: torch.Tensor | None = None,
                    max_rows: int | None = None) -> torch.Tensor:
    """silu(GroupNorm32(x)) with per-batch-item statistics (rows of item b:
    offsets[b] .. offsets[b+1], device int64), optionally gathered:
    out[i] = f(x)[rows[i]] (spc_group_norm_stats + spc_group_norm_silu)."""
    _need_gpu(x, offsets, weight, bias, rows)
    x = x.contiguous()
    n, c = x.shape
    offsets = offsets.to(torch.int64).contiguous()
    nb = offsets.numel() - 1
    if max_rows is None:
        max_rows = int((offsets[1:] - offsets[:-1]).max().item()) if nb > 0 else 0
    L = lib()
    ws = torch.empty(max(8, L.spc_group_norm_workspace_bytes(nb, max_rows, groups)), dtype=torch.uint8,
                     device=x.device)
    stats = torch.empty((nb, groups, 2), dtype=torch.float32, device=x.device)
    st = L.spc_group_norm_stats(_stream(x.device), dtype_code(x.dtype), _ptr(x), c, groups,
                                _ptr(offsets), nb, max_rows, float(eps), _ptr(stats), _ptr(ws),
                                ws.numel())
    _check("spc_group_norm_stats", st)
    w = None if weight is None else weight.detach().to(torch.float32).contiguous()
    b = None if bias is None else bias.detach().to(torch.float32).contiguous()
    if rows is not None:
        rows = rows.to(torch.int32).contiguous()
    n_out = n if rows is None else rows.numel()
    out = torch.empty((n_out, c), dtype=x.dtype, device=x.device)
    st = L.spc_group_norm_silu(_stream(x.device), dtype_code(x.dtype), _ptr(x), n, c, groups,
                               _ptr(offsets), nb, _ptr(stats), _ptr(w), _ptr(b), int(bool(silu)),
                               _ptr(rows), n_out, _ptr(out))
    _check("spc_group_norm_silu", st)
    return out
