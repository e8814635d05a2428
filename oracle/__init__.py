"""TEST INFRASTRUCTURE ONLY -- numpy/ctypes front end of the CPU oracle.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the timed CPU baseline.  The
HIP product path never imports it.

`orc` wraps build/liboracle_spconv.so (spconv_oracle.cpp, the restatement of
the reference's sparse-conv path); `ref` wraps _ref/libref_tables.so, the
reference's own cpp_ggml/src/sparse_ops.cpp compiled by the Makefile here
(present only where the reference tree was available at build time).
Citations for the compiled functions live in spconv_oracle.cpp; the numpy
residual-block pieces at the end of this file carry their own.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "build" / "liboracle_spconv.so"
REF_SO = HERE / "_ref" / "libref_tables.so"

F32, F16, BF16 = 0, 1, 2
OK, BAD_SHAPE, BAD_COORD, DUP_COORD = 0, 1, 2, 3

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_INT = ctypes.c_int


def build(with_ref: bool | None = None) -> None:
    """Compile the oracle (and oracle/_ref when the reference tree exists)."""
    subprocess.run(["make", "-s", "-B", "-C", str(HERE)], check=True)
    if with_ref is None:
        with_ref = Path("/root/reference/cpp_ggml/src/sparse_ops.cpp").exists()
    if with_ref:
        subprocess.run(["make", "-s", "-B", "-C", str(HERE), "ref"], check=True)


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.c_void_p)


def _dtype_code(a: np.ndarray, hint: int | None = None) -> int:
    if hint is not None:
        return hint
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    raise TypeError("uint16 arrays need an explicit dtype code (F16 or BF16)")


class _Oracle:
    def __init__(self, path: Path):
        if not path.exists():
            raise FileNotFoundError(f"{path} missing: run oracle.build()")
        lib = ctypes.CDLL(str(path))
        lib.orc_conv_table_slat.argtypes = [_P, _I64, _P]
        lib.orc_conv_table_mesh.argtypes = [_P, _I64, _I32, _P]
        lib.orc_spconv_tables.argtypes = [_P, _I64, _P, _P, _P]
        lib.orc_spconv_tables.restype = None
        lib.orc_downsample_map.argtypes = [_P, _I64, _P, _P, _P, _P]
        lib.orc_downsample_map.restype = _I64
        lib.orc_stride2_taps.argtypes = [_P, _I64, _P, _I64, _P]
        lib.orc_subdivide.argtypes = [_P, _I64, _P, _P, _P]
        lib.orc_subdivide.restype = _I64
        lib.orc_sparse_conv.argtypes = [_INT, _P, _INT, _P, _INT, _INT, _P, _INT, _P, _P, _INT,
                                        _I64, _I64, _I64, _I64, _I64, _INT]
        lib.orc_sparse_conv_blocked.argtypes = lib.orc_sparse_conv.argtypes
        lib.orc_scatter_mean.argtypes = [_INT, _P, _P, _P, _P, _I64, _I64, _I64, _INT]
        lib.orc_q8_0_quantize.argtypes = [_P, _I64, _P]
        lib.orc_q8_0_dequant.argtypes = [_P, _I64, _INT, _P]
        lib.orc_scatter_case.argtypes = [_I64, _I64, _I64, _I32, _P, _P, _P]
        lib.orc_scatter_case.restype = None
        for f in ("orc_f32_to_f16", "orc_f16_to_f32", "orc_f32_to_bf16"):
            getattr(lib, f).argtypes = [_P, _P, _I64]
            getattr(lib, f).restype = None
        self.lib = lib

    # -- maps ---------------------------------------------------------------
    def conv_table_slat(self, coords: np.ndarray) -> np.ndarray:
        c = np.ascontiguousarray(coords, dtype=np.int32)
        n = c.shape[0]
        out = np.empty(27 * n, np.int32)
        st = self.lib.orc_conv_table_slat(_ptr(c), n, _ptr(out))
        if st != OK:
            raise ValueError(f"orc_conv_table_slat status {st}")
        return out

    def conv_table_mesh(self, coords: np.ndarray, resolution: int) -> tuple[int, np.ndarray]:
        c = np.ascontiguousarray(coords, dtype=np.int32)
        n = c.shape[0]
        out = np.empty(27 * max(n, 1), np.int32)
        st = self.lib.orc_conv_table_mesh(_ptr(c), n, resolution, _ptr(out))
        return st, out[: 27 * n]

    def spconv_tables(self, token_major: np.ndarray, n: int):
        tm = np.ascontiguousarray(token_major, dtype=np.int32)
        om = np.empty(27 * n, np.int32)
        mk = np.empty(n, np.int32)
        ar = np.empty(n, np.int32)
        self.lib.orc_spconv_tables(_ptr(tm), n, _ptr(om), _ptr(mk), _ptr(ar))
        return om, mk, ar

    def downsample_map(self, coords: np.ndarray):
        c = np.ascontiguousarray(coords, dtype=np.int32)
        nf = c.shape[0]
        f2c = np.empty(nf, np.int32)
        cc = np.empty((nf, 4), np.int32)
        ch = np.empty(8 * nf, np.int32)
        cnt = np.empty(nf, np.float32)
        nc = self.lib.orc_downsample_map(_ptr(c), nf, _ptr(f2c), _ptr(cc), _ptr(ch), _ptr(cnt))
        if nc < 0:
            raise ValueError("orc_downsample_map failed")
        return dict(nc=int(nc), fine_to_coarse=f2c, coarse_coords=cc[:nc].copy(),
                    children=ch[: 8 * nc].copy(), counts=cnt[:nc].copy())

    def stride2_taps(self, coords: np.ndarray, fine_to_coarse: np.ndarray, nc: int) -> np.ndarray:
        c = np.ascontiguousarray(coords, dtype=np.int32)
        f2c = np.ascontiguousarray(fine_to_coarse, dtype=np.int32)
        taps = np.empty(8 * nc, np.int32)
        st = self.lib.orc_stride2_taps(_ptr(c), c.shape[0], _ptr(f2c), nc, _ptr(taps))
        if st != OK:
            raise ValueError(f"orc_stride2_taps status {st}")
        return taps

    def subdivide(self, coords: np.ndarray, keep: np.ndarray | None = None):
        c = np.ascontiguousarray(coords, dtype=np.int32)
        n = c.shape[0]
        k = None if keep is None else np.ascontiguousarray(keep, dtype=np.uint8)
        oc = np.empty((8 * n, 4), np.int32)
        par = np.empty(8 * n, np.int32)
        m = self.lib.orc_subdivide(_ptr(c), n, _ptr(k), _ptr(oc), _ptr(par))
        if m < 0:
            raise ValueError("orc_subdivide failed")
        return oc[:m].copy(), par[:m].copy()

    # -- feature ops ----------------------------------------------------------
    def sparse_conv(self, x, w, bias, idx, *, ntaps: int, n_out: int, idx_layout: int,
                    out_dtype: int, x_dtype: int | None = None, w_dtype: int | None = None,
                    b_dtype: int | None = None, w_layout: int = 0, nthreads: int = 1,
                    blocked: bool = False):
        """F32-accumulate sparse conv (the ggml CPU op). Returns a numpy array
        of float32 (out_dtype F32), float16 (F16) or uint16 bf16 bits (BF16).
        blocked: the vectorised restatement (bit-identical results; the
        scalar loop is the one timed as the CPU baseline)."""
        x = np.ascontiguousarray(x)
        w = np.ascontiguousarray(w)
        idx = np.ascontiguousarray(idx, dtype=np.int32)
        n_in, cin = x.shape[0], x.shape[1]
        cout = (w.size // (ntaps * cin))
        ydt = {F32: np.float32, F16: np.float16, BF16: np.uint16}[out_dtype]
        y = np.empty((n_out, cout), ydt)
        bptr = None
        bcode = 0
        if bias is not None:
            bias = np.ascontiguousarray(bias)
            bptr = _ptr(bias)
            bcode = _dtype_code(bias, b_dtype)
        fn = self.lib.orc_sparse_conv_blocked if blocked else self.lib.orc_sparse_conv
        st = fn(_dtype_code(x, x_dtype), _ptr(x), _dtype_code(w, w_dtype), _ptr(w), w_layout,
                bcode, bptr, out_dtype, _ptr(y), _ptr(idx), idx_layout, ntaps, n_out, n_in, cin,
                cout, nthreads)
        if st != OK:
            raise ValueError(f"orc_sparse_conv status {st}")
        return y

    def scatter_mean(self, features, rows, counts, nc: int, dtype: int | None = None,
                     nthreads: int = 1):
        f = np.ascontiguousarray(features)
        r = np.ascontiguousarray(rows, dtype=np.int32)
        cnt = np.ascontiguousarray(counts, dtype=np.float32)
        code = _dtype_code(f, dtype)
        out = np.empty((nc, f.shape[1]), f.dtype)
        st = self.lib.orc_scatter_mean(code, _ptr(f), _ptr(r), _ptr(cnt), _ptr(out), f.shape[1],
                                       f.shape[0], nc, nthreads)
        if st != OK:
            raise ValueError(f"orc_scatter_mean status {st}")
        return out

    def scatter_case(self, channels: int, nf: int, nc: int, seed: int):
        """Inputs of the reference scatter-mean test case (channels, nf, nc,
        seed): (f16 features [nf, channels] as uint16 bits, rows, counts)."""
        f = np.empty((nf, channels), np.uint16)
        r = np.empty(nf, np.int32)
        c = np.empty(nc, np.float32)
        self.lib.orc_scatter_case(channels, nf, nc, seed, _ptr(f), _ptr(r), _ptr(c))
        return f, r, c

    def q8_0_quantize(self, w: np.ndarray) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
        out = np.empty(w.size // 32 * 34, np.uint8)
        st = self.lib.orc_q8_0_quantize(_ptr(w), w.size, _ptr(out))
        if st != OK:
            raise ValueError("size must be a multiple of 32")
        return out

    def q8_0_dequant(self, blocks: np.ndarray, out_dtype: int = F32) -> np.ndarray:
        b = np.ascontiguousarray(blocks, dtype=np.uint8)
        nb = b.size // 34
        ydt = {F32: np.float32, F16: np.float16, BF16: np.uint16}[out_dtype]
        out = np.empty(nb * 32, ydt)
        self.lib.orc_q8_0_dequant(_ptr(b), nb, out_dtype, _ptr(out))
        return out

    def f32_to_bf16(self, a: np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.float32)
        out = np.empty(a.shape, np.uint16)
        self.lib.orc_f32_to_bf16(_ptr(a), _ptr(out), a.size)
        return out

    def f32_to_f16(self, a: np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.float32)
        out = np.empty(a.shape, np.uint16)
        self.lib.orc_f32_to_f16(_ptr(a), _ptr(out), a.size)
        return out


class _Ref:
    """The reference's own SlatTables / MeshTables, compiled from source."""

    def __init__(self, path: Path):
        if not path.exists():
            raise FileNotFoundError(f"{path} missing (reference tree not available at build)")
        lib = ctypes.CDLL(str(path))
        lib.ref_slat_tables.argtypes = [_P, _I64] + [_P] * 11
        lib.ref_slat_tables.restype = _I64
        lib.ref_mesh_tables.argtypes = [_P, _I64, _INT, _P, _P, _P, _P, _P, _P]
        self.lib = lib

    def slat_tables(self, coords: np.ndarray) -> dict:
        c = np.ascontiguousarray(coords, dtype=np.int32)
        nf = c.shape[0]
        a = lambda k: np.empty(k, np.int32)  # noqa: E731
        out = dict(conv_fine=a(27 * nf), conv_fine_spconv=a(27 * nf), fine_mask=a(nf),
                   fine_argsort=a(nf), fine_to_coarse=a(nf), coarse_children=a(8 * nf),
                   coarse_count=np.empty(nf, np.float32), conv_coarse=a(27 * nf),
                   conv_coarse_spconv=a(27 * nf), coarse_mask=a(nf), coarse_argsort=a(nf))
        order = ["conv_fine", "conv_fine_spconv", "fine_mask", "fine_argsort", "fine_to_coarse",
                 "coarse_children", "coarse_count", "conv_coarse", "conv_coarse_spconv",
                 "coarse_mask", "coarse_argsort"]
        nc = self.lib.ref_slat_tables(_ptr(c), nf, *[_ptr(out[k]) for k in order])
        if nc < 0:
            raise ValueError("SlatTables::build failed")
        out["nc"] = int(nc)
        for k, per in (("coarse_children", 8), ("coarse_count", 1), ("conv_coarse", 27),
                       ("conv_coarse_spconv", 27), ("coarse_mask", 1), ("coarse_argsort", 1)):
            out[k] = out[k][: per * nc].copy()
        return out

    def mesh_tables(self, coords: np.ndarray, base_resolution: int = 64):
        c = np.ascontiguousarray(coords, dtype=np.int32)
        sizes = np.zeros(3, np.int64)
        ok = self.lib.ref_mesh_tables(_ptr(c), c.shape[0], base_resolution, _ptr(sizes),
                                      None, None, None, None, None)
        if not ok:
            return None
        n0, n1, n2 = (int(s) for s in sizes)
        c1 = np.empty((n1, 4), np.int32)
        c2 = np.empty((n2, 4), np.int32)
        t0, t1, t2 = np.empty(27 * n0, np.int32), np.empty(27 * n1, np.int32), np.empty(27 * n2, np.int32)
        self.lib.ref_mesh_tables(_ptr(c), c.shape[0], base_resolution, _ptr(sizes), _ptr(c1),
                                 _ptr(c2), _ptr(t0), _ptr(t1), _ptr(t2))
        return dict(sizes=(n0, n1, n2), coords1=c1, coords2=c2, conv0=t0, conv1=t1, conv2=t2)


_orc = None
_ref = None


def orc() -> _Oracle:
    global _orc
    if _orc is None:
        _orc = _Oracle(ORACLE_SO)
    return _orc


def ref_available() -> bool:
    return REF_SO.exists()


def ref() -> _Ref:
    global _ref
    if _ref is None:
        _ref = _Ref(REF_SO)
    return _ref


def cpu_threads() -> int:
    """Host threads for the CPU baseline: the process's CPU affinity."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


# ---------------------------------------------------------------------------
# SLAT sparse residual block (structured_latent_flow.py:61-74), numpy.
# Pinned in tests/test_oracle_block.py against torch's CPU layer_norm / silu
# and closed forms.
# ---------------------------------------------------------------------------

def round_to(o: "_Oracle", a: np.ndarray, dtype: int) -> np.ndarray:
    """Round float32 values to the feature dtype and back (RNE)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    if dtype == F32:
        return a
    if dtype == BF16:
        return (o.f32_to_bf16(a).astype(np.uint32) << 16).view(np.float32)
    return o.f32_to_f16(a).view(np.float16).astype(np.float32)


def layernorm(a: np.ndarray, gamma=None, beta=None, eps: float = 1e-6) -> np.ndarray:
    """Row LayerNorm in F32 (torch.nn.LayerNorm as LayerNorm32 runs it,
    modules/norm.py:6-8): biased variance, eps inside the square root."""
    a = np.asarray(a, dtype=np.float32)
    mean = a.mean(axis=1, dtype=np.float64, keepdims=True)
    var = ((a - mean) ** 2).mean(axis=1, dtype=np.float64, keepdims=True)
    y = ((a - mean) / np.sqrt(var + eps)).astype(np.float32)
    if gamma is not None:
        y = y * np.asarray(gamma, np.float32)
    if beta is not None:
        y = y + np.asarray(beta, np.float32)
    return y.astype(np.float32)


def silu(a: np.ndarray) -> np.ndarray:
    """x * sigmoid(x) in F32 (F.silu)."""
    a = np.asarray(a, dtype=np.float32)
    return (a / (np.float32(1.0) + np.exp(-a))).astype(np.float32)


def res_block(o: "_Oracle", x: np.ndarray, table: np.ndarray, p: dict, scale: np.ndarray,
              shift: np.ndarray, batch: np.ndarray, dtype: int = BF16,
              nthreads: int = 1) -> np.ndarray:
    """SparseResBlock3d.forward after its up/down sampling
    (structured_latent_flow.py:61-74; io_res_block adds the sampling), every
    intermediate rounded to the feature dtype where the reference's tensors
    are:
        h = dt(silu(dt(LN(x) * g + b)));  h = dt(conv1(h))
        h = dt(silu(dt(dt(dt(LN(h)) * dt(1 + scale)) + shift)))
        out = dt(dt(conv2(h)) + skip(x)),  skip = x or dt(x W^T + b).
    x: float32 feature values (already in dtype); table: token-major
    [N*27] map; p: float32 arrays norm1_w, norm1_b, conv1_w [Co,27,Ci],
    conv1_b, conv2_w, conv2_b, optional skip_w [Co,Ci], skip_b; scale /
    shift: [B, Co] dtype values; batch: [N] batch index of each row."""
    n = x.shape[0]
    r = lambda a: round_to(o, a, dtype)  # noqa: E731

    def conv(h, w, b):
        bits = {F32: lambda a: a, BF16: o.f32_to_bf16, F16: o.f32_to_f16}[dtype]
        y = o.sparse_conv(bits(h), bits(w), bits(b), table, ntaps=27, n_out=n, idx_layout=1,
                          out_dtype=F32, x_dtype=dtype, w_dtype=dtype, b_dtype=dtype,
                          nthreads=nthreads, blocked=True)
        return r(y)

    h = r(silu(r(layernorm(x, p["norm1_w"], p["norm1_b"]))))
    h = conv(h, p["conv1_w"], p["conv1_b"])
    u = r(layernorm(h))
    m = r(r(u * r(1.0 + scale[batch])) + shift[batch])
    h = r(silu(m))
    h = conv(h, p["conv2_w"], p["conv2_b"])
    skip = x if "skip_w" not in p else r(x @ p["skip_w"].T.astype(np.float32) + p["skip_b"])
    return r(h + skip)


def io_res_block(o: "_Oracle", x: np.ndarray, coords: np.ndarray, p: dict, scale: np.ndarray,
                 shift: np.ndarray, dtype: int = BF16, mode: str | None = None,
                 fine_coords: np.ndarray | None = None, nthreads: int = 1):
    """SparseResBlock3d.forward with its sampling step (structured_latent_
    flow.py:61-65; the SLAT IO blocks built at :140-200, native graph
    SRC/slat_flow_graph.cpp:286-380, 395-396), then res_block:
      mode None    x on `coords`;
      mode "down"  x on the fine `coords` -> SparseDownsample(2): coarse rows
                   in lexicographic (b, x/2, y/2, z/2) order, each the mean
                   of its children with the sum kept in the dtype and
                   divided by |children| + 1 (orc_downsample_map +
                   orc_scatter_mean: the reference's scatter-mean op,
                   PATCH:151-215; SP/spatial.py:20-65);
      mode "up"    x on the coarse rows of `fine_coords`' downsample ->
                   SparseUpsample(2): fine row i takes coarse row
                   fine_to_coarse[i] (SP/spatial.py:75-105).
    Returns (output coords, output features)."""
    if mode == "down":
        d = o.downsample_map(coords)
        bits = {F32: lambda a: np.ascontiguousarray(a, np.float32), BF16: o.f32_to_bf16,
                F16: o.f32_to_f16}[dtype]
        xs = o.scatter_mean(bits(x), d["fine_to_coarse"], d["counts"], d["nc"], dtype=dtype,
                            nthreads=nthreads)
        if dtype == BF16:
            x = (xs.astype(np.uint32) << 16).view(np.float32)
        elif dtype == F16:
            x = xs.view(np.float16).astype(np.float32)
        else:
            x = xs
        coords = d["coarse_coords"]
    elif mode == "up":
        d = o.downsample_map(fine_coords)
        assert np.array_equal(d["coarse_coords"], coords), "x must sit on fine_coords' coarse rows"
        x = x[d["fine_to_coarse"]]
        coords = fine_coords
    elif mode is not None:
        raise ValueError(f"unknown mode {mode}")
    table = o.conv_table_slat(coords)
    out = res_block(o, x, table, p, scale, shift, coords[:, 0].astype(np.int64), dtype, nthreads)
    return coords, out


def batch_offsets(batch: np.ndarray, n_batch: int | None = None) -> np.ndarray:
    """Row offsets [B + 1] of rows sorted by batch index."""
    batch = np.asarray(batch)
    nb = int(batch.max()) + 1 if n_batch is None else n_batch
    return np.concatenate([[0], np.cumsum(np.bincount(batch, minlength=nb))]).astype(np.int64)


def group_norm_items(a: np.ndarray, offsets: np.ndarray, groups: int, gamma=None, beta=None,
                     eps: float = 1e-5) -> np.ndarray:
    """SparseGroupNorm (modules/sparse/norm.py:15-46): per batch item (rows
    offsets[b] .. offsets[b+1]), nn.GroupNorm over [1, C, rows]: each group
    of C / groups channels normalised with the mean and biased variance of
    all its values in the item, then the per-channel affine.  F32 result."""
    a = np.asarray(a, dtype=np.float32)
    out = np.zeros_like(a)
    c = a.shape[1]
    cpg = c // groups
    for b in range(len(offsets) - 1):
        blk = a[offsets[b]:offsets[b + 1]]
        if blk.shape[0] == 0:
            continue
        g = blk.reshape(blk.shape[0], groups, cpg).astype(np.float64)
        mean = g.mean(axis=(0, 2), keepdims=True)
        var = ((g - mean) ** 2).mean(axis=(0, 2), keepdims=True)
        y = ((g - mean) / np.sqrt(var + eps)).reshape(blk.shape).astype(np.float32)
        if gamma is not None:
            y = y * np.asarray(gamma, np.float32)
        if beta is not None:
            y = y + np.asarray(beta, np.float32)
        out[offsets[b]:offsets[b + 1]] = y
    return out


def subdivide_block(o: "_Oracle", x: np.ndarray, coords: np.ndarray, p: dict, groups: int,
                    dtype: int = BF16, nthreads: int = 1, blocked: bool = False,
                    rows: np.ndarray | None = None):
    """SparseSubdivideBlock3d.forward (decoder_mesh.py:69-83): h =
    dt(silu(dt(GN(x)))) gathered to the children (SparseSubdivide order,
    spatial.py:108-130), conv1, dt(silu(dt(GN))), conv2, + skip(subdivide(x))
    with skip the 1x1x1 conv (the spconv raw view W[co][ci] = buf[ci*Cout +
    co], SRC/mesh_decoder_graph.cpp:349-384) or the identity.  p: float32
    gn0_w, gn0_b, conv1_w [Co,27,Ci], conv1_b, gn1_w, gn1_b, conv2_w,
    conv2_b, optional skip_w (the [Co,1,1,1,Ci] buffer) and skip_b.
    nthreads / blocked select the conv's threads and its vectorised form
    (same values).  rows: output rows to return (conv1 and both GroupNorms
    still run over every child; conv2 and the skip only at these rows).
    Returns (child coords, features) -- features of `rows` when given."""
    r = lambda a: round_to(o, a, dtype)  # noqa: E731
    bits = {F32: lambda a: np.ascontiguousarray(a, np.float32), BF16: o.f32_to_bf16,
            F16: o.f32_to_f16}[dtype]

    def conv(h, w, b, table, ntaps, n_out):
        y = o.sparse_conv(bits(h), bits(w), bits(b), table, ntaps=ntaps, n_out=n_out,
                          idx_layout=1, out_dtype=F32, x_dtype=dtype, w_dtype=dtype, b_dtype=dtype,
                          nthreads=nthreads, blocked=blocked)
        return r(y)

    child, parent = o.subdivide(coords)
    nc = child.shape[0]
    offs_p = batch_offsets(coords[:, 0])
    h = r(silu(r(group_norm_items(x, offs_p, groups, p["gn0_w"], p["gn0_b"]))))[parent]
    table = o.conv_table_slat(child)
    h = conv(h, p["conv1_w"], p["conv1_b"], table, 27, nc)
    offs_c = batch_offsets(child[:, 0])
    h = r(silu(r(group_norm_items(h, offs_c, groups, p["gn1_w"], p["gn1_b"]))))
    out_rows = np.arange(nc) if rows is None else np.asarray(rows)
    sub = np.ascontiguousarray(table.reshape(nc, 27)[out_rows]).reshape(-1)
    h = conv(h, p["conv2_w"], p["conv2_b"], sub, 27, out_rows.shape[0])
    xs = x[parent[out_rows]]
    if "skip_w" in p:
        co, ci = p["conv2_w"].shape[0], x.shape[1]
        w_eff = p["skip_w"].reshape(-1).reshape(ci, co).T.reshape(co, 1, ci)
        ident = np.arange(xs.shape[0], dtype=np.int32)
        skip = conv(xs, w_eff, p["skip_b"], ident, 1, xs.shape[0])
    else:
        skip = xs
    return child, r(h + skip)
