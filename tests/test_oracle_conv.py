"""Pins the oracle's F32-accumulate sparse conv (CPU).

The ggml op (PATCH:217-265) has no published outputs, so the oracle is pinned
by what the mathematics fixes:
  * identity / single-tap kernels: exact closed forms (bias-first F32 add,
    one rounding) -- a wrong tap decode or weight layout moves rows;
  * a dense torch.nn.functional.conv3d (float64, padding=1) on small grids,
    masked to the active sites: fixes o = kd*9 + kh*3 + kw, the neighbour
    direction (cross-correlation, coord + delta) and the [Cout, 27, Cin]
    weight layout;
  * conv3d(kernel 2, stride 2) for the stride-2 tap order;
  * f16 / bf16 output rounding against numpy's float16 and the bf16 bit rule.
"""
import numpy as np
import pytest
import torch

import oracle


def _dense(coords, feats, res, nb):
    c = feats.shape[1]
    d = np.zeros((nb, c, res, res, res), np.float64)
    b, x, y, z = coords.T
    d[b, :, x, y, z] = feats
    return d


def test_identity_kernel_exact(spc, orc):
    c = spc.workloads.random_voxels(400, 9, batches=2, seed=1)
    n = c.shape[0]
    tm = orc.conv_table_slat(c)
    x = spc.workloads.normal((n, 32), 1.0, seed=2)
    b = spc.workloads.normal((32,), 0.5, seed=3)
    w = np.zeros((32, 27, 32), np.float32)
    w[:, 13, :] = np.eye(32, dtype=np.float32)
    y = orc.sparse_conv(x, w, b, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32)
    assert np.array_equal(y, (b[None, :] + x).astype(np.float32))


@pytest.mark.parametrize("o", [0, 4, 13, 22, 26])
def test_single_tap_shift_exact(spc, orc, o):
    c = spc.workloads.random_voxels(500, 8, batches=2, seed=4)
    n = c.shape[0]
    tm = orc.conv_table_slat(c)
    x = spc.workloads.normal((n, 32), 1.0, seed=5)
    w = np.zeros((32, 27, 32), np.float32)
    w[:, o, :] = np.eye(32, dtype=np.float32)
    y = orc.sparse_conv(x, w, None, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32)
    nbr = tm.reshape(n, 27)[:, o]
    expect = np.where((nbr < n)[:, None], x[np.minimum(nbr, n - 1)], 0.0)
    assert np.array_equal(y, expect.astype(np.float32))
    # and the direction: the tap-o neighbour sits at coord + delta(o)
    d = np.array([o // 9 - 1, (o // 3) % 3 - 1, o % 3 - 1])
    has = nbr < n
    assert np.array_equal(c[nbr[has], 1:], c[has, 1:] + d)


def test_offset_major_equals_token_major(spc, orc):
    c = spc.workloads.random_voxels(600, 10, batches=1, seed=6)
    n = c.shape[0]
    tm = orc.conv_table_slat(c)
    om, _, _ = orc.spconv_tables(tm, n)
    x = spc.workloads.normal((n, 32), 1.0, seed=7)
    w = spc.workloads.normal((64, 27, 32), 0.1, seed=8)
    y1 = orc.sparse_conv(x, w, None, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32)
    y0 = orc.sparse_conv(x, w, None, om, ntaps=27, n_out=n, idx_layout=0, out_dtype=oracle.F32)
    assert np.array_equal(y0, y1)


def test_dense_conv3d_brute_force(spc, orc):
    res, nb, cin, cout = 9, 2, 8, 12
    c = spc.workloads.random_voxels(500, res, batches=nb, seed=9)
    n = c.shape[0]
    tm = orc.conv_table_slat(c)
    x = spc.workloads.normal((n, cin), 1.0, seed=10)
    w = spc.workloads.normal((cout, 27, cin), 0.3, seed=11)
    b = spc.workloads.normal((cout,), 0.1, seed=12)
    y = orc.sparse_conv(x, w, b, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32)
    wt = torch.from_numpy(w.astype(np.float64)).reshape(cout, 3, 3, 3, cin).permute(0, 4, 1, 2, 3)
    dense = torch.nn.functional.conv3d(torch.from_numpy(_dense(c, x, res, nb)), wt,
                                       torch.from_numpy(b.astype(np.float64)), padding=1)
    bb, xx, yy, zz = c.T
    ref = dense.numpy()[bb, :, xx, yy, zz]
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_mesh_weight_layout(spc, orc):
    """w_layout 1 ([27, Cout, Cin], the mesh GGUF layout) is the transpose."""
    c = spc.workloads.random_voxels(300, 7, batches=1, seed=13)
    n = c.shape[0]
    tm = orc.conv_table_slat(c)
    x = spc.workloads.normal((n, 16), 1.0, seed=14)
    w = spc.workloads.normal((32, 27, 16), 0.1, seed=15)
    wm = np.ascontiguousarray(w.transpose(1, 0, 2))
    y0 = orc.sparse_conv(x, w, None, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32)
    y1 = orc.sparse_conv(x, wm, None, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32,
                         w_layout=1)
    assert np.array_equal(y0, y1)


def test_stride2_dense_brute_force(spc, orc):
    res, nb, cin, cout = 10, 2, 8, 8
    c = spc.workloads.random_voxels(700, res, batches=nb, seed=16)
    n = c.shape[0]
    d = orc.downsample_map(c)
    taps = orc.stride2_taps(c, d["fine_to_coarse"], d["nc"])
    x = spc.workloads.normal((n, cin), 1.0, seed=17)
    w = spc.workloads.normal((cout, 8, cin), 0.3, seed=18)
    y = orc.sparse_conv(x, w, None, taps, ntaps=8, n_out=d["nc"], idx_layout=1,
                        out_dtype=oracle.F32)
    wt = torch.from_numpy(w.astype(np.float64)).reshape(cout, 2, 2, 2, cin).permute(0, 4, 1, 2, 3)
    dense = torch.nn.functional.conv3d(torch.from_numpy(_dense(c, x, res, nb)), wt, stride=2)
    cc = d["coarse_coords"]
    ref = dense.numpy()[cc[:, 0], :, cc[:, 1], cc[:, 2], cc[:, 3]]
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_output_rounding(spc, orc):
    c = spc.workloads.random_voxels(300, 8, batches=1, seed=19)
    n = c.shape[0]
    tm = orc.conv_table_slat(c)
    x = spc.workloads.normal((n, 32), 1.0, seed=20)
    w = spc.workloads.normal((32, 27, 32), 0.1, seed=21)
    y32 = orc.sparse_conv(x, w, None, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32)
    y16 = orc.sparse_conv(x, w, None, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F16)
    assert np.array_equal(y16, y32.astype(np.float16))
    yb = orc.sparse_conv(x, w, None, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.BF16)
    u = y32.view(np.uint32).astype(np.uint64)
    rne = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(yb, rne)


def test_thread_partition_bit_identical(spc, orc):
    """The token partition cannot change any bit (each row is independent)."""
    c = spc.workloads.random_voxels(900, 10, batches=2, seed=22)
    n = c.shape[0]
    tm = orc.conv_table_slat(c)
    x = spc.workloads.normal((n, 32), 1.0, seed=23)
    w = spc.workloads.normal((32, 27, 32), 0.1, seed=24)
    y1 = orc.sparse_conv(x, w, None, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32)
    y7 = orc.sparse_conv(x, w, None, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32,
                         nthreads=7)
    assert np.array_equal(y1, y7)


def test_f16_bf16_conversions_exhaustive(orc):
    """binary16 conversion against numpy over every finite half value and
    midpoints between neighbours (ties to even)."""
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16)
    fin = np.isfinite(f)
    f32 = f[fin].astype(np.float32)
    assert np.array_equal(orc.f32_to_f16(f32), h[fin])
    # midpoints of consecutive positive halves: numpy rounds them to even
    pos = np.sort(f[fin & (f > 0)].astype(np.float64))
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    assert np.array_equal(orc.f32_to_f16(mids).view(np.float16), mids.astype(np.float16))


@pytest.mark.parametrize("x_dt,w_dt,out_dt,w_layout,idx_layout,ntaps,cin,cout", [
    (oracle.F32, oracle.F32, oracle.F32, 0, 1, 27, 64, 96),
    (oracle.BF16, oracle.BF16, oracle.F32, 0, 1, 27, 128, 320),
    (oracle.BF16, oracle.F16, oracle.BF16, 1, 0, 27, 32, 64),
    (oracle.F16, oracle.F16, oracle.F16, 0, 0, 8, 64, 32),
    (oracle.BF16, oracle.BF16, oracle.F32, 1, 1, 1, 96, 288),
])
def test_blocked_conv_is_bit_identical(spc, orc, x_dt, w_dt, out_dt, w_layout, idx_layout,
                                       ntaps, cin, cout):
    """orc_sparse_conv_blocked reorders the loops (row and output-channel
    blocks, vectorised over output channels) without changing any output
    element's sequence of roundings: its results equal orc_sparse_conv's
    bit for bit, with missing taps, out-of-range sources, a ragged last row
    block and several thread counts."""
    wl = spc.workloads
    rng = np.random.default_rng(ntaps * 1000 + cin + cout)
    n_in, n_out = 700, 530
    idx = rng.integers(-50, n_in + 50, size=n_out * ntaps).astype(np.int32)
    idx[rng.random(idx.size) < 0.3] = n_in  # the sentinel

    def enc(a, dt):
        return {oracle.F32: lambda v: v, oracle.BF16: orc.f32_to_bf16,
                oracle.F16: orc.f32_to_f16}[dt](np.ascontiguousarray(a, np.float32))

    x = enc(wl.normal((n_in, cin), 1.0, seed=1), x_dt)
    wshape = (cout, ntaps, cin) if w_layout == 0 else (ntaps, cout, cin)
    w = enc(wl.normal(wshape, 0.05, seed=2), w_dt)
    b = enc(wl.normal((cout,), 0.1, seed=3), x_dt)
    kw = dict(ntaps=ntaps, n_out=n_out, idx_layout=idx_layout, out_dtype=out_dt, x_dtype=x_dt,
              w_dtype=w_dt, b_dtype=x_dt, w_layout=w_layout)
    ref = orc.sparse_conv(x, w, b, idx, nthreads=1, **kw)
    for th in (1, 3):
        got = orc.sparse_conv(x, w, b, idx, nthreads=th, blocked=True, **kw)
        assert got.dtype == ref.dtype
        assert np.array_equal(got.view(np.uint8), ref.view(np.uint8))
    # no bias
    kw.pop("b_dtype")
    assert np.array_equal(orc.sparse_conv(x, w, None, idx, blocked=True, **kw).view(np.uint8),
                          orc.sparse_conv(x, w, None, idx, **kw).view(np.uint8))
