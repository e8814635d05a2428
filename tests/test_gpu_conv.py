"""GPU sparse-conv parity against the oracle (the ggml CPU op's F32-accumulate
arithmetic, PATCH:217-265).  Tolerances: bf16 / f16 / Q8_0 max-rel
(max|a-b| / max|b|) <= 2e-2; fp32 |a-b| <= 1e-5 + 1e-4 |b|."""
import numpy as np
import pytest

from helpers import bf16_bits, check_16bit, from_dev, oracle_threads, row_subset, to_dev_bf16

pytestmark = pytest.mark.gpu

MAXREL = 2e-2
F32_RTOL, F32_ATOL = 1e-4, 1e-5


def _case(name):
    print(f"[case] {name}", flush=True)


def _bf16_inputs(spc, orc, n, cin, cout, ntaps=27, seed=0):
    wl = spc.workloads
    x = bf16_bits(orc, wl.normal((n, cin), 1.0, seed=seed + 1))
    w = bf16_bits(orc, wl.normal((cout, ntaps, cin), 0.02, seed=seed + 2))
    b = bf16_bits(orc, wl.normal((cout,), 0.01, seed=seed + 3))
    return x, w, b


def _oracle_bf16(orc, x, w, b, idx_tm, rows, ntaps, n_in):
    import oracle

    sub = row_subset(idx_tm, n_in, rows, ntaps)
    return orc.sparse_conv(x, w, b, sub, ntaps=ntaps, n_out=len(rows), idx_layout=1,
                           out_dtype=oracle.F32, x_dtype=oracle.BF16, w_dtype=oracle.BF16,
                           b_dtype=oracle.BF16, nthreads=oracle_threads(), blocked=True)


@pytest.mark.parametrize("cin,cout", [(32, 32), (64, 64), (128, 128), (32, 64), (64, 128),
                                      (128, 256), (96, 160)])
def test_bf16_channels(spc, orc, dev, cin, cout):
    import torch

    nat = spc._native
    coords = spc.workloads.random_voxels(2500, 20, batches=2, seed=cin + cout)
    n = coords.shape[0]
    _case(f"bf16 subm N={n} cin={cin} cout={cout}")
    x, w, b = _bf16_inputs(spc, orc, n, cin, cout, seed=cin)
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    wd = to_dev_bf16(w, dev)
    y = nat.sparse_conv(to_dev_bf16(x, dev), wd, to_dev_bf16(b, dev), m.token_major, ntaps=27,
                        n_out=n)
    yp = nat.sparse_conv(to_dev_bf16(x, dev), nat.pack_weights(wd), to_dev_bf16(b, dev),
                         m.token_major, ntaps=27, n_out=n)
    torch.cuda.synchronize()
    tm = m.token_major.cpu().numpy()
    rows = np.arange(n)
    ref = _oracle_bf16(orc, x, w, b, tm, rows, 27, n)
    check_16bit(f"bf16 subm {cin}->{cout}", from_dev(y), ref)
    # both weight layouts feed identical operands in identical order
    assert torch.equal(y, yp)


@pytest.mark.parametrize("ntaps,cout", [(27, 192), (8, 192), (27, 96), (8, 96)])
def test_bf16_wide_tiles(spc, orc, dev, ntaps, cout):
    """C_out = 192 / 96 with at least 256 row tiles runs the 192-column tile
    (four waves of 128x96) / the 96-column tile (eight waves of 64x48,
    weights loaded per 16-channel block; the 8-tap convs take them with the
    wide geometry forced, as the decoder's merged-tap convs do through their
    weight classes): every row against the oracle, and bit-identical to the
    unpacked-weight launch, which runs 64- / 32-column tiles."""
    import torch

    nat = spc._native
    if ntaps == 27:
        coords = spc.workloads.random_voxels(90000, 64, batches=2, seed=91)
        n = coords.shape[0]
        m = nat.map_build(torch.from_numpy(coords).to(dev))
        idx, n_out, n_in = m.token_major, n, n
    else:  # stride-2 2x2x2 onto the coarse rows
        coords = spc.workloads.random_voxels(400000, 128, batches=1, seed=92)
        d = nat.downsample_map(torch.from_numpy(coords).to(dev), 1, 128, with_taps=True)
        idx, n_out, n_in = d.stride2_taps, d.nc, coords.shape[0]
    assert n_out >= 256 * 256
    _case(f"bf16 {ntaps}-tap conv N_out={n_out} 64->{cout} ({cout}-column tiles)")
    x, w, b = _bf16_inputs(spc, orc, n_in, 64, cout, ntaps=ntaps, seed=93)
    wd = to_dev_bf16(w, dev)
    xd, bd = to_dev_bf16(x, dev), to_dev_bf16(b, dev)
    plan = nat.conv_plan(idx, ntaps=ntaps, n_out=n_out, n_in=n_in)
    pw = nat.pack_weights(wd)
    if ntaps == 8:
        nat.set_tile_geometry(nat.TILES_WIDE)
        assert nat.tile_geometry(torch.bfloat16, ntaps=8, n_out=n_out, cin=64, cout=cout) == nat.TILES_WIDE
    try:
        yp = nat.sparse_conv(xd, pw, bd, idx, ntaps=ntaps, n_out=n_out, plan=plan)
    finally:
        nat.set_tile_geometry(nat.TILES_AUTO)
    y = nat.sparse_conv(xd, wd, bd, idx, ntaps=ntaps, n_out=n_out, plan=plan)
    torch.cuda.synchronize()
    ref = _oracle_bf16(orc, x, w, b, idx.cpu().numpy(), np.arange(n_out), ntaps, n_in)
    check_16bit(f"bf16 {ntaps}-tap 64->{cout} wide tiles", from_dev(yp), ref)
    assert torch.equal(y, yp)


def test_bf16_config2_ellipsoids(spc, orc, dev):
    """4 ellipsoid shells in 64^3 (N=62,710), C=128, bf16, fp32 accumulate;
    every output row against the oracle, in natural and in mask-argsort
    processing order."""
    import torch

    nat = spc._native
    coords = spc.workloads.ellipsoid_batch()
    n = coords.shape[0]
    _case(f"bf16 config2 N={n}")
    x, w, b = _bf16_inputs(spc, orc, n, 128, 128, seed=20)
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    xd, wd, bd = to_dev_bf16(x, dev), to_dev_bf16(w, dev), to_dev_bf16(b, dev)
    y = nat.sparse_conv(xd, nat.pack_weights(wd), bd, m.token_major, ntaps=27, n_out=n)
    # the same conv in mask-argsort processing order (offset-major indices)
    y2 = nat.sparse_conv(xd, wd, bd, m.offset_major, ntaps=27, n_out=n,
                         idx_layout=nat.IDX_OFFSET_MAJOR, row_perm=m.argsort)
    torch.cuda.synchronize()
    tm = m.token_major.cpu().numpy()
    ref = _oracle_bf16(orc, x, w, b, tm, np.arange(n), 27, n)
    check_16bit("config2 bf16 C=128 natural order", from_dev(y), ref)
    check_16bit("config2 bf16 C=128 mask order", from_dev(y2), ref)


def test_bf16_single_shell_c128(spc, orc, dev):
    """The headline metric's shape: one 64^3 sphere shell (N = 21,766), bf16
    C = 128 -> 128, every row against the oracle."""
    import torch

    nat = spc._native
    coords = spc.workloads.sphere_shell()
    n = coords.shape[0]
    _case(f"bf16 single shell N={n} C=128")
    x, w, b = _bf16_inputs(spc, orc, n, 128, 128, seed=25)
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    plan = nat.conv_plan(m.token_major, ntaps=27, n_out=n)
    y = nat.sparse_conv(to_dev_bf16(x, dev), nat.pack_weights(to_dev_bf16(w, dev)),
                        to_dev_bf16(b, dev), m.token_major, ntaps=27, n_out=n, plan=plan)
    torch.cuda.synchronize()
    ref = _oracle_bf16(orc, x, w, b, m.token_major.cpu().numpy(), np.arange(n), 27, n)
    check_16bit("single shell bf16 C=128", from_dev(y), ref)


def test_f32_config1_sphere(spc, orc, dev):
    """One sphere shell in 64^3 (N=21,766) on the GPU: C=64, fp32, zero bias;
    every row within |a-b| <= 1e-5 + 1e-4 |b|."""
    import oracle
    import torch

    nat = spc._native
    wl = spc.workloads
    coords = wl.sphere_shell()
    n = coords.shape[0]
    _case(f"f32 config1 N={n}")
    x = wl.normal((n, 64), 1.0, seed=31)
    w = wl.normal((64, 27, 64), 0.02, seed=32)
    b = np.zeros(64, np.float32)
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    wd = torch.from_numpy(w).to(dev)
    y = nat.sparse_conv(torch.from_numpy(x).to(dev), nat.pack_weights(wd),
                        torch.from_numpy(b).to(dev), m.token_major, ntaps=27, n_out=n)
    y_raw = nat.sparse_conv(torch.from_numpy(x).to(dev), wd, torch.from_numpy(b).to(dev),
                            m.token_major, ntaps=27, n_out=n)
    assert torch.equal(y, y_raw)
    torch.cuda.synchronize()
    ref = orc.sparse_conv(x, w, b, m.token_major.cpu().numpy(), ntaps=27, n_out=n, idx_layout=1,
                          out_dtype=oracle.F32, nthreads=oracle_threads(), blocked=True)
    got = y.cpu().numpy()
    err = np.abs(got - ref)
    print(f"[parity] config1 f32 C=64: rows={n} max_abs={err.max():.3e} "
          f"max_rel={float(err.max() / np.abs(ref).max()):.3e}", flush=True)
    assert np.all(err <= F32_ATOL + F32_RTOL * np.abs(ref))


def test_f16_spconv_bridge(spc, orc, dev):
    """sam3d_spconv_f16_forward: offset-major indices + mask argsort."""
    import oracle
    import torch

    nat = spc._native
    wl = spc.workloads
    coords = wl.random_voxels(3000, 22, batches=2, seed=41)
    n = coords.shape[0]
    _case(f"f16 bridge N={n}")
    x = wl.normal((n, 64), 1.0, seed=42).astype(np.float16)
    w = wl.normal((128, 27, 64), 0.02, seed=43).astype(np.float16)
    b = wl.normal((128,), 0.01, seed=44).astype(np.float16)
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    xd, wd, bd = (torch.from_numpy(a).to(dev) for a in (x, w, b))
    # a failing call (cin 44 is not a multiple of 8): reported, output untouched
    bad_out = torch.full((n, 128), 7.0, dtype=torch.float16, device=dev)
    _, bad = nat.spconv_f16_forward(xd[:, :44].contiguous(), wd[:, :, :44].contiguous(), bd,
                                    m.offset_major, m.mask_sorted, m.argsort, out=bad_out)
    torch.cuda.synchronize()
    assert "unsupported shape" in bad and bool((bad_out == 7.0).all())
    # the next successful call clears the message
    y, msg = nat.spconv_f16_forward(xd, wd, bd, m.offset_major, m.mask_sorted, m.argsort)
    torch.cuda.synchronize()
    assert msg == ""
    ref = orc.sparse_conv(x, w, b, m.offset_major.cpu().numpy(), ntaps=27, n_out=n,
                          idx_layout=0, out_dtype=oracle.F32)
    check_16bit("f16 spconv bridge 64->128", y.float().cpu().numpy(), ref)
    # the bridge packs the weights and runs the packed conv: bit-identical to
    # the unpacked KRSC launch of the same conv
    y_krsc = nat.sparse_conv(xd, wd, bd, m.offset_major, ntaps=27, n_out=n,
                             idx_layout=nat.IDX_OFFSET_MAJOR)
    torch.cuda.synchronize()
    assert torch.equal(y, y_krsc)
    # the bridge's self-refreshing tile plan: a second call over the same
    # indices runs planned, a call over other indices of the same token
    # count refreshes the changed tiles, and the first indices again
    # refresh them back -- every result equal to the unplanned launch
    y2, _ = nat.spconv_f16_forward(xd, wd, bd, m.offset_major, m.mask_sorted, m.argsort)
    cb = coords.copy()
    cb[:, 1] = 21 - cb[:, 1]  # mirrored in x: same count, other neighbour tables
    cb = cb[np.lexsort((cb[:, 3], cb[:, 2], cb[:, 1], cb[:, 0]))]
    mb = nat.map_build(torch.from_numpy(np.ascontiguousarray(cb)).to(dev))
    assert not torch.equal(mb.offset_major, m.offset_major)
    yb, _ = nat.spconv_f16_forward(xd, wd, bd, mb.offset_major, mb.mask_sorted, mb.argsort)
    yb_krsc = nat.sparse_conv(xd, wd, bd, mb.offset_major, ntaps=27, n_out=n,
                              idx_layout=nat.IDX_OFFSET_MAJOR)
    # one token's centre tap dropped: only its tiles refresh
    om = m.offset_major.clone()
    om[13 * n + 17] = -1
    yc, _ = nat.spconv_f16_forward(xd, wd, bd, om, m.mask_sorted, m.argsort)
    yc_krsc = nat.sparse_conv(xd, wd, bd, om, ntaps=27, n_out=n, idx_layout=nat.IDX_OFFSET_MAJOR)
    y3, _ = nat.spconv_f16_forward(xd, wd, bd, m.offset_major, m.mask_sorted, m.argsort)
    torch.cuda.synchronize()
    assert torch.equal(y2, y_krsc)
    assert torch.equal(yb, yb_krsc)
    assert torch.equal(yc, yc_krsc) and not torch.equal(yc, y_krsc)
    assert torch.equal(y3, y_krsc)
    # two column tiles per row tile (C_out 256), and a change of tile
    # geometry over the same indices (C_in 128 runs the wide tiles, 64 the
    # small ones): each call equal to the unplanned launch
    xw = torch.from_numpy(wl.normal((n, 128), 1.0, seed=45).astype(np.float16)).to(dev)
    for cin, cout in ((64, 256), (64, 256), (128, 128), (128, 128), (64, 128)):
        _case(f"f16 bridge plan cache {cin}->{cout}")
        xi = xd if cin == 64 else xw
        wi = torch.from_numpy(wl.normal((cout, 27, cin), 0.02, seed=cin + cout)
                              .astype(np.float16)).to(dev)
        bi = torch.from_numpy(wl.normal((cout,), 0.01, seed=cout).astype(np.float16)).to(dev)
        yi, msg = nat.spconv_f16_forward(xi, wi, bi, m.offset_major, m.mask_sorted, m.argsort)
        yi_krsc = nat.sparse_conv(xi, wi, bi, m.offset_major, ntaps=27, n_out=n,
                                  idx_layout=nat.IDX_OFFSET_MAJOR)
        torch.cuda.synchronize()
        assert msg == "" and torch.equal(yi, yi_krsc)
    # the tall tiles (C_in 32, C_out <= 64) keep their plan in the wide
    # layout: planned, refreshed over other indices and over one changed
    # entry, and back -- each call equal to the unplanned launch
    x32 = torch.from_numpy(wl.normal((n, 32), 1.0, seed=46).astype(np.float16)).to(dev)
    w32 = torch.from_numpy(wl.normal((64, 27, 32), 0.02, seed=47).astype(np.float16)).to(dev)
    b32 = torch.from_numpy(wl.normal((64,), 0.01, seed=48).astype(np.float16)).to(dev)
    assert nat.tile_geometry(torch.float16, ntaps=27, n_out=n, cin=32, cout=64) == nat.TILES_TALL
    for k, om_i in enumerate((m.offset_major, m.offset_major, mb.offset_major, om, m.offset_major)):
        _case(f"f16 bridge tall tiles 32->64 call {k}")
        yt, msg = nat.spconv_f16_forward(x32, w32, b32, om_i, m.mask_sorted, m.argsort)
        yt_krsc = nat.sparse_conv(x32, w32, b32, om_i, ntaps=27, n_out=n,
                                  idx_layout=nat.IDX_OFFSET_MAJOR)
        torch.cuda.synchronize()
        assert msg == "" and torch.equal(yt, yt_krsc)


def test_f16_spconv_bridge_widths_of_8(spc, orc, dev):
    """sam3d_spconv_f16_forward at channel widths that are multiples of 8 but
    not of 32 (the reference's spconv iterators take vectors of 8 channels,
    ForwardDgradSparseIOIterator.h:58-61): zero-padded to 32 inside the
    bridge, checked against the oracle at the caller's widths and bit for
    bit against the conv of explicitly zero-padded operands."""
    import oracle
    import torch

    nat = spc._native
    wl = spc.workloads
    coords = wl.random_voxels(3000, 22, batches=2, seed=51)
    n = coords.shape[0]
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    om = m.offset_major.cpu().numpy()
    for cin, cout in ((48, 40), (40, 64), (64, 56), (8, 8), (200, 136)):
        _case(f"f16 bridge widths {cin}->{cout} N={n}")
        x = wl.normal((n, cin), 1.0, seed=cin).astype(np.float16)
        w = wl.normal((cout, 27, cin), 0.02, seed=cin + cout).astype(np.float16)
        b = wl.normal((cout,), 0.01, seed=cout).astype(np.float16)
        xd, wd, bd = (torch.from_numpy(a).to(dev) for a in (x, w, b))
        y, msg = nat.spconv_f16_forward(xd, wd, bd, m.offset_major, m.mask_sorted, m.argsort)
        torch.cuda.synchronize()
        assert msg == "", msg
        assert y.shape == (n, cout)
        ref = orc.sparse_conv(x, w, b, om, ntaps=27, n_out=n, idx_layout=0, out_dtype=oracle.F32)
        check_16bit(f"f16 bridge {cin}->{cout}", y.float().cpu().numpy(), ref)
        # the same conv over operands padded to multiples of 32 by hand
        cp, cq = (cin + 31) // 32 * 32, (cout + 31) // 32 * 32
        xp = torch.zeros(n, cp, dtype=torch.float16, device=dev)
        xp[:, :cin] = xd
        wp = torch.zeros(cq, 27, cp, dtype=torch.float16, device=dev)
        wp[:cout, :, :cin] = wd
        bp = torch.zeros(cq, dtype=torch.float16, device=dev)
        bp[:cout] = bd
        yp = nat.sparse_conv(xp, wp, bp, m.offset_major, ntaps=27, n_out=n,
                             idx_layout=nat.IDX_OFFSET_MAJOR)
        torch.cuda.synchronize()
        assert torch.equal(y, yp[:, :cout])
    # the plan cache keeps one entry per token count: calls alternating
    # between two coordinate sets stay equal to unplanned launches
    c2 = wl.random_voxels(1800, 18, batches=1, seed=52)
    m2 = nat.map_build(torch.from_numpy(c2).to(dev))
    n2 = c2.shape[0]
    x1 = torch.from_numpy(wl.normal((n, 64), 1.0, seed=53).astype(np.float16)).to(dev)
    x2 = torch.from_numpy(wl.normal((n2, 64), 1.0, seed=54).astype(np.float16)).to(dev)
    w = torch.from_numpy(wl.normal((64, 27, 64), 0.02, seed=55).astype(np.float16)).to(dev)
    b = torch.from_numpy(wl.normal((64,), 0.01, seed=56).astype(np.float16)).to(dev)
    r1 = nat.sparse_conv(x1, w, b, m.offset_major, ntaps=27, n_out=n, idx_layout=nat.IDX_OFFSET_MAJOR)
    r2 = nat.sparse_conv(x2, w, b, m2.offset_major, ntaps=27, n_out=n2, idx_layout=nat.IDX_OFFSET_MAJOR)
    for k in range(3):
        _case(f"f16 bridge alternating token counts call {k}")
        y1, msg1 = nat.spconv_f16_forward(x1, w, b, m.offset_major, m.mask_sorted, m.argsort)
        y2, msg2 = nat.spconv_f16_forward(x2, w, b, m2.offset_major, m2.mask_sorted, m2.argsort)
        torch.cuda.synchronize()
        assert msg1 == "" and msg2 == ""
        assert torch.equal(y1, r1) and torch.equal(y2, r2)


def test_q8_0_config5_sphere(spc, orc, dev):
    """Sphere shell, Q8_0 weights (C=768) dequantised inside the GEMM,
    against the reference's f16(f32(d)*q) GEMM input."""
    import oracle
    import torch

    nat = spc._native
    wl = spc.workloads
    coords = wl.sphere_shell()
    n = coords.shape[0]
    c = 768
    _case(f"q8_0 config5 N={n} C={c}")
    x = bf16_bits(orc, wl.normal((n, c), 1.0, seed=51))
    wf = wl.normal((c, 27, c), 0.02, seed=52)
    b = bf16_bits(orc, wl.normal((c,), 0.01, seed=53))
    blocks = orc.q8_0_quantize(wf)
    qs, d = nat.q8_0_repack(torch.from_numpy(blocks).to(dev))
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    y = nat.sparse_conv(to_dev_bf16(x, dev), qs, to_dev_bf16(b, dev), m.token_major, ntaps=27,
                        n_out=n, w_scale=d, cout=c)
    pw = nat.pack_weights(qs, d, cin=c, cout=c)
    yp = nat.sparse_conv(to_dev_bf16(x, dev), pw, to_dev_bf16(b, dev), m.token_major, ntaps=27,
                         n_out=n)
    # the per-forward expansion to packed bf16, then the bf16 conv: same bits
    px = nat.expand_q8_0(pw)
    yx = nat.sparse_conv(to_dev_bf16(x, dev), px, to_dev_bf16(b, dev), m.token_major, ntaps=27,
                         n_out=n)
    torch.cuda.synchronize()
    assert torch.equal(y, yp)
    assert torch.equal(y, yx)
    # the expansion is the bf16 packing of the oracle's bf16(f32(d) * q)
    wq_b = orc.q8_0_dequant(blocks, oracle.BF16).reshape(c, 27, c)
    pb = nat.pack_weights(to_dev_bf16(wq_b, dev))
    assert torch.equal(px.data, pb.data)
    tm = m.token_major.cpu().numpy()
    kw = dict(ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32, x_dtype=oracle.BF16,
              b_dtype=oracle.BF16, nthreads=oracle_threads(), blocked=True)
    got = from_dev(y)
    # the reference's GEMM input f16(f32(d) * q): the 2e-2 bar
    ref16 = orc.sparse_conv(x, orc.q8_0_dequant(blocks, oracle.F16), b, tm,
                            w_dtype=oracle.F16, **kw)
    check_16bit("config5 Q8_0 C=768 vs f16(d*q) weights", got, ref16, elementwise=False)
    # the kernel's own operands bf16(f32(d) * q): one bf16 rounding per element
    ref_b = orc.sparse_conv(x, orc.q8_0_dequant(blocks, oracle.BF16), b, tm,
                            w_dtype=oracle.BF16, **kw)
    check_16bit("config5 Q8_0 C=768 vs bf16(d*q) weights", got, ref_b)
    # the reference's operands: features cast to f16 (exact but for the
    # few below f16's full-precision range), the expansion to f16(f32(d) *
    # q), the f16 conv, the output cast back to bf16 -- per element within
    # one rounding of the f16(d*q) reference
    px16 = nat.expand_q8_0(pw, dtype=torch.float16)
    wq_h = orc.q8_0_dequant(blocks, oracle.F16).reshape(c, 27, c)
    assert torch.equal(px16.data, nat.pack_weights(torch.from_numpy(wq_h).to(dev)).data)
    xd = to_dev_bf16(x, dev)
    x16 = nat.convert(xd, torch.float16)
    inexact = x16.float() != xd.float()
    assert bool((xd.float().abs()[inexact] < 2.0 ** -17).all())
    print(f"[parity] bf16 -> f16 feature cast: {int(inexact.sum())} of {xd.numel()} values "
          "below 2^-17 rounded", flush=True)
    y16 = nat.sparse_conv(x16, px16, nat.convert(to_dev_bf16(b, dev), torch.float16),
                          m.token_major, ntaps=27, n_out=n)
    yb16 = nat.convert(y16, torch.bfloat16)
    torch.cuda.synchronize()
    check_16bit("config5 Q8_0 C=768 f16 operands vs f16(d*q) weights", from_dev(y16), ref16)
    # the cast back to bf16: round to nearest even, as torch casts
    assert torch.equal(yb16, y16.to(torch.bfloat16))
    check_16bit("config5 Q8_0 C=768 f16 operands, bf16 output", from_dev(yb16), ref16,
                roundings=2)


@pytest.mark.parametrize("ntaps,cin,cout,layout", [(27, 32, 32, "krsc"), (8, 64, 160, "krsc"),
                                                   (1, 96, 64, "tck"), (27, 64, 96, "tck")])
def test_q8_0_expand_matches_packing(spc, orc, dev, ntaps, cin, cout, layout):
    """spc_conv_expand_q8_0 of packed Q8_0 weights == the bf16 packing of
    the oracle's bf16(f32(d) * q), byte for byte (all-zero blocks
    included)."""
    import oracle
    import torch

    nat = spc._native
    _case(f"q8_0 expand ntaps={ntaps} cin={cin} cout={cout} {layout}")
    shape = (cout, ntaps, cin) if layout == "krsc" else (ntaps, cout, cin)
    wf = spc.workloads.normal(shape, 0.05, seed=ntaps + cin + cout)
    wf[0] = 0.0
    blocks = orc.q8_0_quantize(wf)
    qs, d = nat.q8_0_repack(torch.from_numpy(blocks).to(dev))
    lay = nat.W_KRSC if layout == "krsc" else nat.W_TCK
    pw = nat.pack_weights(qs, d, cin=cin, cout=cout, ntaps=ntaps, layout=lay)
    px = nat.expand_q8_0(pw)
    wq_b = orc.q8_0_dequant(blocks, oracle.BF16).reshape(shape)
    pb = nat.pack_weights(to_dev_bf16(wq_b, dev), layout=lay)
    torch.cuda.synchronize()
    assert px.data.numel() == pb.data.numel()
    assert torch.equal(px.data, pb.data)


def test_stride2_conv(spc, orc, dev):
    """The SLAT IO block's first stage: 2x2x2 stride-2 conv 64^3 -> 32^3."""
    import torch

    nat = spc._native
    coords = spc.workloads.ellipsoid_batch()
    nf = coords.shape[0]
    _case(f"stride2 conv nf={nf}")
    d = nat.downsample_map(torch.from_numpy(coords).to(dev), 4, 64)
    x, w, b = _bf16_inputs(spc, orc, nf, 128, 128, ntaps=8, seed=60)
    wd = to_dev_bf16(w, dev)
    y = nat.sparse_conv(to_dev_bf16(x, dev), nat.pack_weights(wd), to_dev_bf16(b, dev),
                        d.stride2_taps, ntaps=8, n_out=d.nc)
    y_raw = nat.sparse_conv(to_dev_bf16(x, dev), wd, to_dev_bf16(b, dev), d.stride2_taps,
                            ntaps=8, n_out=d.nc)
    assert torch.equal(y, y_raw)
    torch.cuda.synchronize()
    taps = d.stride2_taps.cpu().numpy()
    ref = _oracle_bf16(orc, x, w, b, taps, np.arange(d.nc), 8, nf)
    check_16bit("config3 stride-2 2x2x2 128->128", from_dev(y), ref)


def test_empty_and_missing(spc, orc, dev):
    """n_out = 0 is a no-op; an all-missing row yields exactly the bias."""
    import torch

    nat = spc._native
    _case("empty and isolated rows")
    x = torch.zeros((0, 32), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((32, 27, 32), dtype=torch.bfloat16, device=dev)
    idx = torch.zeros(0, dtype=torch.int32, device=dev)
    y = nat.sparse_conv(x, w, None, idx, ntaps=27, n_out=0)
    assert y.shape == (0, 32)
    # rows whose every tap is the sentinel: output = bias
    n = 5
    xb = torch.randn((n, 32), device=dev).to(torch.bfloat16)
    wb = torch.randn((32, 27, 32), device=dev).to(torch.bfloat16)
    bb = torch.randn(32, device=dev).to(torch.bfloat16)
    idx = torch.full((n * 27,), n, dtype=torch.int32, device=dev)
    y = nat.sparse_conv(xb, wb, bb, idx, ntaps=27, n_out=n)
    torch.cuda.synchronize()
    assert torch.equal(y, bb.unsqueeze(0).expand(n, 32))


def _two_slabs():
    """x in {0, 1}, y in [0, 2048), z in [0, 16): a tile's x + 1 neighbours
    lie 32768 rows away, beyond the setup's bitmap window."""
    g = np.stack(np.meshgrid([0], [0, 1], np.arange(2048), np.arange(16), indexing="ij"), -1)
    return np.ascontiguousarray(g.reshape(-1, 4), dtype=np.int32)


def test_wide_span_tiles_stay_on_the_fast_path(spc, orc, dev):
    """Tiles whose source rows span more than the 32768-row bitmap window are
    deduplicated by the hash path: every tile keeps the staged fast path
    (plan header), results match the oracle, and the plan and the in-kernel
    setup agree bit-exactly."""
    import torch

    nat = spc._native
    coords = _two_slabs()
    n = coords.shape[0]
    _case(f"wide-span tiles N={n} bf16 32->32")
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    plan = nat.conv_plan(m.token_major, ntaps=27, n_out=n)
    # the plan's first section: one 19,200-byte plan per 256-row tile
    tiles = (n + 255) // 256
    wide_tile = (64 + 4 * 256 + 4 * 896 + 2 * 28 * 256 + 255) // 256 * 256
    hdr = plan[: tiles * wide_tile].view(torch.int32).cpu().numpy().reshape(tiles, -1)
    assert (hdr[:, 2] == 1).all() and (hdr[:, 0] <= 895).all()
    tm = m.token_major.cpu().numpy().reshape(n, 27)
    span = np.where(tm < n, tm, -1).max(1).max() - np.where(tm < n, tm, n).min(1).min()
    assert span > 32768
    x, w, b = _bf16_inputs(spc, orc, n, 32, 32, seed=97)
    args = (to_dev_bf16(x, dev), nat.pack_weights(to_dev_bf16(w, dev)), to_dev_bf16(b, dev),
            m.token_major)
    y = nat.sparse_conv(*args, ntaps=27, n_out=n, plan=plan)
    y0 = nat.sparse_conv(*args, ntaps=27, n_out=n)
    torch.cuda.synchronize()
    assert torch.equal(y, y0)
    ref = _oracle_bf16(orc, x, w, b, m.token_major.cpu().numpy(), np.arange(n), 27, n)
    check_16bit("wide-span tiles bf16 32->32", from_dev(y), ref)


@pytest.mark.parametrize("case", ["bf16_natural", "bf16_mask_order", "f32", "q8_0", "stride2",
                                  "dense1", "fallback_unsorted"])
def test_plan_matches_in_kernel_setup(spc, orc, dev, case):
    """spc_sparse_conv_plan with a plan from spc_conv_plan computes exactly
    what spc_sparse_conv computes with its in-kernel tile setup."""
    import torch

    nat = spc._native
    wl = spc.workloads
    _case(f"plan vs in-kernel setup: {case}")
    if case == "fallback_unsorted":
        # shell rows in random order: a tile's 256 rows reference ~5000
        # distinct rows, beyond the 1024-row stage -- the fallback path
        coords = wl.ellipsoid_batch(2, seed=72)
        coords = np.ascontiguousarray(coords[np.random.default_rng(71).permutation(len(coords))])
    else:
        coords = wl.ellipsoid_batch(2, seed=72)
    n = coords.shape[0]
    c_dev = torch.from_numpy(coords).to(dev)
    cin, cout, ntaps, n_out, n_in = 64, 128, 27, n, n
    idx_layout, perm = nat.IDX_TOKEN_MAJOR, None
    if case == "stride2":
        d = nat.downsample_map(c_dev, 2, 64)
        idx, ntaps, n_out = d.stride2_taps, 8, d.nc
    elif case == "dense1":
        idx, ntaps = None, 1
    else:
        m = nat.map_build(c_dev)
        idx = m.token_major
        if case == "bf16_mask_order":
            idx, idx_layout, perm = m.offset_major, nat.IDX_OFFSET_MAJOR, m.argsort
    g = torch.Generator(device="cpu").manual_seed(7)
    dt = torch.float32 if case == "f32" else torch.bfloat16
    x = torch.randn((n_in, cin), generator=g).to(dev, dt)
    b = (torch.randn(cout, generator=g) * 0.1).to(dev, dt)
    if case == "q8_0":
        blocks = nat.q8_0_quantize((torch.randn((cout, ntaps, cin), generator=g) * 0.02).to(dev))
        qs, dsc = nat.q8_0_repack(blocks)
        w = nat.pack_weights(qs, dsc, cin=cin, cout=cout, ntaps=ntaps)
    else:
        w = nat.pack_weights((torch.randn((cout, ntaps, cin), generator=g) * 0.02).to(dev, dt))
    plan = nat.conv_plan(idx, ntaps=ntaps, n_out=n_out, n_in=n_in, idx_layout=idx_layout,
                         row_perm=perm, device=dev)
    y0 = nat.sparse_conv(x, w, b, idx, ntaps=ntaps, n_out=n_out, idx_layout=idx_layout,
                         row_perm=perm)
    y1 = nat.sparse_conv(x, w, b, idx, ntaps=ntaps, n_out=n_out, idx_layout=idx_layout,
                         row_perm=perm, plan=plan)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    assert torch.isfinite(y1.float()).all()


@pytest.mark.parametrize("case,n_obj,cin,cout", [("bf16", 5, 64, 192), ("bf16", 2, 128, 128),
                                                 ("f32", 2, 32, 64), ("q8_0", 2, 64, 128)])
def test_fallback_tiles_match_fast_tiles(spc, orc, dev, case, n_obj, cin, cout):
    """Rows in random order put each tile's 256 rows over thousands of
    distinct source rows, beyond the stage: every tile takes the fallback,
    which stages up to 7 taps' rows per round with 8 waves (3 with the
    4-wave 192-column and Q8_0 tiles).  A row accumulates the same steps in
    the same order on both paths (chunks outer, taps ascending; absent taps
    add exact zeros), so the shuffled conv equals the sorted conv row for
    row, bit for bit; every row of the sorted conv matches the oracle."""
    import oracle
    import torch

    nat = spc._native
    wl = spc.workloads
    coords = wl.ellipsoid_batch(n_obj, seed=73)
    n = coords.shape[0]
    _case(f"fallback vs fast tiles: {case} N={n} {cin}->{cout}")
    perm = np.random.default_rng(74).permutation(n)
    wf = wl.normal((cout, 27, cin), 0.02, seed=76)
    if case == "f32":
        x, w, b = wl.normal((n, cin), 1.0, seed=75), wf, wl.normal((cout,), 0.01, seed=77)
        to_dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        pw = nat.pack_weights(to_dev(w))
    else:
        x = bf16_bits(orc, wl.normal((n, cin), 1.0, seed=75))
        b = bf16_bits(orc, wl.normal((cout,), 0.01, seed=77))
        to_dev = lambda a: to_dev_bf16(np.ascontiguousarray(a), dev)  # noqa: E731
        if case == "q8_0":
            blocks = orc.q8_0_quantize(wf)
            qs, dsc = nat.q8_0_repack(torch.from_numpy(blocks).to(dev))
            pw = nat.pack_weights(qs, dsc, cin=cin, cout=cout)
            w = orc.q8_0_dequant(blocks, oracle.F16)
        else:
            w = bf16_bits(orc, wf)
            pw = nat.pack_weights(to_dev(w))
    bd = to_dev(b)

    def conv(c, xx):
        m = nat.map_build(torch.from_numpy(np.ascontiguousarray(c)).to(dev))
        return nat.sparse_conv(to_dev(xx), pw, bd, m.token_major, ntaps=27, n_out=len(c)), m

    y0, m0 = conv(coords, x)
    y1, _ = conv(coords[perm], x[perm])
    torch.cuda.synchronize()
    assert torch.equal(y1, y0[torch.from_numpy(perm).to(dev)])
    tm0 = m0.token_major.cpu().numpy()
    if case == "f32":
        ref = orc.sparse_conv(x, w, b, tm0, ntaps=27, n_out=n, idx_layout=1,
                              out_dtype=oracle.F32, nthreads=oracle_threads(), blocked=True)
        got = y0.cpu().numpy()
        assert np.all(np.abs(got - ref) <= F32_ATOL + F32_RTOL * np.abs(ref))
    else:
        ref = orc.sparse_conv(x, w, b, tm0, ntaps=27, n_out=n, idx_layout=1,
                              out_dtype=oracle.F32, x_dtype=oracle.BF16,
                              w_dtype=oracle.F16 if case == "q8_0" else oracle.BF16,
                              b_dtype=oracle.BF16, nthreads=oracle_threads(), blocked=True)
        check_16bit(f"fallback vs fast tiles {case} {cin}->{cout}", from_dev(y0), ref,
                    elementwise=case != "q8_0")
