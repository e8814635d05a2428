"""GPU tests of the operator surface (sparse.py / tables.py) against the oracle
and, where the semantics are the reference's Python (spconv) ones, against
dense torch brute force.  Bars: maps / coords / scatter-mean bit-exact; f32
|a-b| <= 1e-5 + 1e-4|b|; bf16 / Q8_0 max-rel <= 2e-2."""
import numpy as np
import pytest

from helpers import bf16_bits, check_16bit, from_dev, max_rel

pytestmark = pytest.mark.gpu

MAXREL = 2e-2
F32_RTOL, F32_ATOL = 1e-4, 1e-5


def _case(name):
    print(f"[case] {name}", flush=True)


def _sp(spc):
    return spc.sparse


def _tensor(spc, coords, feats, dev):
    import torch

    return _sp(spc).SparseTensor(torch.from_numpy(feats).to(dev),
                                 torch.from_numpy(coords).to(dev))


def _oracle_conv(orc, x, w_krsc, b, idx_tm, ntaps, n_out, dt):
    import oracle

    return orc.sparse_conv(x, w_krsc, b, idx_tm, ntaps=ntaps, n_out=n_out, idx_layout=1,
                           out_dtype=oracle.F32, x_dtype=dt, w_dtype=dt, b_dtype=dt)


def _close_f32(y, ref):
    np.testing.assert_allclose(y, ref, rtol=F32_RTOL, atol=F32_ATOL)


# ---------------------------------------------------------------------------
# SparseConv3d
# ---------------------------------------------------------------------------
def test_subm3_f32_module(spc, orc, dev):
    import torch

    coords = spc.workloads.random_voxels(3000, 18, batches=2, seed=21)
    n = coords.shape[0]
    _case(f"SparseConv3d subm3 f32 N={n} 64->96")
    x = spc.workloads.normal((n, 64), 1.0, seed=1)
    conv = _sp(spc).SparseConv3d(64, 96, 3).to(dev)
    with torch.no_grad():
        out = conv(_tensor(spc, coords, x, dev))
    assert out.shape == torch.Size([2, 96])
    assert torch.equal(out.coords.cpu(), torch.from_numpy(coords))
    w = conv.conv.weight.detach().cpu().numpy().reshape(96, 27, 64)
    b = conv.conv.bias.detach().cpu().numpy()
    ref = _oracle_conv(orc, x, w, b, orc.conv_table_slat(coords), 27, n, 0)
    _close_f32(out.feats.cpu().numpy(), ref)


def test_subm3_bf16_module_map_cached(spc, orc, dev):
    import oracle
    import torch

    coords = spc.workloads.ellipsoid_batch(2, seed=5)
    n = coords.shape[0]
    _case(f"SparseConv3d subm3 bf16 N={n} 128->128, two convs one map")
    xf = spc.workloads.normal((n, 128), 1.0, seed=2)
    xb = bf16_bits(orc, xf)
    sp = _sp(spc)
    c1 = sp.SparseConv3d(128, 128, 3).to(dev, torch.bfloat16)
    c2 = sp.SparseConv3d(128, 128, 3).to(dev, torch.bfloat16)
    xt = sp.SparseTensor(torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16),
                         torch.from_numpy(coords).to(dev))
    with torch.no_grad():
        h = c1(xt)
        y = c2(h)
    # the second conv reuses the first conv's map (same coordinate tensor)
    assert len(xt.data.indice_dict) == 2 and h.data.indice_dict is xt.data.indice_dict  # map + plan
    tm = orc.conv_table_slat(coords)
    w1 = bf16_bits(orc, c1.conv.weight.detach().float().cpu().numpy().reshape(128, 27, 128))
    b1 = bf16_bits(orc, c1.conv.bias.detach().float().cpu().numpy())
    ref = _oracle_conv(orc, xb, w1, b1, tm, 27, n, oracle.BF16)
    err = max_rel(from_dev(h.feats), ref)
    assert err <= MAXREL, err
    assert y.feats.shape == (n, 128) and y.layout == xt.layout


def test_subm1_raw_view(spc, orc, dev):
    """1x1x1: the saved [Cout,1,1,1,Cin] buffer is read as (Cin, Cout)
    (SRC/mesh_decoder_graph.cpp:349-376); Cin != Cout so a transposed
    reading fails."""
    import torch

    coords = spc.workloads.random_voxels(1500, 14, batches=1, seed=3)
    n = coords.shape[0]
    _case(f"SparseConv3d 1x1x1 f32 N={n} 64->96")
    x = spc.workloads.normal((n, 64), 1.0, seed=4)
    conv = _sp(spc).SparseConv3d(64, 96, 1).to(dev)
    with torch.no_grad():
        out = conv(_tensor(spc, coords, x, dev))
    buf = conv.conv.weight.detach().cpu().numpy().reshape(-1)
    w_eff = np.ascontiguousarray(buf.reshape(64, 96).T).reshape(96, 1, 64)
    b = conv.conv.bias.detach().cpu().numpy()
    ref = _oracle_conv(orc, x, w_eff, b, np.arange(n, dtype=np.int32), 1, n, 0)
    _close_f32(out.feats.cpu().numpy(), ref)
    # and the plain reading is measurably different
    w_plain = buf.reshape(96, 1, 64)
    other = _oracle_conv(orc, x, w_plain, b, np.arange(n, dtype=np.int32), 1, n, 0)
    assert np.abs(other - ref).max() > 1e-2


def test_subm3_unpadded_channels(spc, orc, dev):
    import torch

    coords = spc.workloads.random_voxels(900, 12, batches=2, seed=8)
    n = coords.shape[0]
    _case(f"SparseConv3d subm3 f32 N={n} 8->40 (zero-padded channels)")
    x = spc.workloads.normal((n, 8), 1.0, seed=9)
    conv = _sp(spc).SparseConv3d(8, 40, 3).to(dev)
    with torch.no_grad():
        out = conv(_tensor(spc, coords, x, dev))
    w = conv.conv.weight.detach().cpu().numpy().reshape(40, 27, 8)
    b = conv.conv.bias.detach().cpu().numpy()
    ref = _oracle_conv(orc, x, w, b, orc.conv_table_slat(coords), 27, n, 0)
    _close_f32(out.feats.cpu().numpy(), ref)


def test_stride2_module(spc, orc, dev):
    import oracle
    import torch

    coords = spc.workloads.ellipsoid_batch(3, seed=11)
    n = coords.shape[0]
    _case(f"SparseConv3d k2 s2 bf16 N={n} 64->96")
    xb = bf16_bits(orc, spc.workloads.normal((n, 64), 1.0, seed=5))
    sp = _sp(spc)
    conv = sp.SparseConv3d(64, 96, 2, stride=2).to(dev, torch.bfloat16)
    xt = sp.SparseTensor(torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16),
                         torch.from_numpy(coords).to(dev))
    with torch.no_grad():
        out = conv(xt)
    d = orc.downsample_map(coords)
    assert np.array_equal(out.coords.cpu().numpy(), d["coarse_coords"])
    assert out.shape == torch.Size([3, 96]) and out._scale == (2, 2, 2)
    taps = orc.stride2_taps(coords, d["fine_to_coarse"], d["nc"])
    w = bf16_bits(orc, conv.conv.weight.detach().float().cpu().numpy().reshape(96, 8, 64))
    b = bf16_bits(orc, conv.conv.bias.detach().float().cpu().numpy())
    ref = _oracle_conv(orc, xb, w, b, taps, 8, d["nc"], oracle.BF16)
    assert max_rel(from_dev(out.feats), ref) <= MAXREL
    # batch rows stay contiguous
    cb = out.coords[:, 0].cpu().numpy()
    assert np.all(np.diff(cb) >= 0)
    for i, sl in enumerate(out.layout):
        assert np.all(cb[sl] == i)


def test_inverse_conv_dense_brute_force(spc, dev):
    """SparseInverseConv3d after a stride-2 conv, against torch
    conv_transpose3d on the dense grid, sampled at the fine voxels."""
    import torch
    import torch.nn.functional as F

    coords = spc.workloads.random_voxels(700, 12, batches=2, seed=13)
    n = coords.shape[0]
    _case(f"SparseInverseConv3d k2 s2 f32 N={n} 32->64->32")
    sp = _sp(spc)
    x = spc.workloads.normal((n, 32), 1.0, seed=6)
    down = sp.SparseConv3d(32, 64, 2, stride=2).to(dev)
    up = sp.SparseInverseConv3d(64, 32, 2, stride=2).to(dev)
    with torch.no_grad():
        h = down(_tensor(spc, coords, x, dev))
        y = up(h)
    assert torch.equal(y.coords.cpu(), torch.from_numpy(coords))
    assert y._scale == (1, 1, 1) and y.shape == torch.Size([2, 32])
    hc = h.coords.cpu().long()
    H = torch.zeros(2, 64, 6, 6, 6)
    H[hc[:, 0], :, hc[:, 1], hc[:, 2], hc[:, 3]] = h.feats.cpu()
    W = up.conv.weight.detach().cpu()             # [co, 2, 2, 2, ci]
    dense = F.conv_transpose3d(H, W.permute(4, 0, 1, 2, 3).contiguous(), stride=2)
    c = torch.from_numpy(coords).long()
    ref = dense[c[:, 0], :, c[:, 1], c[:, 2], c[:, 3]] + up.conv.bias.detach().cpu()
    _close_f32(y.feats.cpu().numpy(), ref.numpy())


def test_q8_0_module(spc, orc, dev):
    import oracle
    import torch

    coords = spc.workloads.random_voxels(2500, 18, batches=1, seed=17)
    n = coords.shape[0]
    _case(f"SparseConv3d Q8_0 bf16 N={n} 64->64 (slat and mesh layouts)")
    sp = _sp(spc)
    xb = bf16_bits(orc, spc.workloads.normal((n, 64), 1.0, seed=7))
    conv = sp.SparseConv3d(64, 64, 3).to(dev)
    w32 = conv.conv.weight.detach().cpu().numpy().reshape(64, 27, 64)
    blocks = conv.quantize_q8_0("slat").cpu().numpy()
    assert np.array_equal(blocks, orc.q8_0_quantize(w32))  # converter recipe, bit-exact
    conv = conv.to(torch.bfloat16)
    xt = sp.SparseTensor(torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16),
                         torch.from_numpy(coords).to(dev))
    with torch.no_grad():
        y = conv(xt)
    wq = orc.q8_0_dequant(blocks, oracle.F16).reshape(64, 27, 64)
    bb = bf16_bits(orc, conv.conv.bias.detach().float().cpu().numpy())
    ref = orc.sparse_conv(xb, wq, bb, orc.conv_table_slat(coords), ntaps=27, n_out=n,
                          idx_layout=1, out_dtype=oracle.F32, x_dtype=oracle.BF16,
                          w_dtype=oracle.F16, b_dtype=oracle.BF16)
    # the default f16 operands are the reference's GEMM operands: within
    # the output's two roundings (f16, then bf16) of the oracle per element
    assert conv.q8_operands == "f16"
    check_16bit("SparseConv3d Q8_0 f16 operands", from_dev(y.feats), ref, roundings=2)
    # bf16 operands: in-register dequant (n below the expansion threshold)
    # and the per-forward expansion to packed bf16 give the same bits, the
    # 2e-2 bar against the reference's operands
    conv.q8_operands = "bf16"
    with torch.no_grad():
        yb = conv(xt.replace(xt.feats))
    assert max_rel(from_dev(yb.feats), ref) <= MAXREL
    assert n < sp.Q8_EXPAND_MIN_ROWS
    saved = sp.Q8_EXPAND_MIN_ROWS
    sp.Q8_EXPAND_MIN_ROWS = 0
    try:
        with torch.no_grad():
            yx = conv(xt.replace(xt.feats))
    finally:
        sp.Q8_EXPAND_MIN_ROWS = saved
    assert torch.equal(yx.feats, yb.feats)
    conv.q8_operands = "f16"
    # the mesh GGUF layout of the same quants gives the identical result
    conv_m = sp.SparseConv3d(64, 64, 3).to(dev)
    conv_m.load_state_dict(conv.state_dict())
    conv_m.conv.weight.data = torch.from_numpy(w32.reshape(64, 3, 3, 3, 64)).to(dev)
    mesh_blocks = conv_m.quantize_q8_0("mesh")
    conv_m = conv_m.to(torch.bfloat16)
    with torch.no_grad():
        ym = conv_m(xt.replace(xt.feats))
    assert torch.equal(ym.feats, y.feats)
    assert not torch.equal(mesh_blocks.cpu(), torch.from_numpy(blocks))


def test_q8_0_dequant_f32_path(spc, orc, dev):
    import oracle
    import torch

    coords = spc.workloads.random_voxels(800, 12, batches=1, seed=19)
    n = coords.shape[0]
    _case(f"SparseConv3d Q8_0 weights with f32 feats N={n} 32->64")
    x = spc.workloads.normal((n, 32), 1.0, seed=8)
    conv = _sp(spc).SparseConv3d(32, 64, 3).to(dev)
    blocks = conv.quantize_q8_0().cpu().numpy()
    with torch.no_grad():
        y = conv(_tensor(spc, coords, x, dev))
    wq = orc.q8_0_dequant(blocks, oracle.F32).reshape(64, 27, 32)
    ref = _oracle_conv(orc, x, wq, conv.conv.bias.detach().cpu().numpy(),
                       orc.conv_table_slat(coords), 27, n, 0)
    _close_f32(y.feats.cpu().numpy(), ref)


def test_q8_0_quantize_edge_blocks(spc, orc, dev):
    """Zero block (amax -> 1e-12), exact .5 quotients (ties to even), and
    +-127 clipping, against the oracle's converter restatement."""
    import torch

    _case("q8_0_quantize edge blocks")
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, 32 * 64).astype(np.float32)
    w[:32] = 0.0
    w[32:64] = np.arange(32, dtype=np.float32) - 15.5   # amax 15.5 -> .5 quotients
    w[64:96] = np.float32(1e-30) * (np.arange(32) - 16)
    got = spc._native.q8_0_quantize(torch.from_numpy(w).to(dev)).cpu().numpy()
    assert np.array_equal(got, orc.q8_0_quantize(w))
    back = spc._native.q8_0_dequant(torch.from_numpy(got).to(dev)).cpu().numpy()
    import oracle

    assert np.array_equal(back, orc.q8_0_dequant(got, oracle.F32))


# ---------------------------------------------------------------------------
# spatial ops
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_downsample_upsample(spc, orc, dev, dt):
    import oracle
    import torch

    coords = spc.workloads.ellipsoid_batch(2, seed=23)
    n = coords.shape[0]
    _case(f"SparseDownsample/Upsample {dt} N={n} C=64")
    xf = spc.workloads.normal((n, 64), 1.0, seed=9)
    if dt == "f32":
        x_np, code, tdt = xf, oracle.F32, torch.float32
        feats = torch.from_numpy(xf)
    elif dt == "f16":
        x_np, code, tdt = xf.astype(np.float16), oracle.F16, torch.float16
        feats = torch.from_numpy(x_np)
    else:
        x_np, code, tdt = bf16_bits(orc, xf), oracle.BF16, torch.bfloat16
        feats = torch.from_numpy(x_np.view(np.int16)).view(torch.bfloat16)
    sp = _sp(spc)
    xt = sp.SparseTensor(feats.to(dev), torch.from_numpy(coords).to(dev))
    down = sp.SparseDownsample(2)(xt)
    d = orc.downsample_map(coords)
    assert np.array_equal(down.coords.cpu().numpy(), d["coarse_coords"])
    assert down._scale == tuple(s // 2 for s in xt._scale)  # the reference's s // f
    ref = orc.scatter_mean(x_np, d["fine_to_coarse"], d["counts"], d["nc"], dtype=code)
    got = down.feats.cpu()
    got = got.view(torch.int16).numpy().view(np.uint16) if dt == "bf16" else got.numpy()
    assert np.array_equal(got, ref)
    up = sp.SparseUpsample(2)(down)
    assert torch.equal(up.coords, xt.coords) and up.layout == xt.layout
    assert torch.equal(up.feats, down.feats[torch.from_numpy(d["fine_to_coarse"]).to(dev).long()])
    # the reference's bookkeeping: downsample s // 2, upsample s * 2
    assert up._scale == tuple(s * 2 for s in down._scale)


def test_down_up_reuse_maps(spc, orc, dev):
    """A block's downsample yields the same coarse coordinates on every
    call: the coarse convs' maps and plans are built once (kept with the
    fine coordinates), and the paired upsample hands the fine level's maps
    back -- the same results as tensors without any cached map."""
    import torch

    coords = spc.workloads.ellipsoid_batch(2, seed=31)
    n = coords.shape[0]
    _case(f"down / conv / up / conv map reuse N={n} C=64")
    sp = _sp(spc)
    g = torch.Generator().manual_seed(3)
    xt = sp.SparseTensor(torch.randn((n, 64), generator=g).to(dev, torch.bfloat16),
                         torch.from_numpy(coords).to(dev))
    conv_c = sp.SparseConv3d(64, 64, 3).to(dev, torch.bfloat16)
    conv_f = sp.SparseConv3d(64, 64, 3).to(dev, torch.bfloat16)
    outs = []
    with torch.no_grad():
        for _ in range(2):
            down = sp.SparseDownsample(2)(xt)
            hc = conv_c(down)
            up = sp.SparseUpsample(2)(hc)
            hf = conv_f(up)
            outs.append((hc.feats.clone(), hf.feats.clone(), down.data.indice_dict,
                         up.data.indice_dict))
    torch.cuda.synchronize()
    # one coarse map cache across the calls, the fine level's handed back
    assert outs[0][2] is outs[1][2] and "subm3" in outs[0][2]
    assert outs[0][3] is xt.data.indice_dict and outs[1][3] is xt.data.indice_dict
    assert "subm3" in xt.data.indice_dict
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    # tensors with fresh caches (new coordinate tensors): the same values
    xt2 = sp.SparseTensor(xt.feats.clone(), xt.coords.clone())
    with torch.no_grad():
        hc2 = conv_c(sp.SparseDownsample(2)(xt2))
        hf2 = conv_f(sp.SparseUpsample(2)(hc2))
    torch.cuda.synchronize()
    assert hf2.data.indice_dict is xt2.data.indice_dict
    assert torch.equal(hc2.feats, outs[0][0]) and torch.equal(hf2.feats, outs[0][1])


def test_subdivide_module(spc, orc, dev):
    import torch

    coords = spc.workloads.random_voxels(500, 10, batches=2, seed=29)
    n = coords.shape[0]
    _case(f"SparseSubdivide N={n}")
    x = spc.workloads.normal((n, 48), 1.0, seed=10)
    sp = _sp(spc)
    xt = _tensor(spc, coords, x, dev)
    out = sp.SparseSubdivide()(xt)
    oc, par = orc.subdivide(coords)
    assert np.array_equal(out.coords.cpu().numpy(), oc)
    assert np.array_equal(out.feats.cpu().numpy(), x[par])
    assert out._scale == (1, 1, 1) * 2  # the reference's tuple repetition
    assert out.shape == xt.shape


# ---------------------------------------------------------------------------
# reference table structs
# ---------------------------------------------------------------------------
def test_slat_tables(spc, orc, dev):
    import torch

    coords = spc.workloads.sphere_shell()
    n = coords.shape[0]
    _case(f"SlatTables.build sphere N={n}")
    t = spc.tables.SlatTables.build(torch.from_numpy(coords).to(dev))
    tm = orc.conv_table_slat(coords)
    om, mk, ar = orc.spconv_tables(tm, n)
    d = orc.downsample_map(coords)
    nc = d["nc"]
    assert (t.nf, t.nc) == (n, nc) == (21766, 4092)
    tmc = orc.conv_table_slat(d["coarse_coords"])
    omc, mkc, arc = orc.spconv_tables(tmc, nc)
    pairs = {
        "conv_fine": tm, "conv_fine_spconv": om, "conv_fine_mask": mk, "conv_fine_argsort": ar,
        "conv_coarse": tmc, "conv_coarse_spconv": omc, "conv_coarse_mask": mkc,
        "conv_coarse_argsort": arc, "fine_to_coarse": d["fine_to_coarse"],
        "coarse_children": d["children"], "coarse_count": d["counts"],
        "coarse_coords": d["coarse_coords"],
    }
    for k, v in pairs.items():
        assert np.array_equal(getattr(t, k).cpu().numpy().reshape(v.shape), v), k


def test_mesh_tables(spc, orc, dev):
    import torch

    coords = spc.workloads.random_voxels(400, 16, batches=1, seed=31)
    _case(f"MeshTables.build N={coords.shape[0]}")
    mt = spc.tables.MeshTables.build(torch.from_numpy(coords).to(dev), base_resolution=16)
    c = coords
    res = 16
    for lv in mt.levels:
        st, conv = orc.conv_table_mesh(c, res)
        assert st == 0
        assert lv.resolution == res and lv.n == c.shape[0]
        assert np.array_equal(lv.coords.cpu().numpy(), c)
        assert np.array_equal(lv.conv.cpu().numpy(), conv)
        c, _ = orc.subdivide(c)
        res *= 2
    assert mt.levels[2].n == 64 * coords.shape[0]


def test_forward_only(spc, dev):
    import torch

    coords = spc.workloads.random_voxels(200, 8, batches=1, seed=37)
    _case("SparseConv3d backward raises")
    sp = _sp(spc)
    conv = sp.SparseConv3d(32, 32, 3).to(dev)
    x = sp.SparseTensor(torch.randn(coords.shape[0], 32, device=dev),
                        torch.from_numpy(coords).to(dev))
    y = conv(x)
    assert y.feats.requires_grad
    with pytest.raises(NotImplementedError):
        y.feats.sum().backward()
