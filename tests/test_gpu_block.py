"""GPU parity of the residual-block kernels: spc_layernorm_silu, the conv's
residual and norm/modulation/SiLU epilogues, and SparseResBlock3d
(structured_latent_flow.py:15-74) against the oracle's numpy block."""
import numpy as np
import pytest

from helpers import bf16_bits, from_dev, max_rel, to_dev_bf16

pytestmark = pytest.mark.gpu

MAXREL = 2e-2


def _case(name):
    print(f"[case] {name}", flush=True)


def _dev_feats(orc, a, dt, dev):
    import torch

    if dt == "bf16":
        return to_dev_bf16(bf16_bits(orc, a), dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(
        {"f16": torch.float16, "f32": torch.float32}[dt])


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("c,affine,silu", [(128, True, True), (96, False, True), (1024, True, True),
                                            (512, True, True), (32, True, False), (2048, False, False)])
def test_layernorm_silu(spc, orc, dev, dt, c, affine, silu):
    import oracle

    _case(f"layernorm_silu {dt} c={c} affine={affine} silu={silu}")
    nat = spc._native
    rng = np.random.default_rng(c)
    n = 777
    x = (rng.standard_normal((n, c)) * 2 + 0.5).astype(np.float32)
    xd = _dev_feats(orc, x, dt, dev)
    code = {"bf16": oracle.BF16, "f16": oracle.F16, "f32": oracle.F32}[dt]
    xr = oracle.round_to(orc, x, code)
    g = rng.standard_normal(c).astype(np.float32) if affine else None
    b = rng.standard_normal(c).astype(np.float32) if affine else None
    import torch

    y = nat.layernorm_silu(xd, None if g is None else torch.from_numpy(g).to(dev),
                           None if b is None else torch.from_numpy(b).to(dev), eps=1e-6, silu=silu)
    ref = oracle.round_to(orc, oracle.layernorm(xr, g, b, 1e-6), code)
    if silu:
        ref = oracle.round_to(orc, oracle.silu(ref), code)
    got = from_dev(y)
    if dt == "f32":
        assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)
    else:
        # F32 statistics in another summation order: at most a rounding step apart
        assert max_rel(got, ref) <= 1e-2
        assert np.mean(got == ref) >= 0.98


def _subm_setup(spc, orc, dev, n_target, grid, batches, cin, cout, seed):
    import torch

    sp = spc.sparse
    coords = spc.workloads.random_voxels(n_target, grid, batches=batches, seed=seed)
    n = coords.shape[0]
    x = spc.workloads.normal((n, cin), 1.0, seed=seed + 1)
    xt = sp.SparseTensor(_dev_feats(orc, x, "bf16", dev), torch.from_numpy(coords).to(dev))
    conv = sp.SparseConv3d(cin, cout, 3).to(dev)
    with torch.no_grad():
        conv.conv.bias.normal_(0, 0.05)
    return coords, n, x, xt, conv.to(torch.bfloat16)


def test_conv_residual_epilogue(spc, orc, dev):
    import torch

    coords, n, x, xt, conv = _subm_setup(spc, orc, dev, 3000, 20, 2, 64, 128, 31)
    _case(f"conv residual epilogue bf16 N={n} 64->128")
    r = _dev_feats(orc, spc.workloads.normal((n, 128), 1.0, seed=33), "bf16", dev)
    with torch.no_grad():
        y = conv(xt).feats
        yf = conv.forward_fused(xt, residual=r).feats
    assert torch.equal(yf, y + r)  # dt(dt(conv) + r): bit-exact with the two-step sum


@pytest.mark.parametrize("cout", [128, 64, 32])
def test_conv_norm_mod_silu_epilogue(spc, orc, dev, cout):
    import torch

    coords, n, x, xt, conv = _subm_setup(spc, orc, dev, 3000, 20, 3, 64, cout, 41 + cout)
    _case(f"conv norm/modulate/SiLU epilogue bf16 N={n} 64->{cout}")
    nat = spc._native
    rng = np.random.default_rng(cout)
    scale = torch.from_numpy(rng.standard_normal((3, cout)).astype(np.float32) * 0.3).to(dev)
    shift = torch.from_numpy(rng.standard_normal((3, cout)).astype(np.float32) * 0.3).to(dev)
    scale, shift = scale.bfloat16(), shift.bfloat16()  # emb_out.type(x.dtype)
    with torch.no_grad():
        y = conv(xt)
        u = y.replace(nat.layernorm_silu(y.feats, eps=1e-6, silu=False))
        ref = torch.nn.functional.silu((u * (1 + scale) + shift).feats)
        yf = conv.forward_fused(xt, norm_mod=(scale.float(), shift.float(), 1e-6)).feats
    a, b = from_dev(yf), from_dev(ref)
    assert max_rel(a, b) <= 1e-2
    assert np.mean(a == b) >= 0.98


@pytest.mark.parametrize("cout", [256, 96])
def test_norm_epilogue_rejects_other_widths(spc, orc, dev, cout):
    """Only 32-, 64- and 128-channel rows fit the epilogue's lane groups;
    other widths are refused (the block runs spc_layernorm_mod_silu)."""
    import torch

    coords, n, x, xt, conv = _subm_setup(spc, orc, dev, 500, 10, 1, 64, cout, 51)
    _case(f"norm epilogue with cout={cout} is refused")
    s = torch.zeros(1, cout, device=dev)
    with pytest.raises(spc._native.SparseConvError, match="cout 32, 64 or 128"):
        conv.forward_fused(xt, norm_mod=(s, s, 1e-6))


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("c", [96, 1024, 2048])
def test_layernorm_mod_silu(spc, orc, dev, dt, c):
    """spc_layernorm_mod_silu against the oracle's composition:
    dt(silu(dt(dt(dt(LN(x)) * dt(1 + scale[b])) + shift[b])))."""
    import oracle
    import torch

    _case(f"layernorm_mod_silu {dt} c={c}")
    nat = spc._native
    rng = np.random.default_rng(c + 7)
    sizes = [400, 3, 520]
    n = sum(sizes)
    coords = np.zeros((n, 4), np.int32)
    coords[:, 0] = np.repeat(np.arange(3), sizes)
    x = (rng.standard_normal((n, c)) * 2 + 0.3).astype(np.float32)
    code = {"bf16": oracle.BF16, "f16": oracle.F16, "f32": oracle.F32}[dt]
    r = lambda a: oracle.round_to(orc, a, code)  # noqa: E731
    xr = r(x)
    scale = r(rng.standard_normal((3, c)).astype(np.float32) * 0.3)
    shift = r(rng.standard_normal((3, c)).astype(np.float32) * 0.3)
    y = nat.layernorm_mod_silu(_dev_feats(orc, x, dt, dev), torch.from_numpy(scale).to(dev),
                               torch.from_numpy(shift).to(dev), torch.from_numpy(coords).to(dev),
                               eps=1e-6)
    b = coords[:, 0]
    u = r(oracle.layernorm(xr, None, None, 1e-6))
    ref = r(oracle.silu(r(r(u * r(1.0 + scale[b])) + shift[b])))
    got = from_dev(y)
    if dt == "f32":
        assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)
    else:
        assert max_rel(got, ref) <= 1e-2
        assert np.mean(got == ref) >= 0.98


def _block_params(blk):
    p = {"norm1_w": blk.norm1.weight, "norm1_b": blk.norm1.bias,
         "conv1_w": blk.conv1.conv.weight, "conv1_b": blk.conv1.conv.bias,
         "conv2_w": blk.conv2.conv.weight, "conv2_b": blk.conv2.conv.bias}
    if hasattr(blk.skip_connection, "weight"):
        p["skip_w"], p["skip_b"] = blk.skip_connection.weight, blk.skip_connection.bias
    out = {}
    for k, v in p.items():
        a = v.detach().float().cpu().numpy()
        if k.startswith("conv") and k.endswith("_w"):
            a = a.reshape(a.shape[0], 27, a.shape[-1])
        out[k] = a
    return out


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("cin,cout", [(128, 128), (64, 128), (128, 256), (64, 96), (96, 32)])
def test_res_block(spc, orc, dev, cin, cout, dt):
    """SparseResBlock3d on the fused kernels (32-, 64- and 128-channel
    blocks take the conv's norm epilogue; 96 and 256 the conv plus the
    spc_layernorm_mod_silu row pass) against the oracle's block with the
    reference's rounding points."""
    import oracle
    import torch

    blocks = spc.blocks
    td, code = {"bf16": (torch.bfloat16, oracle.BF16), "f16": (torch.float16, oracle.F16)}[dt]
    coords = spc.workloads.random_voxels(4000, 22, batches=2, seed=61 + cout)
    n = coords.shape[0]
    _case(f"SparseResBlock3d {dt} N={n} {cin}->{cout}")
    torch.manual_seed(cin + cout)
    blk = blocks.SparseResBlock3d(cin, 96, cout).to(dev)
    with torch.no_grad():
        for p in blk.conv2.parameters():  # the reference zero-initialises conv2
            p.normal_(0, 0.02)
        blk.norm1.weight.normal_(1, 0.1)
        blk.norm1.bias.normal_(0, 0.1)
    blk = blk.to(td)
    # keep LayerNorm affine parameters f32 like LayerNorm32 (computed in F32)
    blk.norm1.float()
    x = spc.workloads.normal((n, cin), 1.0, seed=62)
    xt = spc.sparse.SparseTensor(_dev_feats(orc, x, dt, dev), torch.from_numpy(coords).to(dev))
    emb = torch.randn(2, 96, device=dev).to(td)
    with torch.no_grad():
        y = blk(xt, emb)
        emb_out = blk.emb_layers(emb).float().cpu().numpy()
    scale, shift = emb_out[:, :cout], emb_out[:, cout:]
    xr = oracle.round_to(orc, x, code)
    p = _block_params(blk)
    ref = oracle.res_block(orc, xr, orc.conv_table_slat(coords), p, scale, shift,
                           coords[:, 0].astype(np.int64), code)
    got = from_dev(y.feats)
    assert got.shape == ref.shape
    mr = max_rel(got, ref)
    print(f"[parity] SparseResBlock3d {dt} {cin}->{cout}: max_rel={mr:.3e}", flush=True)
    assert mr <= MAXREL


@pytest.mark.parametrize("mode", ["down", "up"])
def test_io_res_block(spc, orc, dev, mode):
    """The SLAT flow model's IO blocks at their real widths (structured_
    latent_flow.py:140-200; native SRC/slat_flow_graph.cpp:286-380, 395-396),
    bf16:
      down  SparseResBlock3d(128, 1024, 1024, downsample=True) on the 4
            ellipsoid shells (62,710 fine -> 11,774 coarse rows): scatter-mean
            downsample, LayerNorm + SiLU, conv 128 -> 1024, norm2 /
            modulation / SiLU (the row pass), conv 1024 -> 1024, + the
            128 -> 1024 skip;
      up    SparseResBlock3d(2048, 1024, 128, upsample=True) (out_blocks[0]:
            the 2 x 1024 concatenation of the skip) on 2 shells: coarse ->
            fine gather, conv 2048 -> 128 at the fine rows, the fused norm
            epilogue, conv 128 -> 128, + the 2048 -> 128 skip.
    Against oracle.io_res_block, max-rel <= 2e-2."""
    import oracle
    import torch
    from helpers import oracle_threads

    sp = spc.sparse
    fine = spc.workloads.ellipsoid_batch(4 if mode == "down" else 2)
    cin, cout = (128, 1024) if mode == "down" else (2048, 128)
    torch.manual_seed(7 + cin)
    blk = spc.blocks.SparseResBlock3d(cin, 1024, cout, downsample=mode == "down",
                                      upsample=mode == "up").to(dev)
    with torch.no_grad():
        for prm in blk.conv2.parameters():  # the reference zero-initialises conv2
            prm.normal_(0, 0.02)
        blk.norm1.weight.normal_(1, 0.1)
        blk.norm1.bias.normal_(0, 0.1)
    blk = blk.to(torch.bfloat16)
    blk.norm1.float()
    fd = torch.from_numpy(fine).to(dev)
    if mode == "down":
        x = spc.workloads.normal((fine.shape[0], cin), 1.0, seed=81)
        xt = sp.SparseTensor(_dev_feats(orc, x, "bf16", dev), fd)
        coords_in = fine
    else:
        # a coarse tensor with the upsample cache of its fine rows
        ft = sp.SparseTensor(torch.zeros((fine.shape[0], 32), dtype=torch.bfloat16, device=dev),
                             fd)
        ct = sp.SparseDownsample(2)(ft)
        coords_in = ct.coords.cpu().numpy()
        x = spc.workloads.normal((coords_in.shape[0], cin), 1.0, seed=82)
        xt = ct.replace(_dev_feats(orc, x, "bf16", dev))
    _case(f"IO res block {mode} bf16 N_in={coords_in.shape[0]} {cin}->{cout}")
    emb = torch.randn(len(np.unique(fine[:, 0])), 1024, device=dev).bfloat16()
    with torch.no_grad():
        y = blk(xt, emb)
        emb_out = blk.emb_layers(emb).float().cpu().numpy()
    torch.cuda.synchronize()
    scale, shift = emb_out[:, :cout], emb_out[:, cout:]
    oc, ref = oracle.io_res_block(orc, oracle.round_to(orc, x, oracle.BF16), coords_in,
                                  _block_params(blk), scale, shift, oracle.BF16, mode=mode,
                                  fine_coords=fine if mode == "up" else None,
                                  nthreads=oracle_threads())
    assert np.array_equal(y.coords.cpu().numpy(), oc)
    got = from_dev(y.feats)
    mr = max_rel(got, ref)
    print(f"[parity] IO res block {mode} {cin}->{cout}: rows={ref.shape[0]} max_rel={mr:.3e}",
          flush=True)
    assert mr <= MAXREL
    if mode == "up":
        # norm1 / SiLU and the skip on the coarse rows (the default) against
        # the reference's order over the upsampled copies: conv1 sees the same
        # values, so only the skip Linear's rounding over other row counts
        # may differ
        assert blk.coarse_rows
        blk.coarse_rows = False
        with torch.no_grad():
            y_ref_order = blk(xt, emb)
        blk.coarse_rows = True
        torch.cuda.synchronize()
        assert np.array_equal(y_ref_order.coords.cpu().numpy(), oc)
        alt = from_dev(y_ref_order.feats)
        assert max_rel(alt, ref) <= MAXREL
        d = max_rel(got, alt)
        print(f"[parity] IO res block up: coarse-row norm/skip vs upsampled copies max_rel={d:.3e}, "
              f"{int((got != alt).sum())} of {got.size} values differ", flush=True)
        assert d <= 1e-2


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("c,groups,gather", [(64, 32, True), (32, 32, False), (768, 32, True),
                                             (128, 8, False)])
def test_group_norm_silu(spc, orc, dev, dt, c, groups, gather):
    import oracle
    import torch

    _case(f"group_norm_silu {dt} c={c} groups={groups} gather={gather}")
    nat = spc._native
    rng = np.random.default_rng(c + groups)
    sizes = [300, 1021, 2, 700]
    n = sum(sizes)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    x = (rng.standard_normal((n, c)) * 1.5 + 0.2).astype(np.float32)
    code = {"bf16": oracle.BF16, "f32": oracle.F32}[dt]
    xr = oracle.round_to(orc, x, code)
    g = rng.standard_normal(c).astype(np.float32)
    b = rng.standard_normal(c).astype(np.float32)
    rows = rng.integers(0, n, size=3000).astype(np.int32) if gather else None
    y = nat.group_norm_silu(_dev_feats(orc, x, dt, dev), torch.from_numpy(offs).to(dev), groups,
                            torch.from_numpy(g).to(dev), torch.from_numpy(b).to(dev), eps=1e-5,
                            silu=True, rows=None if rows is None else torch.from_numpy(rows).to(dev))
    ref = oracle.round_to(orc, oracle.silu(oracle.round_to(
        orc, oracle.group_norm_items(xr, offs, groups, g, b, 1e-5), code)), code)
    if rows is not None:
        ref = ref[rows]
    got = from_dev(y)
    if dt == "f32":
        assert np.allclose(got, ref, rtol=1e-4, atol=1e-5)
    else:
        assert max_rel(got, ref) <= 1e-2
        assert np.mean(got == ref) >= 0.98


def test_compose_rows(spc, dev):
    import torch

    _case("compose_rows n=4099 (ragged tail), sentinels and out-of-range entries")
    nat = spc._native
    rng = np.random.default_rng(5)
    rows = rng.integers(0, 500, size=800).astype(np.int32)
    idx = rng.integers(-3, 820, size=4099).astype(np.int32)
    got = nat.compose_rows(torch.from_numpy(idx).to(dev), torch.from_numpy(rows).to(dev))
    ok = (idx >= 0) & (idx < 800)
    ref = np.where(ok, rows[np.clip(idx, 0, 799)], -1)
    assert np.array_equal(got.cpu().numpy(), ref)


def test_conv_residual_rows_epilogue(spc, orc, dev):
    """residual[residual_rows[t]] added in the epilogue: bit-exact with the
    gathered two-step sum; entries outside [0, R) add nothing."""
    import torch

    coords, n, x, xt, conv = _subm_setup(spc, orc, dev, 3000, 20, 2, 64, 96, 35)
    _case(f"conv residual-rows epilogue bf16 N={n} 64->96")
    r = _dev_feats(orc, spc.workloads.normal((700, 96), 1.0, seed=36), "bf16", dev)
    rng = np.random.default_rng(37)
    rows = rng.integers(0, 700, size=n).astype(np.int32)
    rows[::97] = -1
    rows[5::101] = 700
    rows_d = torch.from_numpy(rows).to(dev)
    with torch.no_grad():
        y = conv(xt).feats
        yf = conv.forward_fused(xt, residual=r, residual_rows=rows_d).feats
    valid = torch.from_numpy((rows >= 0) & (rows < 700)).to(dev)
    add = torch.where(valid[:, None], r[rows_d.clamp(0, 699).long()], torch.zeros_like(r[:1]))
    assert torch.equal(yf, y + add)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("cin,cout", [(64, 32), (32, 32)])
def test_subdivide_block(spc, orc, dev, cin, cout, dt):
    """SparseSubdivideBlock3d (GroupNorm/SiLU/gather pass, conv, GroupNorm/
    SiLU, conv with the residual epilogue) against the oracle's block."""
    import oracle
    import torch

    blocks = spc.blocks
    td, code = {"bf16": (torch.bfloat16, oracle.BF16), "f16": (torch.float16, oracle.F16)}[dt]
    coords = spc.workloads.random_voxels(1500, 16, batches=2, seed=71 + cin)
    n = coords.shape[0]
    _case(f"SparseSubdivideBlock3d {dt} N={n} {cin}->{cout}")
    torch.manual_seed(cin)
    blk = blocks.SparseSubdivideBlock3d(cin, 16, cout).to(dev)
    with torch.no_grad():
        for prm in blk.out_layers[3].parameters():  # the reference zero-initialises it
            prm.normal_(0, 0.02)
        for gn in (blk.act_layers[0], blk.out_layers[1]):
            gn.weight.normal_(1, 0.1)
            gn.bias.normal_(0, 0.1)
    blk = blk.to(td)
    blk.act_layers[0].float()
    blk.out_layers[1].float()
    x = spc.workloads.normal((n, cin), 1.0, seed=72)
    xt = spc.sparse.SparseTensor(_dev_feats(orc, x, dt, dev), torch.from_numpy(coords).to(dev))
    with torch.no_grad():
        y = blk(xt)
    f = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    p = {"gn0_w": f(blk.act_layers[0].weight), "gn0_b": f(blk.act_layers[0].bias),
         "conv1_w": f(blk.out_layers[0].conv.weight).reshape(cout, 27, cin),
         "conv1_b": f(blk.out_layers[0].conv.bias),
         "gn1_w": f(blk.out_layers[1].weight), "gn1_b": f(blk.out_layers[1].bias),
         "conv2_w": f(blk.out_layers[3].conv.weight).reshape(cout, 27, cout),
         "conv2_b": f(blk.out_layers[3].conv.bias)}
    if cin != cout:
        p["skip_w"] = f(blk.skip_connection.conv.weight)
        p["skip_b"] = f(blk.skip_connection.conv.bias)
    child, ref = oracle.subdivide_block(orc, oracle.round_to(orc, x, code), coords, p, 32, code)
    assert np.array_equal(y.coords.cpu().numpy(), child)
    assert max_rel(from_dev(y.feats), ref) <= MAXREL
    # merged taps: the same block with the 27-tap conv1 agrees to the
    # rounding of the summed weights; the 27-tap form reads parent rows
    # through composed tables and gives the same bits as the block over
    # materialised child copies
    assert blk.merged_taps
    blk.merged_taps = False
    with torch.no_grad():
        y27 = blk(xt)
    blk.merged_taps = True
    assert max_rel(from_dev(y.feats), from_dev(y27.feats)) <= 1e-2
    y = y27
    nat, sp = spc._native, spc.sparse
    with torch.no_grad():
        cc, par = blk.sub.map(xt)
        gn0, gn1 = blk.act_layers[0], blk.out_layers[1]
        h = blk.sub.assemble(xt, cc, nat.group_norm_silu(
            xt.feats, sp.batch_offsets(xt), 32, gn0.weight, gn0.bias, gn0.eps, rows=par))
        xs = blk.sub.assemble(xt, cc, nat.gather_rows(xt.feats, par))
        h = blk.out_layers[0](h)
        h = h.replace(nat.group_norm_silu(h.feats, sp.batch_offsets(h), 32, gn1.weight, gn1.bias,
                                          gn1.eps))
        want = blk.out_layers[3](h) + blk.skip_connection(xs)
    assert torch.equal(y.feats, want.feats)


def test_subdivide_block_merged_taps_f32(spc, orc, dev):
    """F32 features: the merged-tap conv1 (weights summed in F64, rounded to
    F32) against the 27-tap conv1, and both against the oracle's block."""
    import oracle
    import torch

    blocks = spc.blocks
    coords = spc.workloads.random_voxels(1200, 14, batches=2, seed=81)
    n = coords.shape[0]
    _case(f"SparseSubdivideBlock3d f32 merged vs 27 taps N={n} 64->32")
    torch.manual_seed(5)
    blk = blocks.SparseSubdivideBlock3d(64, 14, 32).to(dev)
    with torch.no_grad():
        for prm in blk.out_layers[3].parameters():
            prm.normal_(0, 0.05)
    x = spc.workloads.normal((n, 64), 1.0, seed=82)
    xt = spc.sparse.SparseTensor(torch.from_numpy(x).to(dev), torch.from_numpy(coords).to(dev))
    with torch.no_grad():
        ym = blk(xt).feats
        blk.merged_taps = False
        y27 = blk(xt).feats
    assert torch.allclose(ym, y27, rtol=1e-4, atol=1e-5)
    f = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    p = {"gn0_w": f(blk.act_layers[0].weight), "gn0_b": f(blk.act_layers[0].bias),
         "conv1_w": f(blk.out_layers[0].conv.weight).reshape(32, 27, 64),
         "conv1_b": f(blk.out_layers[0].conv.bias),
         "gn1_w": f(blk.out_layers[1].weight), "gn1_b": f(blk.out_layers[1].bias),
         "conv2_w": f(blk.out_layers[3].conv.weight).reshape(32, 27, 32),
         "conv2_b": f(blk.out_layers[3].conv.bias),
         "skip_w": f(blk.skip_connection.conv.weight), "skip_b": f(blk.skip_connection.conv.bias)}
    _, ref = oracle.subdivide_block(orc, x, coords, p, 32, oracle.F32)
    assert np.allclose(ym.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)


def test_subdivide_block_192_channels(spc, orc, dev):
    """C_out = 192 over 75k children (the 192-column conv tiles): merged taps
    against the 27-tap conv1, and the 27-tap block bit-identical to the block
    over materialised child rows."""
    import torch

    blocks, nat, sp = spc.blocks, spc._native, spc.sparse
    coords = spc.workloads.random_voxels(9600, 40, batches=2, seed=95)
    n = coords.shape[0]
    assert 8 * n >= 256 * 256
    _case(f"SparseSubdivideBlock3d bf16 N={n} -> {8 * n} children 64->192")
    torch.manual_seed(6)
    blk = blocks.SparseSubdivideBlock3d(64, 40, 192).to(dev)
    with torch.no_grad():
        for prm in blk.out_layers[3].parameters():
            prm.normal_(0, 0.02)
    blk = blk.to(torch.bfloat16)
    blk.act_layers[0].float()
    blk.out_layers[1].float()
    x = spc.workloads.normal((n, 64), 1.0, seed=96)
    xt = sp.SparseTensor(_dev_feats(orc, x, "bf16", dev), torch.from_numpy(coords).to(dev))
    with torch.no_grad():
        ym = blk(xt)
        blk.merged_taps = False
        y27 = blk(xt)
        cc, par = blk.sub.map(xt)
        gn0, gn1 = blk.act_layers[0], blk.out_layers[1]
        h = blk.sub.assemble(xt, cc, nat.group_norm_silu(
            xt.feats, sp.batch_offsets(xt), 32, gn0.weight, gn0.bias, gn0.eps, rows=par))
        xs = blk.sub.assemble(xt, cc, nat.gather_rows(xt.feats, par))
        h = blk.out_layers[0](h)
        h = h.replace(nat.group_norm_silu(h.feats, sp.batch_offsets(h), 32, gn1.weight, gn1.bias,
                                          gn1.eps))
        want = blk.out_layers[3](h) + blk.skip_connection(xs)
    assert torch.equal(y27.feats, want.feats)
    assert max_rel(from_dev(ym.feats), from_dev(y27.feats)) <= 1e-2


@pytest.mark.parametrize("case", ["768to192", "192to96"])
def test_subdivide_block_decoder_widths(spc, orc, dev, case):
    """The mesh decoder's own SparseSubdivideBlock3d widths against the
    oracle's block (decoder_mesh.py:69-83; SRC/mesh_decoder_graph.cpp:
    399-437): 768 -> 192 from the 64^3 sphere shell's 21,766 voxels to their
    174,128 children (every output row), and 192 -> 96 from those 174,128
    voxels to their 1,393,024 children (20,000 sampled output rows; the
    oracle's conv1 and both GroupNorms still run over every child).  Both
    conv1 forms: merged taps (the default, summed weights rounded once to
    bf16) and the reference's 27 taps."""
    import oracle
    import torch
    from helpers import oracle_threads

    blocks, sp = spc.blocks, spc.sparse
    cin, cout, res = {"768to192": (768, 192, 64), "192to96": (192, 96, 128)}[case]
    coords = spc.workloads.sphere_shell()
    if res == 128:
        coords, _ = orc.subdivide(coords)
    n = coords.shape[0]
    _case(f"SparseSubdivideBlock3d bf16 decoder widths {cin}->{cout}, {n} parents -> {8 * n} "
          "children")
    torch.manual_seed(cin + cout)
    blk = blocks.SparseSubdivideBlock3d(cin, res, cout).to(dev)
    with torch.no_grad():
        for prm in blk.out_layers[3].parameters():  # the reference zero-initialises it
            prm.normal_(0, 0.02)
        for gn in (blk.act_layers[0], blk.out_layers[1]):
            gn.weight.normal_(1, 0.1)
            gn.bias.normal_(0, 0.1)
    blk = blk.to(torch.bfloat16)
    blk.act_layers[0].float()
    blk.out_layers[1].float()
    x = spc.workloads.normal((n, cin), 1.0, seed=cin + 7)
    xt = sp.SparseTensor(_dev_feats(orc, x, "bf16", dev), torch.from_numpy(coords).to(dev))
    f = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    p = {"gn0_w": f(blk.act_layers[0].weight), "gn0_b": f(blk.act_layers[0].bias),
         "conv1_w": f(blk.out_layers[0].conv.weight).reshape(cout, 27, cin),
         "conv1_b": f(blk.out_layers[0].conv.bias),
         "gn1_w": f(blk.out_layers[1].weight), "gn1_b": f(blk.out_layers[1].bias),
         "conv2_w": f(blk.out_layers[3].conv.weight).reshape(cout, 27, cout),
         "conv2_b": f(blk.out_layers[3].conv.bias),
         "skip_w": f(blk.skip_connection.conv.weight), "skip_b": f(blk.skip_connection.conv.bias)}
    rows = None
    if case == "192to96":
        rows = np.sort(np.random.default_rng(97).choice(8 * n, 20000, replace=False))
    child, ref = oracle.subdivide_block(orc, oracle.round_to(orc, x, oracle.BF16), coords, p, 32,
                                        oracle.BF16, nthreads=oracle_threads(), blocked=True,
                                        rows=rows)
    for merged in (True, False):
        blk.merged_taps = merged
        with torch.no_grad():
            y = blk(xt)
        torch.cuda.synchronize()
        got = from_dev(y.feats)
        if rows is not None:
            got = got[rows]
        mr = max_rel(got, ref)
        print(f"[parity] SparseSubdivideBlock3d {cin}->{cout} merged_taps={merged}: "
              f"rows={ref.shape[0]} max_rel={mr:.3e}", flush=True)
        assert np.array_equal(y.coords.cpu().numpy(), child)
        assert mr <= MAXREL, (merged, mr)
    blk.merged_taps = True
