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
                                            (32, True, False), (2048, False, False)])
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


def test_norm_epilogue_rejects_wide_rows(spc, orc, dev):
    import torch

    coords, n, x, xt, conv = _subm_setup(spc, orc, dev, 500, 10, 1, 64, 256, 51)
    _case("norm epilogue with cout=256 is refused")
    s = torch.zeros(1, 256, device=dev)
    with pytest.raises(spc._native.SparseConvError, match="cout <= 128"):
        conv.forward_fused(xt, norm_mod=(s, s, 1e-6))


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


@pytest.mark.parametrize("cin,cout", [(128, 128), (64, 128), (128, 256)])
def test_res_block(spc, orc, dev, cin, cout):
    """SparseResBlock3d on the fused kernels (the 256-channel block runs the
    unfused norm path) against the oracle's block with the reference's
    rounding points."""
    import oracle
    import torch

    blocks = spc.blocks
    coords = spc.workloads.random_voxels(4000, 22, batches=2, seed=61 + cout)
    n = coords.shape[0]
    _case(f"SparseResBlock3d bf16 N={n} {cin}->{cout}")
    torch.manual_seed(cin + cout)
    blk = blocks.SparseResBlock3d(cin, 96, cout).to(dev)
    with torch.no_grad():
        for p in blk.conv2.parameters():  # the reference zero-initialises conv2
            p.normal_(0, 0.02)
        blk.norm1.weight.normal_(1, 0.1)
        blk.norm1.bias.normal_(0, 0.1)
    blk = blk.to(torch.bfloat16)
    # keep LayerNorm affine parameters f32 like LayerNorm32 (computed in F32)
    blk.norm1.float()
    x = spc.workloads.normal((n, cin), 1.0, seed=62)
    xt = spc.sparse.SparseTensor(_dev_feats(orc, x, "bf16", dev), torch.from_numpy(coords).to(dev))
    emb = torch.randn(2, 96, device=dev).bfloat16()
    with torch.no_grad():
        y = blk(xt, emb)
        emb_out = blk.emb_layers(emb).float().cpu().numpy()
    scale, shift = emb_out[:, :cout], emb_out[:, cout:]
    xr = oracle.round_to(orc, x, oracle.BF16)
    p = _block_params(blk)
    ref = oracle.res_block(orc, xr, orc.conv_table_slat(coords), p, scale, shift,
                           coords[:, 0].astype(np.int64), oracle.BF16)
    got = from_dev(y.feats)
    assert got.shape == ref.shape
    assert max_rel(got, ref) <= MAXREL
