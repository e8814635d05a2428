"""GPU scatter-mean and row gather.  Scatter-mean must be bit-exact with the
oracle's restatement of the ggml CPU op (PATCH:151-215: partial sums in the
storage dtype, ascending fine rows, F32 division), on the cases of the
reference's regression test SRC/scatter_mean_backend_test.cpp:96-104 (inputs
regenerated with the same mt19937 recipe) and on the SLAT downsample map."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

KAT_CASES = [(4, 1, 1, 1), (4, 7, 3, 2), (33, 65, 17, 3), (128, 512, 100, 4),
             (128, 26281, 5239, 5)]


def _case(name):
    print(f"[case] {name}", flush=True)


@pytest.mark.parametrize("channels,nf,nc,seed", KAT_CASES)
def test_scatter_mean_reference_cases(spc, orc, dev, channels, nf, nc, seed):
    import oracle
    import torch

    _case(f"scatter_mean f16 C={channels} nf={nf} nc={nc} seed={seed}")
    f, rows, counts = orc.scatter_case(channels, nf, nc, seed)
    ref = orc.scatter_mean(f, rows, counts, nc, dtype=oracle.F16)
    feats = torch.from_numpy(f.view(np.int16)).to(dev).view(torch.float16)
    out = spc._native.scatter_mean(feats, torch.from_numpy(rows).to(dev),
                                   torch.from_numpy(counts).to(dev), nc)
    got = out.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_scatter_mean_downsample_map(spc, orc, dev, dt):
    import oracle
    import torch

    coords = spc.workloads.ellipsoid_batch()
    n = coords.shape[0]
    _case(f"scatter_mean {dt} on the ellipsoid downsample map N={n} C=128")
    d = orc.downsample_map(coords)
    x = spc.workloads.normal((n, 128), 1.0, seed=3)
    if dt == "bf16":
        x_np = orc.f32_to_bf16(x)
        feats = torch.from_numpy(x_np.view(np.int16)).view(torch.bfloat16)
        code = oracle.BF16
    else:
        x_np, feats, code = x, torch.from_numpy(x), oracle.F32
    ref = orc.scatter_mean(x_np, d["fine_to_coarse"], d["counts"], d["nc"], dtype=code)
    out = spc._native.scatter_mean(feats.to(dev), torch.from_numpy(d["fine_to_coarse"]).to(dev),
                                   torch.from_numpy(d["counts"]).to(dev), d["nc"]).cpu()
    got = out.view(torch.int16).numpy().view(np.uint16) if dt == "bf16" else out.numpy()
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("dt,channels", [("bf16", 128), ("f16", 13), ("f32", 64)])
def test_children_mean_equals_scatter_mean(spc, orc, dev, dt, channels):
    """spc_children_mean over the downsample map's children lists gives
    spc_scatter_mean's values (and the oracle's) bit for bit."""
    import oracle
    import torch

    coords = spc.workloads.ellipsoid_batch(3, seed=17)
    n = coords.shape[0]
    _case(f"children_mean {dt} C={channels} N={n}")
    nat = spc._native
    d = nat.downsample_map(torch.from_numpy(coords).to(dev), 3, 64)
    x = spc.workloads.normal((n, channels), 1.0, seed=channels)
    if dt == "bf16":
        x_np, code = orc.f32_to_bf16(x), oracle.BF16
        feats = torch.from_numpy(x_np.view(np.int16)).view(torch.bfloat16)
    elif dt == "f16":
        x_np, code = x.astype(np.float16), oracle.F16
        feats = torch.from_numpy(x_np)
    else:
        x_np, code, feats = x, oracle.F32, torch.from_numpy(x)
    feats = feats.to(dev)
    a = nat.children_mean(feats, d.children, d.counts, d.nc)
    b = nat.scatter_mean(feats, d.fine_to_coarse, d.counts, d.nc)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16) if dt != "f32" else a,
                       b.view(torch.int16) if dt != "f32" else b)
    ref = orc.scatter_mean(x_np, d.fine_to_coarse.cpu().numpy(), d.counts.cpu().numpy(), d.nc,
                           dtype=code)
    got = a.cpu()
    got = got.numpy() if dt == "f32" else got.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref.view(np.uint16) if dt == "f16" else ref)


@pytest.mark.parametrize("dt,channels", [("f32", 64), ("bf16", 128), ("f16", 96), ("bf16", 3),
                                         ("f32", 1)])
def test_gather_rows(spc, dev, dt, channels):
    import torch

    _case(f"gather_rows {dt} C={channels}")
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dt]
    g = torch.Generator().manual_seed(channels)
    src = torch.randn(1000, channels, generator=g).to(tdt)
    idx = torch.randint(-5, 1010, (4321,), generator=g, dtype=torch.int32)
    out = spc._native.gather_rows(src.to(dev), idx.to(dev)).cpu()
    valid = (idx >= 0) & (idx < 1000)
    exp = torch.zeros(4321, channels, dtype=tdt)
    exp[valid] = src[idx[valid].long()]
    assert torch.equal(out, exp)
