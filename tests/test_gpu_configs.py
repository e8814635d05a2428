"""GPU parity at the workloads' full shapes for the stages not covered by
test_gpu_conv.py, every output row against the oracle:

  config 3  the coarse-map submanifold convs of the SLAT IO block at 32^3
            (4 ellipsoid shells, 62,710 fine -> 11,774 coarse rows):
            128 -> 1024 and 1024 -> 1024, bf16 (SRC/slat_flow_graph.cpp:
            168-221 via the res block at :395-396);
  config 4  the mesh decoder's upsample levels (sphere shell subdivided twice
            with seeded 50% pruning: 86,922 rows at 128^3, 347,860 at 256^3):
            submanifold convs C=64 and C=32, bf16, weights in the decoder's
            [27, Cout, Cin] GGUF layout (SRC/mesh_decoder_graph.cpp:290-347;
            cpp_ggml/scripts/convert_sam3d_to_gguf.py:508-511).

Bars: max|a-b| / max|b| <= 2e-2 and |a-b| <= 2^-8 |b| + 2^-12 max|b| per
element (tests/helpers.py check_16bit)."""
import numpy as np
import pytest

from helpers import bf16_bits, check_16bit, from_dev, oracle_threads, to_dev_bf16

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[case] {name}", flush=True)


@pytest.fixture(scope="module")
def coarse(spc, orc, dev):
    """Config-3 coarse level: the downsample of the config-2 coords and its
    submanifold table (both checked against the oracle)."""
    import torch

    nat = spc._native
    coords = spc.workloads.ellipsoid_batch()
    d = nat.downsample_map(torch.from_numpy(coords).to(dev), 4, 64)
    ref = orc.downsample_map(coords)
    assert d.nc == ref["nc"] == 11774
    cc = d.coarse_coords.cpu().numpy()
    assert np.array_equal(cc, ref["coarse_coords"])
    m = nat.map_build(d.coarse_coords)
    tm = orc.conv_table_slat(cc)
    assert np.array_equal(m.token_major.cpu().numpy(), tm)
    return d, m, tm


@pytest.mark.parametrize("cin,cout", [(128, 1024), (1024, 1024)])
def test_config3_coarse_subm(spc, orc, dev, coarse, cin, cout):
    import oracle
    import torch

    nat = spc._native
    wl = spc.workloads
    d, m, tm = coarse
    nc = d.nc
    _case(f"config3 coarse subm N={nc} {cin}->{cout}")
    x = bf16_bits(orc, wl.normal((nc, cin), 1.0, seed=cin + 1))
    w = bf16_bits(orc, wl.normal((cout, 27, cin), 0.02, seed=cin + 2))
    b = bf16_bits(orc, wl.normal((cout,), 0.01, seed=cin + 3))
    y = nat.sparse_conv(to_dev_bf16(x, dev), nat.pack_weights(to_dev_bf16(w, dev)),
                        to_dev_bf16(b, dev), m.token_major, ntaps=27, n_out=nc, plan=m.plan())
    torch.cuda.synchronize()
    ref = orc.sparse_conv(x, w, b, tm, ntaps=27, n_out=nc, idx_layout=1, out_dtype=oracle.F32,
                          x_dtype=oracle.BF16, w_dtype=oracle.BF16, b_dtype=oracle.BF16,
                          nthreads=oracle_threads(), blocked=True)
    check_16bit(f"config3 coarse subm {cin}->{cout}", from_dev(y), ref)


@pytest.fixture(scope="module")
def mesh_levels(spc, orc, dev):
    """Config-4 levels: (coords, token-major table, resolution) at 128^3 and
    256^3, subdivided and pruned on the GPU and checked against the oracle."""
    import torch

    nat = spc._native
    wl = spc.workloads
    c = wl.sphere_shell()
    keeps = wl.prune_masks(c.shape[0])
    out = []
    cd, res = torch.from_numpy(c).to(dev), 64
    for keep in keeps:
        ref_c, _ = orc.subdivide(cd.cpu().numpy(), keep)
        oc, _ = nat.subdivide_map(cd, torch.from_numpy(keep).to(dev))
        assert np.array_equal(oc.cpu().numpy(), ref_c)
        res *= 2
        st, tm_ref = orc.conv_table_mesh(ref_c, res)
        assert st == 0
        m = nat.map_build(oc, mesh_resolution=res)
        assert np.array_equal(m.token_major.cpu().numpy(), tm_ref)
        out.append((oc, m, tm_ref, res))
        cd = oc
    assert [o[0].shape[0] for o in out] == [86922, 347860]
    return out


@pytest.mark.parametrize("level,ch", [(0, 64), (1, 32)])
def test_config4_mesh_conv(spc, orc, dev, mesh_levels, level, ch):
    """The mesh decoder's conv at the pruned level: weights stored as the
    GGUF [27, Cout, Cin] rows (SPC_W_TCK), packed, run over the level's mesh
    table; the oracle reads the same [27, Cout, Cin] buffer (w_layout 1)."""
    import oracle
    import torch

    nat = spc._native
    wl = spc.workloads
    oc, m, tm, res = mesh_levels[level]
    n = oc.shape[0]
    _case(f"config4 mesh conv {res}^3 N={n} C={ch}")
    x = bf16_bits(orc, wl.normal((n, ch), 1.0, seed=400 + ch))
    w_tck = bf16_bits(orc, wl.normal((27, ch, ch), 0.02, seed=401 + ch))
    b = bf16_bits(orc, wl.normal((ch,), 0.01, seed=402 + ch))
    pw = nat.pack_weights(to_dev_bf16(w_tck, dev), layout=nat.W_TCK)
    y = nat.sparse_conv(to_dev_bf16(x, dev), pw, to_dev_bf16(b, dev), m.token_major, ntaps=27,
                        n_out=n, plan=m.plan())
    torch.cuda.synchronize()
    ref = orc.sparse_conv(x, w_tck, b, tm, ntaps=27, n_out=n, idx_layout=1, w_layout=1,
                          out_dtype=oracle.F32, x_dtype=oracle.BF16, w_dtype=oracle.BF16,
                          b_dtype=oracle.BF16, nthreads=oracle_threads(), blocked=True)
    check_16bit(f"config4 mesh conv {res}^3 C={ch}", from_dev(y), ref)
