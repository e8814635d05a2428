"""Pins the oracle's residual-block pieces (oracle.layernorm / silu /
round_to) against torch's CPU layer_norm and silu (library routines) and
closed forms, before they check the GPU block."""
import numpy as np
import pytest


def test_layernorm_matches_torch_and_closed_forms():
    import oracle
    import torch

    rng = np.random.default_rng(0)
    x = (rng.standard_normal((64, 128)) * 3 + 1).astype(np.float32)
    g = rng.standard_normal(128).astype(np.float32)
    b = rng.standard_normal(128).astype(np.float32)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x), (128,), torch.from_numpy(g),
                                         torch.from_numpy(b), eps=1e-6).numpy()
    assert np.allclose(oracle.layernorm(x, g, b, 1e-6), ref, rtol=1e-5, atol=1e-5)
    y = oracle.layernorm(x)
    assert np.allclose(y.mean(axis=1), 0, atol=1e-5)
    assert np.allclose(y.var(axis=1), 1, atol=1e-3)
    assert np.array_equal(oracle.layernorm(np.full((2, 8), 5.0, np.float32)), np.zeros((2, 8), np.float32))


def test_silu_matches_torch_and_closed_forms():
    import oracle
    import torch

    x = np.linspace(-20, 20, 4001, dtype=np.float32)
    assert np.allclose(oracle.silu(x), torch.nn.functional.silu(torch.from_numpy(x)).numpy(),
                       rtol=1e-6, atol=1e-7)
    assert oracle.silu(np.zeros(1, np.float32))[0] == 0.0
    assert abs(oracle.silu(np.float32([30.0]))[0] - 30.0) < 1e-5


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_round_to_matches_torch_casts(orc, dt):
    import oracle
    import torch

    x = np.random.default_rng(1).standard_normal(10000).astype(np.float32) * 100
    code = {"bf16": oracle.BF16, "f16": oracle.F16, "f32": oracle.F32}[dt]
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dt]
    want = torch.from_numpy(x).to(tdt).float().numpy()
    assert np.array_equal(oracle.round_to(orc, x, code), want)


def test_group_norm_items_matches_torch():
    """Per batch item, torch's group_norm over [1, C, rows] -- what the
    reference's SparseGroupNorm runs (modules/sparse/norm.py:19-31)."""
    import oracle
    import torch

    rng = np.random.default_rng(3)
    sizes = [37, 120, 5]
    a = (rng.standard_normal((sum(sizes), 64)) * 2 + 0.3).astype(np.float32)
    offs = np.concatenate([[0], np.cumsum(sizes)])
    g = rng.standard_normal(64).astype(np.float32)
    b = rng.standard_normal(64).astype(np.float32)
    got = oracle.group_norm_items(a, offs, 32, g, b, 1e-5)
    for k in range(3):
        blk = torch.from_numpy(a[offs[k]:offs[k + 1]]).T.reshape(1, 64, -1)
        ref = torch.nn.functional.group_norm(blk, 32, torch.from_numpy(g), torch.from_numpy(b),
                                             eps=1e-5).reshape(64, -1).T.numpy()
        assert np.allclose(got[offs[k]:offs[k + 1]], ref, rtol=1e-5, atol=1e-5)
    # closed form: a constant group normalises to 0 (then + beta)
    z = oracle.group_norm_items(np.ones((4, 64), np.float32), np.array([0, 4]), 32, None, b)
    assert np.allclose(z, np.broadcast_to(b, z.shape))
    assert np.array_equal(oracle.batch_offsets(np.array([0, 0, 1, 3, 3])), [0, 2, 3, 3, 5])


def test_tap_merge_matrix_reproduces_child_conv(spc, orc):
    """The merged-tap form of the subdivided child conv (8 parent taps per
    child class with summed weights) equals the 27-tap conv over the copied
    rows on the oracle's child table (F64, every batch / boundary case of a
    random support)."""
    import importlib

    import oracle

    blocks = importlib.import_module(spc.__name__ + ".blocks")
    rng = np.random.default_rng(3)
    coords = oracle_voxels(rng)
    npar = coords.shape[0]
    child, par = orc.subdivide(coords)
    ptab = orc.conv_table_slat(coords).reshape(npar, 27)
    ctab = orc.conv_table_slat(child).reshape(-1, 27)
    ci, co = 5, 3
    w = rng.standard_normal((co, 27, ci))
    xp = rng.standard_normal((npar, ci))
    xc = np.vstack([xp[par], np.zeros((1, ci))])           # row nc = missing
    y27 = np.einsum("oci,noi->nc", w.transpose(1, 0, 2), xc[ctab])
    m = blocks._tap_merge_matrix().numpy()
    wm = np.einsum("vo,coi->vci", m, w)                     # [64, co, ci]
    xq = np.vstack([xp, np.zeros((1, ci))])                 # row npar = missing
    nc = child.shape[0]
    c = np.arange(nc)
    p, d = c // 8, c % 8
    y8 = np.zeros((nc, co))
    for t in range(8):
        j = [(d >> 2) - 1 + (t >> 2), ((d >> 1) & 1) - 1 + ((t >> 1) & 1), (d & 1) - 1 + (t & 1)]
        o = (j[0] + 1) * 9 + (j[1] + 1) * 3 + (j[2] + 1)
        q = ptab[p, o]
        y8 += np.einsum("nci,ni->nc", wm[d * 8 + t], xq[q])
    assert np.allclose(y8, y27, rtol=1e-12, atol=1e-12)


def oracle_voxels(rng):
    """Two batch items of random voxels in a 6^3 box (boundaries included)."""
    pts = []
    for b in range(2):
        v = np.unique(rng.integers(0, 6, size=(60, 3)), axis=0)
        pts.append(np.hstack([np.full((v.shape[0], 1), b), v]))
    return np.ascontiguousarray(np.vstack(pts), dtype=np.int32)


def _io_params(rng, ci, co):
    f = lambda *s: (rng.standard_normal(s) * 0.05).astype(np.float32)  # noqa: E731
    p = {"norm1_w": 1 + f(ci), "norm1_b": f(ci), "conv1_w": f(co, 27, ci), "conv1_b": f(co),
         "conv2_w": f(co, 27, co), "conv2_b": f(co)}
    if ci != co:
        p["skip_w"], p["skip_b"] = f(co, ci), f(co)
    return p


def test_io_res_block_sampling_closed_forms(orc, spc):
    """io_res_block's sampling step, F32: "down" runs res_block on the
    coarse rows np.unique gives (lexicographic (b, x//2, y//2, z//2)) with
    features sum(children) / (|children| + 1) -- torch scatter_reduce 'mean'
    over a zero-initialised output counts the initial zero (SP/spatial.py:
    37-49); "up" runs it on the fine rows with each fine row's coarse
    parent's features (SP/spatial.py:92)."""
    import oracle

    rng = np.random.default_rng(5)
    fine = spc.workloads.random_voxels(900, 12, batches=2, seed=5)
    nf = fine.shape[0]
    x = rng.standard_normal((nf, 32)).astype(np.float32)
    p = _io_params(rng, 32, 64)
    scale = (rng.standard_normal((2, 64)) * 0.2).astype(np.float32)
    shift = (rng.standard_normal((2, 64)) * 0.2).astype(np.float32)
    key = np.concatenate([fine[:, :1], fine[:, 1:] // 2], 1)
    cc, inv = np.unique(key, axis=0, return_inverse=True)
    inv = inv.reshape(-1)
    sums = np.zeros((cc.shape[0], 32), np.float64)
    np.add.at(sums, inv, x)
    xc = (sums / (np.bincount(inv, minlength=cc.shape[0]) + 1)[:, None]).astype(np.float32)
    oc, got = oracle.io_res_block(orc, x, fine, p, scale, shift, oracle.F32, mode="down")
    assert np.array_equal(oc, cc.astype(np.int32))
    want = oracle.res_block(orc, xc, orc.conv_table_slat(oc), p, scale, shift,
                            oc[:, 0].astype(np.int64), oracle.F32)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-5)
    # up: coarse features broadcast to the fine rows
    xu = rng.standard_normal((cc.shape[0], 32)).astype(np.float32)
    oc2, got2 = oracle.io_res_block(orc, xu, cc.astype(np.int32), p, scale, shift, oracle.F32,
                                    mode="up", fine_coords=fine)
    assert np.array_equal(oc2, fine)
    want2 = oracle.res_block(orc, xu[inv], orc.conv_table_slat(fine), p, scale, shift,
                             fine[:, 0].astype(np.int64), oracle.F32)
    assert np.array_equal(got2, want2)


def test_subdivide_block_row_sampling_and_blocked_conv(orc, spc):
    """oracle.subdivide_block's `rows` option returns exactly those rows of
    the whole block, and its threaded, vectorised convs give the scalar
    loop's values -- so the large-width GPU checks that sample rows with the
    fast convs compare against the same block."""
    import oracle

    co = spc.workloads.random_voxels(300, 10, batches=2, seed=3)
    n = co.shape[0]
    rng = np.random.default_rng(0)
    cin, cout = 64, 32

    def nrm(mu, sd, shape):
        return rng.normal(mu, sd, shape).astype(np.float32)

    p = {"gn0_w": nrm(1, .1, cin), "gn0_b": nrm(0, .1, cin),
         "conv1_w": nrm(0, .02, (cout, 27, cin)), "conv1_b": nrm(0, .01, cout),
         "gn1_w": nrm(1, .1, cout), "gn1_b": nrm(0, .1, cout),
         "conv2_w": nrm(0, .02, (cout, 27, cout)), "conv2_b": nrm(0, .01, cout),
         "skip_w": nrm(0, .02, (cout, 1, 1, 1, cin)), "skip_b": nrm(0, .01, cout)}
    x = oracle.round_to(orc, nrm(0, 1, (n, cin)), oracle.BF16)
    c1, full = oracle.subdivide_block(orc, x, co, p, 32, oracle.BF16)
    rows = np.sort(rng.choice(8 * n, 100, replace=False))
    c2, part = oracle.subdivide_block(orc, x, co, p, 32, oracle.BF16, nthreads=4, blocked=True,
                                      rows=rows)
    assert np.array_equal(c1, c2)
    assert np.array_equal(full[rows], part)
    assert full.shape == (8 * n, cout)
