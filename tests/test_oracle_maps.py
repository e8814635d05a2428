"""Pins the oracle's map builders (CPU): against the golden fixtures written
from the reference's own compiled SlatTables / MeshTables, against
oracle/_ref directly where it was built, against the reference tests' KATs,
and against invariants and brute force that a plausible mistake (a wrong
offset decode, an unstable sort, a transposed table) would break."""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = json.loads((Path(__file__).parent / "golden" / "maps_golden.json").read_text())


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def oracle_slat(orc, c):
    n = c.shape[0]
    tm = orc.conv_table_slat(c)
    om, ms, ar = orc.spconv_tables(tm, n)
    ds = orc.downsample_map(c)
    ctm = orc.conv_table_slat(ds["coarse_coords"])
    com, cms, car = orc.spconv_tables(ctm, ds["nc"])
    return {"conv_fine": tm, "conv_fine_spconv": om, "fine_mask": ms, "fine_argsort": ar,
            "fine_to_coarse": ds["fine_to_coarse"], "coarse_children": ds["children"],
            "coarse_count": ds["counts"], "conv_coarse": ctm, "conv_coarse_spconv": com,
            "coarse_mask": cms, "coarse_argsort": car, "nc": ds["nc"]}


def _large_sets(spc):
    wl = spc.workloads
    o = oracle.orc()
    c0 = wl.sphere_shell()
    keeps = wl.prune_masks(c0.shape[0])
    c1, _ = o.subdivide(c0, keeps[0])
    c2, _ = o.subdivide(c1, keeps[1])
    return {"sphere64": c0, "ellipsoids4": wl.ellipsoid_batch(), "mesh128_pruned": c1,
            "mesh256_pruned": c2}


@pytest.fixture(scope="module")
def large_sets(spc):
    return _large_sets(spc)


@pytest.mark.parametrize("name", ["sphere64", "ellipsoids4", "mesh128_pruned", "mesh256_pruned"])
def test_oracle_matches_golden_large(orc, large_sets, name):
    g = GOLDEN["large"][name]
    c = large_sets[name]
    assert sha(c) == g["coords_sha256"], "workload generator drifted"
    t = oracle_slat(orc, c)
    assert t["nc"] == g["nc"]
    for k, v in g.items():
        if k in t and k != "nc":
            assert sha(t[k]) == v, k


def test_workload_sizes(large_sets):
    """Sizes quoted for the configs (shell rule |d - r| <= 1.5, seeds 2024/7)."""
    assert large_sets["sphere64"].shape[0] == 21766
    assert large_sets["ellipsoids4"].shape[0] == 62710
    assert large_sets["mesh128_pruned"].shape[0] == 86922
    assert large_sets["mesh256_pruned"].shape[0] == 347860
    assert GOLDEN["large"]["sphere64"]["pairs"] == 453614
    assert GOLDEN["large"]["ellipsoids4"]["pairs"] == 1306542


@pytest.mark.parametrize("name", list(GOLDEN["small"].keys()))
def test_oracle_matches_golden_small(orc, name):
    g = GOLDEN["small"][name]
    c = np.array(g["coords"], np.int32)
    t = oracle_slat(orc, c)
    assert t["nc"] == g["nc"]
    for k in ["conv_fine", "conv_fine_spconv", "fine_mask", "fine_argsort", "fine_to_coarse",
              "coarse_children", "conv_coarse", "conv_coarse_spconv", "coarse_mask",
              "coarse_argsort"]:
        assert t[k].tolist() == g[k], k
    assert np.array_equal(t["coarse_count"], np.array(g["coarse_count"], np.float32))


def test_kat_sparse_tables_test(orc):
    """SRC/sparse_tables_test.cpp:11-27 of the reference."""
    c = np.array([[0, 0, 0, 0], [0, 1, 0, 0], [0, 3, 0, 0]], np.int32)
    tm = orc.conv_table_slat(c)
    _, ms, ar = orc.spconv_tables(tm, 3)
    assert ms.tolist() == [1 << 13, (1 << 4) | (1 << 13), (1 << 13) | (1 << 22)]
    assert ar.tolist() == [2, 1, 0]
    assert np.all(np.diff(ms) >= 0)


@pytest.mark.parametrize("name", list(GOLDEN["mesh"].keys()))
def test_mesh_tables_golden(orc, name):
    """MeshTables::build (two unpruned subdivisions + mesh conv tables)."""
    g = GOLDEN["mesh"][name]
    c0 = np.array(g["coords"], np.int32)
    res = g["base_resolution"]
    st, t0 = orc.conv_table_mesh(c0, res)
    assert st == 0 and t0.tolist() == g["conv0"]
    c1, p1 = orc.subdivide(c0)
    c2, p2 = orc.subdivide(c1)
    assert [c0.shape[0], c1.shape[0], c2.shape[0]] == g["sizes"]
    assert sha(c1) == g["coords1_sha256"] and sha(c2) == g["coords2_sha256"]
    assert c2[0].tolist() == g["coords2_first"] and c2[-1].tolist() == g["coords2_last"]
    st1, t1 = orc.conv_table_mesh(c1, res * 2)
    st2, t2 = orc.conv_table_mesh(c2, res * 4)
    assert st1 == 0 and st2 == 0
    assert sha(t1) == g["conv1_sha256"] and sha(t2) == g["conv2_sha256"]
    assert np.array_equal(p1, np.arange(c1.shape[0]) // 8)


def test_kat_mesh_tables_test(orc):
    """SRC/mesh_tables_test.cpp:6-35: (0,1,2,3) -> 1/8/64 voxels, first child
    (0,4,8,12), last (0,7,11,15), centre tap maps to itself."""
    c0 = np.array([[0, 1, 2, 3]], np.int32)
    c1, _ = orc.subdivide(c0)
    c2, _ = orc.subdivide(c1)
    assert (c1.shape[0], c2.shape[0]) == (8, 64)
    assert c2[0].tolist() == [0, 4, 8, 12] and c2[-1].tolist() == [0, 7, 11, 15]
    st, t2 = orc.conv_table_mesh(c2, 256)
    assert st == 0
    assert np.array_equal(t2.reshape(64, 27)[:, 13], np.arange(64))


def test_mesh_errors(orc):
    """build_mesh_conv_table rejects out-of-range and duplicate coordinates
    (SRC/sparse_ops.cpp:319-328)."""
    st, _ = orc.conv_table_mesh(np.array([[0, 0, 0, 64]], np.int32), 64)
    assert st == oracle.BAD_COORD
    st, _ = orc.conv_table_mesh(np.array([[0, -1, 0, 0]], np.int32), 64)
    assert st == oracle.BAD_COORD
    st, _ = orc.conv_table_mesh(np.array([[0, 1, 1, 1], [0, 1, 1, 1]], np.int32), 64)
    assert st == oracle.DUP_COORD


def brute_force_table(c):
    """O(N^2 * 27) scan: first row with coord + delta in the same batch."""
    n = c.shape[0]
    out = np.full((n, 27), n, np.int64)
    first = {}
    for i, row in enumerate(map(tuple, c.tolist())):
        first.setdefault(row, i)
    for i, (b, x, y, z) in enumerate(c.tolist()):
        if first[(b, x, y, z)] != i:
            continue  # a later duplicate keeps its sentinels
        for o in range(27):
            k = (b, x + o // 9 - 1, y + (o // 3) % 3 - 1, z + o % 3 - 1)
            if k in first:
                out[i, o] = first[k]
    return out.reshape(-1)


def test_brute_force_with_duplicates(spc, orc):
    wl = spc.workloads
    c = np.ascontiguousarray(np.concatenate([wl.random_voxels(120, 5, batches=2, seed=4, sort=False),
                                             wl.random_voxels(120, 5, batches=2, seed=4,
                                                              sort=False)[:30]]))
    assert np.array_equal(orc.conv_table_slat(c), brute_force_table(c))


def test_invariants(spc, orc):
    c = spc.workloads.random_voxels(3000, 18, batches=3, seed=8)
    n = c.shape[0]
    tm = orc.conv_table_slat(c).reshape(n, 27)
    # centre tap is the row itself (unique coords)
    assert np.array_equal(tm[:, 13], np.arange(n))
    # symmetry: nbr(i, o) = j  <=>  nbr(j, 26 - o) = i
    i, o = np.nonzero(tm < n)
    j = tm[i, o]
    assert np.array_equal(tm[j, 26 - o], i)
    om, ms, ar = orc.spconv_tables(tm.reshape(-1), n)
    # popcounts of the masks add up to the pairs
    pop = np.array([bin(int(m)).count("1") for m in ms])
    assert pop.sum() == (tm < n).sum()
    # argsort is a permutation, masks ascend, ties keep token order
    assert np.array_equal(np.sort(ar), np.arange(n))
    assert np.all(np.diff(ms) >= 0)
    same = np.diff(ms) == 0
    assert np.all(np.diff(ar)[same] > 0)
    # offset-major is the transpose with -1 for missing
    tt = np.where(tm < n, tm, -1).T.reshape(-1)
    assert np.array_equal(om, tt)


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref needs the reference tree")
def test_oracle_vs_reference_direct(spc, orc):
    """Direct comparison with the compiled reference on fresh random sets,
    including unsorted input with duplicates."""
    wl = spc.workloads
    ref = oracle.ref()
    for seed in range(4):
        c = wl.random_voxels(2000, 12, batches=3, seed=100 + seed, sort=seed % 2 == 0,
                             unique=seed < 2)
        t = ref.slat_tables(c)
        o = oracle_slat(orc, c)
        for k in ["conv_fine", "conv_fine_spconv", "fine_mask", "fine_argsort", "fine_to_coarse",
                  "coarse_children", "coarse_count", "conv_coarse", "conv_coarse_spconv",
                  "coarse_mask", "coarse_argsort"]:
            assert np.array_equal(o[k], t[k]), (seed, k)


def test_downsample_closed_form(spc, orc):
    """Coarse rows are the sorted unique (b, x//2, y//2, z//2) (torch
    unique order, SP/spatial.py:28-34); counts = children + 1."""
    c = spc.workloads.random_voxels(1500, 16, batches=2, seed=12)
    d = orc.downsample_map(c)
    key = np.concatenate([c[:, :1], c[:, 1:] // 2], 1)
    uniq, inv, cnt = np.unique(key, axis=0, return_inverse=True, return_counts=True)
    assert np.array_equal(d["coarse_coords"], uniq)
    assert np.array_equal(d["fine_to_coarse"], inv.reshape(-1))
    assert np.array_equal(d["counts"], (cnt + 1).astype(np.float32))
    ch = d["children"].reshape(-1, 8)
    for r in range(d["nc"]):
        kids = np.nonzero(inv.reshape(-1) == r)[0]
        assert ch[r, : len(kids)].tolist() == kids.tolist()
        assert np.all(ch[r, len(kids):] == c.shape[0])


def test_stride2_taps_closed_form(spc, orc):
    c = spc.workloads.random_voxels(1500, 16, batches=2, seed=13)
    d = orc.downsample_map(c)
    taps = orc.stride2_taps(c, d["fine_to_coarse"], d["nc"]).reshape(-1, 8)
    for i, (b, x, y, z) in enumerate(c.tolist()):
        k = (x & 1) * 4 + (y & 1) * 2 + (z & 1)
        assert taps[d["fine_to_coarse"][i], k] == i
    assert (taps < c.shape[0]).sum() == c.shape[0]


def test_subdivide_keep_closed_form(spc, orc):
    """orc_subdivide with a keep mask is the unpruned subdivision (itself
    pinned by MeshTables::build above: torch.nonzero child order, row p*8 +
    c) filtered by the mask in row order, with each survivor's parent =
    unpruned row // 8 -- for random masks, the all-kept and all-dropped
    masks and the config-4 seeded masks."""
    c0 = spc.workloads.random_voxels(700, 20, batches=3, seed=21)
    full, fpar = orc.subdivide(c0)
    assert np.array_equal(fpar, np.arange(full.shape[0]) // 8)
    rng = np.random.default_rng(22)
    for keep in (rng.random(full.shape[0]) < 0.5, rng.random(full.shape[0]) < 0.05,
                 np.ones(full.shape[0], bool)):
        k = keep.astype(np.uint8)
        got_c, got_p = orc.subdivide(c0, k)
        sel = np.nonzero(keep)[0]
        assert np.array_equal(got_c, full[sel])
        assert np.array_equal(got_p, sel // 8)
    got_c, got_p = orc.subdivide(c0, np.zeros(full.shape[0], np.uint8))  # nothing survives
    assert got_c.shape == (0, 4) and got_p.shape == (0,)
    # the config-4 levels: the seeded masks, level by level
    lvl = spc.workloads.sphere_shell()
    for keep in spc.workloads.prune_masks(lvl.shape[0]):
        full, _ = orc.subdivide(lvl)
        got_c, got_p = orc.subdivide(lvl, keep)
        sel = np.nonzero(keep)[0]
        assert np.array_equal(got_c, full[sel]) and np.array_equal(got_p, sel // 8)
        lvl = got_c
    assert lvl.shape[0] == 347860


@pytest.mark.parametrize("dims,lo,hi", [((2, 256, 60), 0, 32768), ((2, 768, 60), 32768, 65536),
                                        ((2, 1120, 60), 65536, 1 << 30)])
def test_dedupe_path_spans(orc, dims, lo, hi):
    """The premise of tests/test_gpu_geometry.py::test_dedupe_paths: in a
    dense 2 x ny x 60 block every 256-row (and 128-row) tile's source rows
    span more than `lo` and at most `hi` rows, and their union fits the
    895-row (511-row) stage."""
    nx, ny, nz = dims
    g = np.stack(np.meshgrid(np.arange(nx), np.arange(ny), np.arange(nz), indexing="ij"),
                 -1).reshape(-1, 3)
    c = np.zeros((g.shape[0], 4), np.int32)
    c[:, 1:] = g
    n = c.shape[0]
    tm = orc.conv_table_slat(c).reshape(n, 27)
    for tile, umax in ((256, 895), (128, 511)):
        for t0 in range(0, n, tile):
            v = tm[t0:t0 + tile]
            v = v[v < n]
            span = int(v.max() - v.min() + 1)
            assert lo < span <= hi, (tile, t0, span)
            assert len(np.unique(v)) <= umax, (tile, t0)
