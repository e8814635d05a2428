"""GPU kernel-map parity: every table bit-exact with the oracle (which is
itself pinned to the reference's compiled SlatTables / MeshTables in
tests/test_oracle_maps.py and to the golden fixtures)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[case] {name}", flush=True)


def _coord_sets(spc):
    wl = spc.workloads
    return {
        "sphere64": wl.sphere_shell(),
        "ellipsoids4": wl.ellipsoid_batch(),
        "random_dups_unsorted": np.ascontiguousarray(
            np.concatenate([wl.random_voxels(900, 10, batches=3, seed=5, sort=False),
                            wl.random_voxels(300, 10, batches=3, seed=5, sort=False)[:150]])),
        "single": np.array([[0, 5, 5, 5]], np.int32),
        "ragged_193": wl.random_voxels(193, 7, batches=2, seed=9),
    }


@pytest.mark.parametrize("dense", [False, True])
@pytest.mark.parametrize("name", ["sphere64", "ellipsoids4", "random_dups_unsorted", "single",
                                  "ragged_193"])
def test_map_build_matches_oracle(spc, orc, dev, name, dense):
    """Hash-table and dense-grid builds, bit-exact with the oracle (the
    compiled reference's SlatTables)."""
    import torch

    coords = _coord_sets(spc)[name]
    _case(f"map_build {name} N={coords.shape[0]} dense={dense}")
    n = coords.shape[0]
    tm_ref = orc.conv_table_slat(coords)
    om_ref, ms_ref, ar_ref = orc.spconv_tables(tm_ref, n)
    ext = (int(coords[:, 0].max()) + 1, int(coords[:, 1:].max()) + 1) if dense else None
    m = spc._native.map_build(torch.from_numpy(coords).to(dev), dense=ext)
    assert np.array_equal(m.token_major.cpu().numpy(), tm_ref)
    assert np.array_equal(m.offset_major.cpu().numpy(), om_ref)
    assert np.array_equal(m.mask_sorted.cpu().numpy(), ms_ref)
    assert np.array_equal(m.argsort.cpu().numpy(), ar_ref)
    mn = m.mask_natural.cpu().numpy()
    assert np.array_equal(mn[ar_ref], ms_ref)


def test_map_kat_sparse_tables_test(spc, dev):
    """KAT of the reference's sparse_tables_test.cpp:11-27."""
    import torch

    _case("map_build KAT sparse_tables_test")
    coords = np.array([[0, 0, 0, 0], [0, 1, 0, 0], [0, 3, 0, 0]], np.int32)
    m = spc._native.map_build(torch.from_numpy(coords).to(dev))
    assert m.mask_sorted.cpu().tolist() == [1 << 13, (1 << 4) | (1 << 13), (1 << 13) | (1 << 22)]
    assert m.argsort.cpu().tolist() == [2, 1, 0]


def test_map_mesh_errors(spc, dev):
    import torch

    nat = spc._native
    _case("map_build mesh errors")
    ok = np.array([[0, 1, 2, 3], [0, 1, 2, 4]], np.int32)
    m = nat.map_build(torch.from_numpy(ok).to(dev), mesh_resolution=8)
    assert m.token_major.cpu().numpy().reshape(2, 27)[0, 14] == 1
    dup = np.array([[0, 1, 2, 3], [0, 1, 2, 3]], np.int32)
    with pytest.raises(nat.SparseConvError) as e:
        nat.map_build(torch.from_numpy(dup).to(dev), mesh_resolution=8)
    assert e.value.status == nat.DUP_COORD
    oor = np.array([[0, 1, 2, 8]], np.int32)
    with pytest.raises(nat.SparseConvError) as e:
        nat.map_build(torch.from_numpy(oor).to(dev), mesh_resolution=8)
    assert e.value.status == nat.BAD_COORD
    neg = np.array([[0, -1, 2, 3]], np.int32)
    with pytest.raises(nat.SparseConvError) as e:
        nat.map_build(torch.from_numpy(neg).to(dev))
    assert e.value.status == nat.BAD_COORD
    # the dense grid: mesh duplicates, coordinates or batches beyond the bound
    with pytest.raises(nat.SparseConvError) as e:
        nat.map_build(torch.from_numpy(dup).to(dev), mesh_resolution=8, dense=(1, 8))
    assert e.value.status == nat.DUP_COORD
    m = nat.map_build(torch.from_numpy(ok).to(dev), mesh_resolution=8, dense=(1, 8))
    assert m.token_major.cpu().numpy().reshape(2, 27)[0, 14] == 1
    for bad, ext in ((oor, (1, 8)), (neg, (1, 8)), (np.array([[1, 1, 2, 3]], np.int32), (1, 8))):
        with pytest.raises(nat.SparseConvError) as e:
            nat.map_build(torch.from_numpy(bad).to(dev), dense=ext)
        assert e.value.status == nat.BAD_COORD


def test_map_build_domain_edges(spc, orc, dev):
    """Voxels at both ends of the accepted domain (x, y, z in [0, 32768), b in
    [0, 262144)): a neighbour past an end is absent, no two keys alias (the
    oracle keys on the full integers), and one past either end is
    BAD_COORD."""
    import torch

    nat = spc._native
    _case("map_build domain edges")
    rng = np.random.default_rng(11)
    vals = np.array([0, 1, 2, 32765, 32766, 32767])
    pts = np.stack(np.meshgrid(vals, vals, vals, indexing="ij"), -1).reshape(-1, 3)
    parts = []
    for b in (0, 1, 262142, 262143):
        keep = pts[rng.random(len(pts)) < 0.7]
        parts.append(np.concatenate([np.full((len(keep), 1), b), keep], 1))
    coords = np.ascontiguousarray(np.concatenate(parts), dtype=np.int32)
    n = coords.shape[0]
    tm_ref = orc.conv_table_slat(coords)
    om_ref, ms_ref, ar_ref = orc.spconv_tables(tm_ref, n)
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    assert np.array_equal(m.token_major.cpu().numpy(), tm_ref)
    assert np.array_equal(m.offset_major.cpu().numpy(), om_ref)
    assert np.array_equal(m.mask_sorted.cpu().numpy(), ms_ref)
    assert np.array_equal(m.argsort.cpu().numpy(), ar_ref)
    for bad in ([0, 32768, 0, 0], [0, 0, 32768, 0], [0, 0, 0, 32768], [262144, 0, 0, 0]):
        c = np.array([[0, 5, 5, 5], bad], np.int32)
        with pytest.raises(nat.SparseConvError) as e:
            nat.map_build(torch.from_numpy(c).to(dev))
        assert e.value.status == nat.BAD_COORD
    with pytest.raises(nat.SparseConvError) as e:  # 2^63 cells: refused on the host
        nat.map_build(torch.from_numpy(coords).to(dev), dense=(262144, 32768))
    assert e.value.status == nat.BAD_SHAPE


def test_mesh_levels_match_oracle(spc, orc, dev):
    """Config-4 subdivision (seeded 50% pruning) and the mesh conv tables."""
    import torch

    wl = spc.workloads
    nat = spc._native
    c0 = wl.sphere_shell()
    keeps = wl.prune_masks(c0.shape[0])
    coords, res = c0, 64
    for lvl, keep in enumerate(keeps, start=1):
        _case(f"subdivide level {lvl} from N={coords.shape[0]}")
        ref_c, ref_p = orc.subdivide(coords, keep)
        oc, par = nat.subdivide_map(torch.from_numpy(coords).to(dev),
                                    torch.from_numpy(keep).to(dev))
        assert np.array_equal(oc.cpu().numpy(), ref_c)
        assert np.array_equal(par.cpu().numpy(), ref_p)
        res *= 2
        st, tm_ref = orc.conv_table_mesh(ref_c, res)
        assert st == 0
        m = nat.map_build(oc, mesh_resolution=res)
        assert np.array_equal(m.token_major.cpu().numpy(), tm_ref)
        coords = ref_c
    assert coords.shape[0] == 347860


def test_subdivide_unpruned(spc, orc, dev):
    import torch

    _case("subdivide unpruned")
    c = spc.workloads.random_voxels(500, 16, batches=2, seed=3)
    ref_c, ref_p = orc.subdivide(c)
    oc, par = spc._native.subdivide_map(torch.from_numpy(c).to(dev))
    assert np.array_equal(oc.cpu().numpy(), ref_c)
    assert np.array_equal(par.cpu().numpy(), ref_p)
    # queued without the status read-back: the same rows
    oq, pq = spc._native.subdivide_map(torch.from_numpy(c).to(dev), sync=False)
    assert np.array_equal(oq.cpu().numpy(), ref_c)
    assert np.array_equal(pq.cpu().numpy(), ref_p)


def test_subdivide_range_status(spc, dev):
    """A parent coordinate at 2^14 would put children past the 2^15 grid:
    the synchronising call returns BAD_COORD; the queued one returns OK and
    leaves BAD_COORD in the workspace's status word for spc_read_status."""
    import ctypes

    import torch

    nat = spc._native
    L = nat.lib()
    _case("subdivide range status")
    c = torch.tensor([[0, 3, 4, 5], [0, 1 << 14, 2, 2]], dtype=torch.int32, device=dev)
    with pytest.raises(nat.SparseConvError):
        nat.subdivide_map(c)
    oc = torch.empty((16, 4), dtype=torch.int32, device=dev)
    par = torch.empty(16, dtype=torch.int32, device=dev)
    ws = torch.empty(L.spc_subdivide_workspace_bytes(2), dtype=torch.uint8, device=dev)
    m = ctypes.c_int64(0)
    s = torch.cuda.current_stream(dev).cuda_stream
    st = L.spc_subdivide_map(ctypes.c_void_p(s), ctypes.c_void_p(c.data_ptr()), 2, None, 0,
                             ctypes.c_void_p(oc.data_ptr()), ctypes.c_void_p(par.data_ptr()),
                             ctypes.byref(m), ctypes.c_void_p(ws.data_ptr()), ws.numel())
    assert st == nat.OK and m.value == 16
    assert L.spc_read_status(ctypes.c_void_p(s), ctypes.c_void_p(ws.data_ptr())) == nat.BAD_COORD
    # the in-range parent's children are written all the same
    assert oc[:8].cpu().tolist() == [[0, 6 + d // 4, 8 + (d // 2) % 2, 10 + d % 2] for d in range(8)]


@pytest.mark.parametrize("name", ["sphere64", "ellipsoids4", "ragged_193"])
def test_downsample_map_matches_oracle(spc, orc, dev, name):
    import torch

    coords = _coord_sets(spc)[name]
    _case(f"downsample_map {name}")
    ref = orc.downsample_map(coords)
    taps_ref = orc.stride2_taps(coords, ref["fine_to_coarse"], ref["nc"])
    nb = int(coords[:, 0].max()) + 1
    d = spc._native.downsample_map(torch.from_numpy(coords).to(dev), nb, 64)
    assert d.nc == ref["nc"]
    assert np.array_equal(d.fine_to_coarse.cpu().numpy(), ref["fine_to_coarse"])
    assert np.array_equal(d.coarse_coords.cpu().numpy(), ref["coarse_coords"])
    assert np.array_equal(d.children.cpu().numpy(), ref["children"])
    assert np.array_equal(d.counts.cpu().numpy(), ref["counts"])
    assert np.array_equal(d.stride2_taps.cpu().numpy(), taps_ref)


@pytest.mark.parametrize("name", ["sphere64", "ellipsoids4", "random_dups_unsorted", "single",
                                  "ragged_193"])
def test_subdivide_neighbors_matches_child_map(spc, orc, dev, name):
    """The child table derived from the parents' table equals the hash-built
    table of the subdivided coordinates and the oracle's table, duplicates
    (first-row rule) and batch boundaries included."""
    import torch

    nat = spc._native
    coords = _coord_sets(spc)[name]
    n = coords.shape[0]
    _case(f"subdivide_neighbors {name} np={n}")
    c = torch.from_numpy(coords).to(dev)
    pm = nat.map_build(c, outputs="token")
    child, par = nat.subdivide_map(c)
    got = nat.subdivide_neighbors(pm.token_major, n).token_major
    want = nat.map_build(child.contiguous(), outputs="token").token_major
    assert torch.equal(got, want)
    ref = orc.conv_table_slat(child.cpu().numpy())
    assert np.array_equal(got.cpu().numpy().reshape(-1), ref.reshape(-1))


def test_large_subdivided_shell_maps(spc, dev):
    """The 256^3 level of the mesh decoder (sphere shell subdivided twice,
    1.39M voxels): the hash-built table satisfies the closed-form invariants
    (centre tap = self, symmetry nbr(i, o) = j <=> nbr(j, 26 - o) = i, masks =
    valid taps, argsort stable by mask) and equals the table derived from the
    128^3 parents' table."""
    import torch

    nat = spc._native
    kids = np.array([[0, dx, dy, dz] for dx in (0, 1) for dy in (0, 1) for dz in (0, 1)], np.int32)
    up = lambda c: (c[:, None, :] * np.array([1, 2, 2, 2], np.int32) + kids[None]).reshape(-1, 4)  # noqa: E731
    par = np.ascontiguousarray(up(spc.workloads.sphere_shell()), dtype=np.int32)
    child = np.ascontiguousarray(up(par), dtype=np.int32)
    n, npar = child.shape[0], par.shape[0]
    _case(f"large maps: {npar} parents at 128^3 -> {n} children at 256^3")
    m = nat.map_build(torch.from_numpy(child).to(dev))
    assert torch.equal(nat.map_build(torch.from_numpy(child).to(dev), outputs="token",
                                     dense=(1, 256)).token_major, m.token_major)
    pm = nat.map_build(torch.from_numpy(par).to(dev))
    # the parents' mask sort: 86 tiles of 2,048 keys, past the 64 tiles whose
    # counts each downsweep block reads in one batch
    pmask = ((pm.token_major.cpu().numpy().reshape(npar, 27) < npar) << np.arange(27)).sum(1)
    assert np.array_equal(pm.argsort.cpu().numpy(), np.argsort(pmask, kind="stable"))
    assert np.array_equal(pm.mask_sorted.cpu().numpy(), pmask[np.argsort(pmask, kind="stable")])
    derived = nat.subdivide_neighbors(pm.token_major, npar).token_major
    assert torch.equal(derived, m.token_major)
    tm = m.token_major.cpu().numpy().reshape(n, 27)
    assert np.array_equal(tm[:, 13], np.arange(n))
    i, o = np.nonzero(tm < n)
    j = tm[i, o]
    assert np.array_equal(tm[j, 26 - o], i)
    om = m.offset_major.cpu().numpy().reshape(27, n)
    assert np.array_equal(np.where(tm < n, tm, -1).T, om)
    mask = ((tm < n) << np.arange(27)).sum(1)
    assert np.array_equal(m.mask_natural.cpu().numpy(), mask)
    ar = m.argsort.cpu().numpy()
    assert np.array_equal(ar, np.argsort(mask, kind="stable"))
    assert np.array_equal(m.mask_sorted.cpu().numpy(), mask[ar])
