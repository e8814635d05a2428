"""Writes tests/golden/maps_golden.json from the reference's own table builders.

Runs oracle/_ref/libref_tables.so -- the reference's cpp_ggml/src/
sparse_ops.cpp (SlatTables::build, MeshTables::build) compiled from source by
oracle/Makefile -- on the seeded voxel sets of the workloads module and
records:
  * sha256 of every table for the full-size sets (configs 1, 2, 4),
  * full arrays for small sets (<= 512 voxels), including duplicates,
  * the reference test KATs' inputs.
Usage (where the reference tree exists):  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402
import oracle  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


SLAT_KEYS = ["conv_fine", "conv_fine_spconv", "fine_mask", "fine_argsort", "fine_to_coarse",
             "coarse_children", "coarse_count", "conv_coarse", "conv_coarse_spconv",
             "coarse_mask", "coarse_argsort"]


def coord_sets(wl):
    sets = {
        "sphere64": wl.sphere_shell(),
        "ellipsoids4": wl.ellipsoid_batch(),
    }
    c0 = sets["sphere64"]
    keeps = wl.prune_masks(c0.shape[0])
    o = oracle.orc()
    c1, _ = o.subdivide(c0, keeps[0])
    c2, _ = o.subdivide(c1, keeps[1])
    sets["mesh128_pruned"] = c1
    sets["mesh256_pruned"] = c2
    return sets


def small_sets(wl):
    dups = np.concatenate([wl.random_voxels(160, 6, batches=2, seed=21, sort=False),
                           wl.random_voxels(160, 6, batches=2, seed=21, sort=False)[:40]])
    return {
        "kat_sparse_tables_test": np.array([[0, 0, 0, 0], [0, 1, 0, 0], [0, 3, 0, 0]], np.int32),
        "small_sorted_b2": wl.random_voxels(300, 8, batches=2, seed=17),
        "small_unsorted_dups": np.ascontiguousarray(dups, dtype=np.int32),
        "small_dense_cube": np.ascontiguousarray(
            np.stack(np.meshgrid([0], np.arange(5), np.arange(5), np.arange(5), indexing="ij"),
                     -1).reshape(-1, 4).astype(np.int32)),
    }


def main() -> None:
    spc = __graft_entry__.load()
    wl = spc.workloads
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref not built (needs the reference tree): make -C oracle ref")
    ref = oracle.ref()
    out = {"generator": "tests/golden/make_golden.py", "source": "reference SlatTables::build "
           "and MeshTables::build (cpp_ggml/src/sparse_ops.cpp) compiled by oracle/Makefile",
           "large": {}, "small": {}, "mesh": {}}
    for name, c in coord_sets(wl).items():
        t = ref.slat_tables(c)
        out["large"][name] = {"n": int(c.shape[0]), "coords_sha256": sha(c), "nc": t["nc"],
                              "pairs": int((t["conv_fine"] < c.shape[0]).sum()),
                              **{k: sha(t[k]) for k in SLAT_KEYS}}
        print(name, c.shape[0], t["nc"], flush=True)
    for name, c in small_sets(wl).items():
        t = ref.slat_tables(c)
        out["small"][name] = {"coords": c.tolist(), "nc": t["nc"],
                              **{k: t[k].tolist() for k in SLAT_KEYS}}
    # MeshTables (unpruned subdivision x2 + build_mesh_conv_table per level)
    for name, c, res in [("mesh_kat_single", np.array([[0, 1, 2, 3]], np.int32), 64),
                         ("mesh_small_b2", wl.random_voxels(40, 8, batches=2, seed=33), 64)]:
        m = ref.mesh_tables(c, res)
        out["mesh"][name] = {"coords": c.tolist(), "base_resolution": res,
                             "sizes": list(m["sizes"]), "coords1_sha256": sha(m["coords1"]),
                             "coords2_sha256": sha(m["coords2"]), "conv0": m["conv0"].tolist(),
                             "conv1_sha256": sha(m["conv1"]), "conv2_sha256": sha(m["conv2"]),
                             "coords2_first": m["coords2"][0].tolist(),
                             "coords2_last": m["coords2"][-1].tolist()}
    (HERE / "maps_golden.json").write_text(json.dumps(out, separators=(",", ":")))
    print("wrote", HERE / "maps_golden.json")


if __name__ == "__main__":
    main()
