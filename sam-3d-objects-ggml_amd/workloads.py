"""Seeded synthetic voxel sets for the sparse-conv workloads.

Coordinates are int32 (b, x, y, z), lexicographically sorted within each
object (what torch.argwhere produces, sam3d_objects/pipeline/
inference_pipeline.py:703 in the reference), objects concatenated in batch
order.

Shell rule: a voxel p of the 64^3 grid is active iff its distance to the
surface is at most 1.5 voxels:
  sphere     | ||p - c|| - r | <= 1.5, c = (32, 32, 32), r = 24  (N = 21,766)
  ellipsoid  | (f - 1) / ||grad f|| | <= 1.5,  f = || R^T (p - c) / a ||
The literal "within 1 voxel" rule (<= 1.0) gives N = 14,534 for the sphere.
"""
from __future__ import annotations

import numpy as np

GRID = 64


def _grid(res: int = GRID) -> np.ndarray:
    ax = np.arange(res)
    return np.stack(np.meshgrid(ax, ax, ax, indexing="ij"), -1).reshape(-1, 3)


def sphere_shell(res: int = GRID, radius: float = 24.0, band: float = 1.5, batch: int = 0):
    g = _grid(res)
    c = res / 2.0
    d = np.linalg.norm(g - c, axis=1)
    p = g[np.abs(d - radius) <= band]
    out = np.empty((p.shape[0], 4), np.int32)
    out[:, 0] = batch
    out[:, 1:] = p
    return out


def ellipsoid_shell(axes: np.ndarray, rot: np.ndarray, res: int = GRID, band: float = 1.5,
                    batch: int = 0):
    g = _grid(res).astype(np.float64)
    c = res / 2.0
    u = (g - c) @ rot  # R^T (p - c) for row vectors
    q = u / axes
    f = np.linalg.norm(q, axis=1)
    grad = np.linalg.norm(q / axes, axis=1) / np.maximum(f, 1e-12)
    dist = np.abs(f - 1.0) / np.maximum(grad, 1e-12)
    p = _grid(res)[dist <= band]
    out = np.empty((p.shape[0], 4), np.int32)
    out[:, 0] = batch
    out[:, 1:] = p
    return out


def ellipsoid_batch(n_objects: int = 4, seed: int = 2024) -> np.ndarray:
    """Config-2 coords: per object a ~ U(16, 28)^3 and a Haar rotation drawn
    by scipy from a seed taken off the same generator.  Seed 2024 gives
    N = 62,710 (16,294 / 16,178 / 13,418 / 16,820)."""
    from scipy.spatial.transform import Rotation

    rng = np.random.default_rng(seed)
    parts = []
    for b in range(n_objects):
        a = rng.uniform(16, 28, size=3)
        r = Rotation.random(random_state=int(rng.integers(1 << 31))).as_matrix()
        parts.append(ellipsoid_shell(a, r, batch=b))
    return np.ascontiguousarray(np.concatenate(parts, 0))


def prune_masks(n0: int, seed: int = 7, levels: int = 2, keep_p: float = 0.5):
    """Config-4 child keep masks: level l keeps each of the 8 children of
    every surviving parent with probability keep_p, drawn in parent-major
    order from one generator (seed 7 gives 86,922 and 347,860 voxels)."""
    rng = np.random.default_rng(seed)
    masks = []
    n = n0
    for _ in range(levels):
        k = rng.random(n * 8) < keep_p
        masks.append(k.astype(np.uint8))
        n = int(k.sum())
    return masks


def normal(shape, std: float = 1.0, seed: int = 0) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def random_voxels(n: int, res: int, batches: int = 1, seed: int = 0, sort: bool = True,
                  unique: bool = True) -> np.ndarray:
    """Random voxel sets for edge-case tests (optionally with duplicates)."""
    rng = np.random.default_rng(seed)
    c = np.empty((n, 4), np.int32)
    c[:, 0] = rng.integers(0, batches, n)
    c[:, 1:] = rng.integers(0, res, (n, 3))
    if unique:
        c = np.unique(c, axis=0)
    if sort:
        c = c[np.lexsort((c[:, 3], c[:, 2], c[:, 1], c[:, 0]))]
    return np.ascontiguousarray(c, dtype=np.int32)
