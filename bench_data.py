"""Seeded synthetic voxel clouds for bench.py and the parity tests.

* ``uniform_cloud``: unique voxels drawn uniformly in a grid (config 1).
* ``surface_cloud``: a union of random sphere shells and plane patches,
  voxelised and deduplicated per batch sample (configs 2 and 5) -- about
  1-3 % occupancy of a 256^3 grid at 200k voxels.
* ``lidar_cloud``: ground plane with range fall-off plus random boxes in a
  [41, 1600, 1408] zyx grid (config 3).
* ``urban_cloud``: road plane, building walls and object boxes in a
  [128, 2048, 2048] zyx grid (config 4).

Voxel rows are returned in ascending batch-major linear-key order, the order
a voxeliser followed by a sort (or torch.unique) produces.  Indices are
int32 [N, ndim + 1] with the batch in column 0.
"""

from __future__ import annotations

import numpy as np


def _finish(keys_per_batch, shape):
    rows = []
    for b, keys in enumerate(keys_per_batch):
        c = np.stack(np.unravel_index(keys, shape), 1)
        rows.append(np.concatenate([np.full((c.shape[0], 1), b), c], 1))
    return np.ascontiguousarray(np.concatenate(rows, 0).astype(np.int32))


def uniform_cloud(n: int, shape, seed: int = 0, batch: int = 1) -> np.ndarray:
    rng = np.random.default_rng(seed)
    vol = int(np.prod(shape))
    keys = [np.sort(rng.choice(vol, size=n, replace=False)) for _ in range(batch)]
    return _finish(keys, list(shape))


def _sphere_points(rng, grid, count):
    centre = rng.uniform(0.15, 0.85, 3) * grid
    radius = rng.uniform(0.04, 0.2) * grid
    d = rng.standard_normal((count, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    return centre + radius * d


def _plane_points(rng, grid, count):
    normal = rng.standard_normal(3)
    normal /= np.linalg.norm(normal)
    u = np.cross(normal, [1.0, 0.0, 0.0] if abs(normal[0]) < 0.9 else [0.0, 1.0, 0.0])
    u /= np.linalg.norm(u)
    v = np.cross(normal, u)
    centre = rng.uniform(0.2, 0.8, 3) * grid
    half = rng.uniform(0.05, 0.3) * grid
    a = rng.uniform(-half, half, (count, 1))
    b = rng.uniform(-half, half, (count, 1))
    return centre + a * u + b * v


def surface_cloud(n: int, grid: int = 256, seed: int = 0, batch: int = 1) -> np.ndarray:
    """Exactly n unique surface voxels per sample in a grid^3 volume."""
    shape = [grid] * 3
    out = []
    for b in range(batch):
        rng = np.random.default_rng(seed * 1000 + b)
        keys = np.zeros(0, np.int64)
        while keys.size < n:
            pts = []
            for _ in range(16):
                if rng.random() < 0.5:
                    pts.append(_sphere_points(rng, grid, 60000))
                else:
                    pts.append(_plane_points(rng, grid, 60000))
            p = np.floor(np.concatenate(pts, 0)).astype(np.int64)
            p = p[((p >= 0) & (p < grid)).all(1)]
            keys = np.unique(np.concatenate([keys, np.ravel_multi_index(p.T, shape)]))
        pick = np.sort(rng.choice(keys.size, size=n, replace=False))
        out.append(keys[pick])
    return _finish(out, shape)


def lidar_cloud(per_sample: int = 20000, batch: int = 4, seed: int = 0,
                shape=(41, 1600, 1408)) -> np.ndarray:
    """Ground plane (z ~ 2-4, density falling with range) plus 30 boxes per sample."""
    zdim, ydim, xdim = shape
    out = []
    for b in range(batch):
        rng = np.random.default_rng(seed * 1000 + b)
        keys = np.zeros(0, np.int64)
        while keys.size < per_sample:
            m = 200000
            y = rng.uniform(0, ydim, m)
            x = rng.uniform(0, xdim, m)
            r = np.hypot(y - ydim / 2, x) / np.hypot(ydim / 2, xdim)
            keep = rng.random(m) < 0.6 * (1.0 - r) ** 2
            z = rng.uniform(2, 4, m)
            ground = np.stack([z, y, x], 1)[keep]
            boxes = []
            for _ in range(30):
                ext = rng.uniform(20, 50, 3) * np.array([0.2, 1.0, 1.0])
                c = np.array([rng.uniform(4, zdim - 8), rng.uniform(0, ydim), rng.uniform(0, xdim)])
                face = rng.uniform(-0.5, 0.5, (4000, 3)) * ext
                axis = rng.integers(0, 3, 4000)
                face[np.arange(4000), axis] = np.sign(face[np.arange(4000), axis]) * ext[axis] / 2
                boxes.append(c + face)
            p = np.floor(np.concatenate([ground] + boxes, 0)).astype(np.int64)
            p = p[((p >= 0) & (p < np.asarray(shape))).all(1)]
            keys = np.unique(np.concatenate([keys, np.ravel_multi_index(p.T, shape)]))
        pick = np.sort(rng.choice(keys.size, size=per_sample, replace=False))
        out.append(keys[pick])
    return _finish(out, list(shape))


def urban_cloud(per_sample: int = 120000, batch: int = 2, seed: int = 0,
                shape=(128, 2048, 2048)) -> np.ndarray:
    """Road plane (z ~ 4-6), vertical building walls and object boxes."""
    zdim, ydim, xdim = shape
    out = []
    for b in range(batch):
        rng = np.random.default_rng(seed * 1000 + 500 + b)
        keys = np.zeros(0, np.int64)
        while keys.size < per_sample:
            m = per_sample
            road = np.stack([rng.uniform(4, 6, m), rng.uniform(0, ydim, m), rng.uniform(0, xdim, m)], 1)
            parts = [road]
            for _ in range(12):  # walls: vertical rectangles along y or x
                length = rng.uniform(0.1, 0.5) * max(ydim, xdim)
                height = rng.uniform(0.3, 0.9) * zdim
                c = np.array([0.0, rng.uniform(0, ydim), rng.uniform(0, xdim)])
                t = rng.uniform(-0.5, 0.5, m // 8) * length
                z = rng.uniform(4, 4 + height, m // 8)
                wall = np.stack([z, np.full_like(z, c[1]), c[2] + t], 1)
                if rng.random() < 0.5:
                    wall = np.stack([z, c[1] + t, np.full_like(z, c[2])], 1)
                parts.append(wall)
            for _ in range(40):  # objects: box surfaces standing on the road
                ext = rng.uniform(0.01, 0.03, 3) * np.array([zdim * 4, ydim, xdim])
                c = np.array([5 + ext[0] / 2, rng.uniform(0, ydim), rng.uniform(0, xdim)])
                face = rng.uniform(-0.5, 0.5, (2000, 3)) * ext
                axis = rng.integers(0, 3, 2000)
                face[np.arange(2000), axis] = np.sign(face[np.arange(2000), axis]) * ext[axis] / 2
                parts.append(c + face)
            p = np.floor(np.concatenate(parts, 0)).astype(np.int64)
            p = p[((p >= 0) & (p < np.asarray(shape))).all(1)]
            keys = np.unique(np.concatenate([keys, np.ravel_multi_index(p.T, shape)]))
        pick = np.sort(rng.choice(keys.size, size=per_sample, replace=False))
        out.append(keys[pick])
    return _finish(out, list(shape))
