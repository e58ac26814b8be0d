"""The reference's SDF bake call, restated — TEST INFRASTRUCTURE ONLY.

python/surfgym/vision.py:428-438 turns a solid-occupancy grid into its SDF
with scipy (the third-party routine the reference depends on; scipy 1.15.3 in
this image):

    occ = np.pad(occ, 1, constant_values=1)          # outside counts as solid
    dist = distance_transform_edt(occ == 0, sampling=cell)
    sdf = dist[1:-1, 1:-1, 1:-1]
    sdf.astype(np.float16 if sdf.size > 100e6 else np.float32)

`bake` is that call. `brute_force` is an independent O(voxels x solids)
evaluation used to pin it on tiny grids (tests/test_oracle.py).
"""
from __future__ import annotations

import numpy as np


def bake(occ: np.ndarray, cell: float) -> np.ndarray:
    """float64 distances [nz,ny,nx] in map units, 0 in solid voxels."""
    from scipy.ndimage import distance_transform_edt
    o = np.pad(np.asarray(occ, dtype=np.uint8), 1, constant_values=1)
    dist = distance_transform_edt(o == 0, sampling=cell)
    return dist[1:-1, 1:-1, 1:-1]


def stored(dist: np.ndarray) -> np.ndarray:
    """The dtype the reference stores (vision.py:436-437)."""
    return dist.astype(np.float16 if dist.size > 100e6 else np.float32)


def brute_force(occ: np.ndarray, cell: float) -> np.ndarray:
    """Distance from every voxel centre to the nearest solid centre, the
    one-voxel shell around the grid counting as solid."""
    o = np.pad(np.asarray(occ, dtype=np.uint8), 1, constant_values=1)
    solid = np.argwhere(o != 0).astype(np.float64)
    nz, ny, nx = occ.shape
    idx = np.argwhere(np.ones((nz, ny, nx), bool)).astype(np.float64) + 1.0
    d2 = ((idx[:, None, :] - solid[None, :, :]) ** 2).sum(-1).min(1)
    return (np.sqrt(d2) * cell).reshape(nz, ny, nx)
