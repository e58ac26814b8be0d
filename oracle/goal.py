"""The reference's goal field, restated — TEST INFRASTRUCTURE ONLY.

python/surfgym/goalfield.py builds a geodesic distance-to-goal field over the
free voxels of an occupancy grid (build_goal_field, :159-298) and samples it
trilinearly over "honest" corners (GoalField.sample, :68-94). This module is
the oracle for the GPU bake and sampler:

* :func:`distance` / :func:`bake` — ``oracle/goal.c``: Dijkstra in fp32 to
  the relaxation's fixpoint, then the sentinel and uint16 quantisation;
* :func:`jacobi_distance` — the reference's own relaxation order (whole-grid
  sweeps over the 26 shifted neighbours, all reading the previous sweep's
  values, until a sweep changes nothing), in numpy, for tiny grids: it pins
  the Dijkstra order above;
* :func:`sample` — ``oracle/goal.c``: GoalField.sample in its numpy types.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _load, _ptr

OFFSETS = [(oz, oy, ox) for oz in (-1, 0, 1) for oy in (-1, 0, 1) for ox in (-1, 0, 1)
           if (oz, oy, ox) != (0, 0, 0)]


def distance(occ: np.ndarray, cell: float, lo, hi):
    """Relaxed fp32 distances [nz,ny,nx] (+inf unreachable or solid) and the
    seed count. lo/hi: inclusive voxel box (x, y, z)."""
    lib = _load()
    o = np.ascontiguousarray(occ != 0, dtype=np.uint8)
    nz, ny, nx = o.shape
    d = np.empty(o.shape, np.float32)
    lo_a = np.ascontiguousarray(lo, dtype=np.int32)
    hi_a = np.ascontiguousarray(hi, dtype=np.int32)
    n = lib.oracle_goal_distance(_ptr(o), nx, ny, nz, float(cell), _ptr(lo_a), _ptr(hi_a), _ptr(d))
    if n < 0:
        raise MemoryError("oracle_goal_distance: allocation failed")
    return d, int(n)


def quantise(d: np.ndarray, cell: float) -> dict:
    """Sentinel, reach_max and the uint16 grid from relaxed distances."""
    lib = _load()
    d = np.ascontiguousarray(d, dtype=np.float32)
    q = np.empty(d.shape, np.uint16)
    g = np.empty(d.shape, np.float32)
    reach, sent, quant = ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
    rc = lib.oracle_goal_quantise(_ptr(d), d.size, float(cell), _ptr(q), _ptr(g),
                                  ctypes.byref(reach), ctypes.byref(sent), ctypes.byref(quant))
    if rc != 0:
        raise RuntimeError("goal field sentinel exceeds the uint16 range")
    return {"grid_q": q, "grid": g, "reach_max": np.float32(reach.value),
            "sentinel": np.float32(sent.value), "quant": np.float32(quant.value)}


def bake(occ: np.ndarray, cell: float, lo, hi) -> dict:
    d, n = distance(occ, cell, lo, hi)
    if n == 0:
        raise RuntimeError("goal zone contains no free voxel")
    out = quantise(d, cell)
    out["d"] = d
    out["n_seed"] = n
    return out


def jacobi_distance(occ: np.ndarray, cell: float, lo, hi, max_sweeps: int = 100000):
    """The reference's sweep order: each sweep takes the minimum over the 26
    shifted copies of the previous sweep's grid plus the edge weight, in fp32,
    then re-pins solids at +inf; stop when a sweep changes nothing."""
    solid = np.asarray(occ) != 0
    nz, ny, nx = solid.shape
    d = np.full(solid.shape, np.inf, np.float32)
    lx, ly, lz = (max(int(v), 0) for v in lo)
    hx, hy, hz = int(hi[0]), int(hi[1]), int(hi[2])
    seed = np.zeros_like(solid)
    seed[lz:hz + 1, ly:hy + 1, lx:hx + 1] = True
    seed &= ~solid
    d[seed] = 0.0
    w = {o: np.float32(cell * float(np.sqrt(o[0] ** 2 + o[1] ** 2 + o[2] ** 2))) for o in OFFSETS}
    pad = np.full((nz + 2, ny + 2, nx + 2), np.inf, np.float32)
    for _ in range(max_sweeps):
        pad[1:-1, 1:-1, 1:-1] = d
        new = d.copy()
        for (oz, oy, ox) in OFFSETS:
            src = pad[1 + oz:1 + oz + nz, 1 + oy:1 + oy + ny, 1 + ox:1 + ox + nx]
            np.minimum(new, src + w[(oz, oy, ox)], out=new)
        new[solid] = np.inf
        if np.array_equal(new, d):
            return d, int(seed.sum())
        d = new
    raise RuntimeError("jacobi_distance did not converge")


def sample(grid: np.ndarray, mins, cell: float, reach_max: float, pos: np.ndarray) -> np.ndarray:
    lib = _load()
    g = np.ascontiguousarray(grid, dtype=np.float32)
    nz, ny, nx = g.shape
    p = np.ascontiguousarray(np.atleast_2d(np.asarray(pos, np.float64)))
    m = np.ascontiguousarray(mins, dtype=np.float64)
    out = np.empty(len(p), np.float32)
    lib.oracle_goal_sample(_ptr(g), nx, ny, nz, _ptr(m), float(cell), float(reach_max), _ptr(p),
                           len(p), _ptr(out))
    return out
