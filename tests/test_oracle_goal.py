"""Pins the goal-field oracle (oracle/goal.c) to the reference's semantics.

The reference (python/surfgym/goalfield.py) has no golden vectors or tests
for the geodesic field (its reward tests cover only EuclidField), so the
oracle is pinned by:

* a second relaxation order — the reference's own whole-grid sweeps, in
  numpy (oracle.goal.jacobi_distance) — that must agree bit for bit with the
  oracle's Dijkstra order on random grids;
* closed forms: the 26-neighbour distance in an empty box
  (c*sqrt3 + (b-c)*sqrt2 + (a-b) cells for sorted offsets a >= b >= c),
  additivity through a one-voxel hole, exact symmetry under axis swaps;
* the stated invariants of the stored field (sentinel, quantisation,
  uint16 overflow refusal) and of the sampler (voxel centres, linear fields,
  honest-corner renormalisation, the all-dishonest sentinel, clamping).

CPU only: no GPU, no native renderer.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import goal

F32 = np.float32


def _octile(a, b, c):
    a, b, c = sorted((abs(a), abs(b), abs(c)), reverse=True)
    return c * math.sqrt(3.0) + (b - c) * math.sqrt(2.0) + (a - b)


# ------------------------------------------------------------- relaxation --
@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("cell", [16.0, 8.0, 12.0, 32.0])
def test_dijkstra_equals_reference_sweep_order(seed, cell):
    rng = np.random.default_rng(seed * 7 + int(cell))
    shp = tuple(int(v) for v in rng.integers(3, 12, 3))   # (nz, ny, nx)
    occ = (rng.random(shp) < rng.uniform(0.0, 0.45)).astype(np.uint8)
    nz, ny, nx = shp
    lo = [int(rng.integers(0, n)) for n in (nx, ny, nz)]
    hi = [int(min(l + rng.integers(0, 3), n - 1)) for l, n in zip(lo, (nx, ny, nz))]
    d_ref, n_ref = goal.jacobi_distance(occ, cell, lo, hi)
    d, n = goal.distance(occ, cell, lo, hi)
    assert n == n_ref
    assert np.array_equal(d, d_ref), (shp, lo, hi)


def test_empty_box_is_the_26_neighbour_metric():
    cell = 16.0
    occ = np.zeros((9, 10, 11), np.uint8)
    d, n = goal.distance(occ, cell, [0, 0, 0], [0, 0, 0])
    assert n == 1 and d[0, 0, 0] == 0.0
    for z in range(9):
        for y in range(10):
            for x in range(11):
                want = cell * _octile(x, y, z)
                assert abs(float(d[z, y, x]) - want) <= 1e-5 * max(want, 1.0), (x, y, z)


def test_axis_swaps_give_identical_values():
    # the least fp32 path sum does not depend on which axis a step moves
    occ = np.zeros((8, 8, 8), np.uint8)
    d, _ = goal.distance(occ, 16.0, [0, 0, 0], [0, 0, 0])
    assert np.array_equal(d, np.transpose(d, (0, 2, 1)))
    assert np.array_equal(d, np.transpose(d, (2, 1, 0)))
    assert np.array_equal(d, np.transpose(d, (1, 0, 2)))


def test_one_voxel_hole_is_additive():
    cell = 16.0
    occ = np.zeros((9, 9, 12), np.uint8)
    occ[:, :, 6] = 1
    occ[4, 4, 6] = 0                        # the hole (x=6, y=4, z=4)
    d, _ = goal.distance(occ, cell, [0, 0, 0], [0, 0, 0])
    for (x, y, z) in [(7, 4, 4), (11, 8, 8), (9, 0, 2), (11, 4, 0)]:
        want = cell * (_octile(6, 4, 4) + _octile(x - 6, y - 4, z - 4))
        assert abs(float(d[z, y, x]) - want) <= 1e-5 * want, (x, y, z)
    for (x, y, z) in [(9, 0, 2), (11, 4, 0)]:                # off the hole's cone: a detour
        assert float(d[z, y, x]) > cell * _octile(x, y, z) + cell


def test_enclosed_pocket_is_unreachable_and_solid_is_inf():
    occ = np.zeros((10, 10, 10), np.uint8)
    occ[3:8, 3:8, 3:8] = 1
    occ[4:7, 4:7, 4:7] = 0                  # a sealed 3^3 cavity
    d, _ = goal.distance(occ, 16.0, [0, 0, 0], [1, 1, 1])
    assert np.all(np.isinf(d[4:7, 4:7, 4:7]))
    assert np.all(np.isinf(d[occ != 0]))
    assert np.all(np.isfinite(d[:3]))


def test_seeds_skip_solid_voxels_and_clip_to_the_grid():
    occ = np.zeros((4, 5, 6), np.uint8)
    occ[0, 0, :] = 1
    d, n = goal.distance(occ, 16.0, [-5, -5, -5], [10, 0, 0])
    assert n == 0 and np.all(np.isinf(d))
    d, n = goal.distance(occ, 16.0, [-5, -5, -5], [10, 1, 0])
    assert n == 6 and np.all(d[0, 1, :] == 0.0)


# ----------------------------------------------------------- stored field --
def test_quantise_sentinel_and_rounding():
    cell = 16.0
    occ = np.zeros((6, 7, 8), np.uint8)
    occ[2, :, :] = 1
    occ[2, 3, 3] = 0
    occ[4:6, 5:7, 6:8] = 1
    out = goal.bake(occ, cell, [0, 0, 0], [0, 0, 0])
    d, q, g = out["d"], out["grid_q"], out["grid"]
    fin = np.isfinite(d)
    assert out["reach_max"] == d[fin].max()
    assert out["sentinel"] == F32(float(out["reach_max"]) + 2.0 * cell)
    assert out["quant"] == F32(2.0)
    assert np.all(np.abs(q[fin].astype(np.float64) * 2.0 - d[fin]) <= 1.0)
    assert np.all(q[~fin] == np.round(float(out["sentinel"]) / 2.0))
    assert np.array_equal(g, q.astype(np.float32) * F32(2.0))


def test_quantise_rounds_half_to_even():
    d = np.array([1.0, 3.0, 5.0, 2.5, np.inf], np.float32).reshape(1, 1, 5)
    out = goal.quantise(d, 16.0)            # quant 2: 0.5, 1.5, 2.5, 1.25
    assert out["grid_q"].ravel()[:4].tolist() == [0, 2, 2, 1]


def test_uint16_overflow_is_refused():
    occ = np.zeros((1, 1, 8200), np.uint8)  # a corridor 8200 voxels long
    d, _ = goal.distance(occ, 16.0, [0, 0, 0], [0, 0, 0])
    assert float(d.max()) > 131000
    with pytest.raises(RuntimeError, match="uint16"):
        goal.quantise(d, 16.0)


# ---------------------------------------------------------------- sampler --
def _grid_centres(shape, mins, cell):
    nz, ny, nx = shape
    z, y, x = np.meshgrid(np.arange(nz), np.arange(ny), np.arange(nx), indexing="ij")
    return np.stack([mins[0] + (x + 0.5) * cell, mins[1] + (y + 0.5) * cell,
                     mins[2] + (z + 0.5) * cell], -1).reshape(-1, 3)


def test_sample_at_voxel_centres_returns_the_grid():
    rng = np.random.default_rng(3)
    grid = rng.uniform(0, 900, (5, 6, 7)).astype(np.float32)
    mins = np.array([-100.0, 40.0, -8.0])
    out = goal.sample(grid, mins, 16.0, 1000.0, _grid_centres(grid.shape, mins, 16.0))
    assert np.array_equal(out, grid.ravel())


def test_sample_reproduces_a_linear_field():
    cell, mins = 16.0, np.array([0.0, 0.0, 0.0])
    c = _grid_centres((6, 7, 8), mins, cell)
    grid = (3.0 * c[:, 0] - 2.0 * c[:, 1] + 0.5 * c[:, 2] + 700.0).astype(np.float32).reshape(6, 7, 8)
    rng = np.random.default_rng(4)
    p = rng.uniform(0.5 * cell, [7.5 * cell, 6.5 * cell, 5.5 * cell], (500, 3))
    out = goal.sample(grid, mins, cell, 1e6, p)
    want = 3.0 * p[:, 0] - 2.0 * p[:, 1] + 0.5 * p[:, 2] + 700.0
    assert np.max(np.abs(out - want)) < 1e-3


def test_sample_renormalises_over_honest_corners():
    cell, mins, reach = 16.0, np.zeros(3), 500.0
    grid = np.full((2, 2, 2), 532.0, np.float32)            # sentinel = reach + 2*cell
    grid[0, 0, 0] = 100.0
    grid[1, 1, 1] = 300.0
    p = np.array([[16.0 + 4.0, 16.0 + 4.0, 16.0 + 4.0]])    # f = 0.75 along every axis
    wa, wb = F32(0.25) ** 3, F32(0.75) ** 3
    want = (wa * F32(100.0) + wb * F32(300.0)) / (wa + wb)
    assert abs(float(goal.sample(grid, mins, cell, reach, p)[0]) - float(want)) < 1e-4
    grid[1, 1, 1] = 532.0
    assert abs(float(goal.sample(grid, mins, cell, reach, p)[0]) - 100.0) < 1e-4
    grid[0, 0, 0] = 532.0
    assert goal.sample(grid, mins, cell, reach, p)[0] == F32(reach + 2.0 * cell)


def test_sample_honest_threshold_is_half_a_cell_above_reach():
    cell, reach = 16.0, 500.0
    grid = np.full((1, 1, 1), reach + 0.5 * cell, np.float32)   # exactly at the limit: dishonest
    assert goal.sample(grid, np.zeros(3), cell, reach, [[8.0, 8.0, 8.0]])[0] == F32(reach + 2 * cell)
    grid[:] = np.nextafter(F32(reach + 0.5 * cell), F32(0))
    assert goal.sample(grid, np.zeros(3), cell, reach, [[8.0, 8.0, 8.0]])[0] == grid[0, 0, 0]


def test_sample_clamps_outside_the_grid():
    rng = np.random.default_rng(5)
    grid = rng.uniform(0, 400, (3, 4, 5)).astype(np.float32)
    far = np.array([[-1e5, -1e5, -1e5], [1e6, 1e6, 1e6], [-1e5, 1e6, 24.0]])
    out = goal.sample(grid, np.zeros(3), 16.0, 1000.0, far)
    assert abs(float(out[0]) - float(grid[0, 0, 0])) <= 1e-4 * float(grid[0, 0, 0])
    assert abs(float(out[1]) - float(grid[-1, -1, -1])) <= 1e-4 * float(grid[-1, -1, -1])
