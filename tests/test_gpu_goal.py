"""Goal-field bake and sampler on the GPU against the CPU oracle.

The bake (csrc/goal.hip) must reproduce the oracle's fp32 fixpoint bit for
bit — relaxed distances, reach_max, the uint16 grid and its dequantisation —
and the sampler must reproduce GoalField.sample (python/surfgym/goalfield.py
:68-94) bit for bit. A torch restatement of the reference's bake, run on the
GPU with torch's own CUDA ops, checks the semantics the oracle assumes of
torch (the fp32 scalar add, the division by a Python scalar, round half even).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import goal as ogoal
from surfgym import goalfield, synth

pytestmark = pytest.mark.gpu


def _bake_both(occ, mins, zone, cell, dev, **kw):
    nz, ny, nx = occ.shape
    lo, hi = goalfield.seed_voxel_box(zone, mins, cell, (nx, ny, nz))
    ref = ogoal.bake(occ, cell, lo, hi)
    field = goalfield.goal_field_from_occupancy(occ, mins, zone, cell, device=dev, **kw)
    return ref, field


def _check_field(ref, field):
    q = field.grid_q.cpu().numpy().view(np.uint16)
    assert np.array_equal(q, ref["grid_q"])
    assert np.array_equal(field.grid.cpu().numpy(), ref["grid"])
    assert np.float32(field.reach_max) == ref["reach_max"]
    assert field.bake_info["n_seed"] == ref["n_seed"]
    assert np.float32(field.bake_info["sentinel"]) == ref["sentinel"]


def _zone_at(x, y, z, cell, mins=(0.0, 0.0, 0.0), half=1.0):
    c = np.asarray(mins) + (np.array([x, y, z]) + 0.5) * cell
    return {"mins": (c - half).tolist(), "maxs": (c + half).tolist()}


@pytest.mark.parametrize("seed", range(8))
def test_random_grids_match_oracle(dev, seed):
    rng = np.random.default_rng(100 + seed)
    shp = tuple(int(v) for v in rng.integers(1, 40, 3))
    occ = (rng.random(shp) < rng.uniform(0.0, 0.5)).astype(np.uint8)
    cell = float(rng.choice([8.0, 16.0, 32.0, 12.0]))
    nz, ny, nx = shp
    zone = _zone_at(rng.integers(0, nx), rng.integers(0, ny), rng.integers(0, nz), cell)
    print(f"case goal random seed={seed} shape={shp} cell={cell}", flush=True)
    lo, hi = goalfield.seed_voxel_box(zone, np.zeros(3), cell, (nx, ny, nz))
    d, n = ogoal.distance(occ, cell, lo, hi)
    if n == 0:
        with pytest.raises(RuntimeError, match="no free voxel"):
            goalfield.goal_field_from_occupancy(occ, np.zeros(3), zone, cell, device=dev)
        return
    ref, field = _bake_both(occ, np.zeros(3), zone, cell, dev)
    _check_field(ref, field)


@pytest.mark.parametrize("name", ["small_ramps", "maze", "ramp_field"])
def test_scene_fields_match_oracle(dev, name):
    w = synth.goal_workload(name)
    print(f"case goal scene {name} {w.occ.shape}", flush=True)
    ref, field = _bake_both(w.occ, w.mins, w.zone, w.cell, dev)
    _check_field(ref, field)
    assert field.bake_info["sweeps"] > 0 and field.bake_info["tile_visits"] > 0


def _torch_reference_bake(occ, cell, lo, hi, dev):
    """The reference's bake order in torch CUDA ops: whole-grid sweeps of the
    26 shifted minimum-plus-weight updates, solids re-pinned to +inf, run to
    a sweep that changes nothing; then sentinel, divide by the Python scalar
    quant, round, clamp."""
    solid = torch.as_tensor(occ != 0, device=dev)
    nz, ny, nx = occ.shape
    d = torch.full((nz, ny, nx), float("inf"), device=dev)
    seed = torch.zeros_like(solid)
    seed[lo[2]:hi[2] + 1, lo[1]:hi[1] + 1, lo[0]:hi[0] + 1] = True
    d[seed & ~solid] = 0.0
    pad = torch.full((nz + 2, ny + 2, nx + 2), float("inf"), device=dev)
    tmp = torch.empty_like(d)
    for _ in range(100000):
        prev = d.clone()
        pad[1:-1, 1:-1, 1:-1].copy_(d)
        for (oz, oy, ox) in ogoal.OFFSETS:
            w = cell * float(np.sqrt(oz * oz + oy * oy + ox * ox))
            torch.add(pad[1 + oz:1 + oz + nz, 1 + oy:1 + oy + ny, 1 + ox:1 + ox + nx], w, out=tmp)
            torch.minimum(d, tmp, out=d)
        d.masked_fill_(solid, float("inf"))
        if torch.equal(d, prev):
            break
    reach = float(d[torch.isfinite(d)].max())
    d.nan_to_num_(posinf=reach + 2.0 * cell)
    d.div_(cell / 8.0).round_().clamp_(0, 65535)
    return d.to(torch.int32).cpu().numpy().astype(np.uint16), reach


@pytest.mark.parametrize("cell", [16.0, 12.0, 7.0])
def test_matches_torch_restatement_of_reference_bake(dev, cell):
    rng = np.random.default_rng(int(cell))
    occ = (rng.random((12, 20, 24)) < 0.3).astype(np.uint8)
    zone = _zone_at(3, 4, 5, cell, half=cell)
    lo, hi = goalfield.seed_voxel_box(zone, np.zeros(3), cell, (24, 20, 12))
    print(f"case goal torch-restatement cell={cell}", flush=True)
    q_ref, reach = _torch_reference_bake(occ, cell, lo, hi, dev)
    field = goalfield.goal_field_from_occupancy(occ, np.zeros(3), zone, cell, device=dev)
    assert field.reach_max == reach
    assert np.array_equal(field.grid_q.cpu().numpy().view(np.uint16), q_ref)


def test_edge_cases(dev):
    cell = 16.0
    # one-voxel-thin grids along each axis, dims not multiples of the tile
    for shp in [(1, 1, 37), (1, 29, 1), (19, 1, 1), (9, 1, 17), (1, 1, 1)]:
        occ = np.zeros(shp, np.uint8)
        ref, field = _bake_both(occ, np.zeros(3), _zone_at(0, 0, 0, cell), cell, dev)
        _check_field(ref, field)
    occ = np.zeros((8, 8, 8), np.uint8)
    far = _zone_at(100, 100, 100, cell)
    with pytest.raises(RuntimeError, match="no free voxel"):
        goalfield.goal_field_from_occupancy(occ, np.zeros(3), far, cell, device=dev)
    occ[:] = 1
    with pytest.raises(RuntimeError, match="no free voxel"):
        goalfield.goal_field_from_occupancy(occ, np.zeros(3), _zone_at(1, 1, 1, cell), cell,
                                            device=dev)
    corridor = np.zeros((1, 1, 8200), np.uint8)
    with pytest.raises(RuntimeError, match="uint16"):
        goalfield.goal_field_from_occupancy(corridor, np.zeros(3), _zone_at(0, 0, 0, cell), cell,
                                            device=dev)
    # a sealed cavity stays at the sentinel
    occ = np.zeros((16, 16, 16), np.uint8)
    occ[4:12, 4:12, 4:12] = 1
    occ[6:10, 6:10, 6:10] = 0
    ref, field = _bake_both(occ, np.zeros(3), _zone_at(0, 0, 0, cell), cell, dev)
    _check_field(ref, field)
    assert np.all(field.grid.cpu().numpy()[6:10, 6:10, 6:10] == ref["grid"][6, 6, 6])


def test_bake_is_deterministic_and_u16_storage_samples_identically(dev):
    w = synth.goal_workload("maze")
    a = goalfield.goal_field_from_occupancy(w.occ, w.mins, w.zone, w.cell, device=dev)
    b = goalfield.goal_field_from_occupancy(w.occ, w.mins, w.zone, w.cell, device=dev,
                                            keep_u16=True)
    assert torch.equal(a.grid_q, b.grid_q)
    rng = np.random.default_rng(7)
    hi = w.mins + np.array(w.occ.shape[::-1]) * w.cell
    p = rng.uniform(w.mins - 3 * w.cell, hi + 3 * w.cell, (20000, 3))
    assert np.array_equal(a.sample(p), b.sample(p))


def test_sample_matches_oracle(dev):
    w = synth.goal_workload("ramp_field")
    field = goalfield.goal_field_from_occupancy(w.occ, w.mins, w.zone, w.cell, device=dev)
    grid = field.grid.cpu().numpy()
    rng = np.random.default_rng(11)
    hi = w.mins + np.array(w.occ.shape[::-1]) * w.cell
    p = rng.uniform(w.mins - 4 * w.cell, hi + 4 * w.cell, (200000, 3))
    # voxel centres and cell corners too: fractions of exactly 0 and 0.5
    p[:1000] = w.mins + (rng.integers(0, 128, (1000, 3)) + 0.5) * w.cell
    p[1000:2000] = w.mins + rng.integers(0, 128, (1000, 3)) * w.cell
    print("case goal sample ramp_field 200000", flush=True)
    want = ogoal.sample(grid, w.mins, w.cell, field.reach_max, p)
    got = field.sample(p)
    assert got.dtype == np.float32
    assert np.array_equal(got, want)
    assert (want == np.float32(field.sentinel)).any() and (want < field.reach_max).any()
    # device tensors: f64 and f32 rows, strided (N, 6) rows, no host round trip
    pt = torch.as_tensor(p, device=dev)
    assert np.array_equal(field.sample(pt).cpu().numpy(), want)
    p32 = p.astype(np.float32)
    want32 = ogoal.sample(grid, w.mins, w.cell, field.reach_max, p32.astype(np.float64))
    assert np.array_equal(field.sample(torch.as_tensor(p32, device=dev)).cpu().numpy(), want32)
    wide = torch.zeros((len(p), 6), dtype=torch.float64, device=dev)
    wide[:, 1:4] = pt
    assert np.array_equal(field.sample(wide[:, 1:4]).cpu().numpy(), want)
    assert len(field.sample(np.zeros((0, 3)))) == 0


def test_reachable_and_descent_yaw(dev):
    w = synth.goal_workload("maze")
    field = goalfield.goal_field_from_occupancy(w.occ, w.mins, w.zone, w.cell, device=dev)
    grid = field.grid.cpu().numpy()
    rng = np.random.default_rng(12)
    hi = w.mins + np.array(w.occ.shape[::-1]) * w.cell
    p = rng.uniform(w.mins, hi, (5000, 3))
    s = ogoal.sample(grid, w.mins, w.cell, field.reach_max, p)
    assert np.array_equal(field.reachable(p), s < np.float32(field.reach_max - 0.5 * field.cell))
    h = field.cell
    dx = (ogoal.sample(grid, w.mins, w.cell, field.reach_max, p + [h, 0, 0])
          - ogoal.sample(grid, w.mins, w.cell, field.reach_max, p - [h, 0, 0]))
    dy = (ogoal.sample(grid, w.mins, w.cell, field.reach_max, p + [0, h, 0])
          - ogoal.sample(grid, w.mins, w.cell, field.reach_max, p - [0, h, 0]))
    want = np.degrees(np.arctan2(-dy, -dx)) % 360.0
    got = field.descent_yaw(p)
    diff = np.abs(got - want)
    diff = np.minimum(diff, 360.0 - diff)          # 0 and 360 are one direction
    assert diff.max() < 1e-3


def test_goal_field_from_cached_u16_grid(dev, tmp_path):
    """A GoalField built from the reference's cache arrays samples like one
    holding the dequantised grid (goalfield.py:178-183, :297)."""
    w = synth.goal_workload("small_ramps")
    baked = goalfield.goal_field_from_occupancy(w.occ, w.mins, w.zone, w.cell, device=dev)
    q = baked.grid_q.cpu().numpy().view(np.uint16)
    f = tmp_path / "m.goal_16.npz"
    np.savez_compressed(f, grid=q, quant=np.float32(baked.bake_info["quant"]), mins=w.mins,
                        cell=np.float32(w.cell), reach_max=np.float32(baked.reach_max),
                        sig=np.str_("x"))
    z = np.load(f, allow_pickle=False)
    from_cache = goalfield.GoalField(z["grid"], z["mins"], float(z["cell"]),
                                     float(z["reach_max"]), quant=float(z["quant"]), device=dev)
    ref_grid = z["grid"].astype(np.float32) * float(z["quant"])
    p = np.random.default_rng(13).uniform(w.mins, w.mins + 1024.0, (4000, 3))
    want = ogoal.sample(ref_grid, z["mins"], float(z["cell"]), float(z["reach_max"]), p)
    assert np.array_equal(from_cache.sample(p), want)
    assert np.array_equal(baked.sample(p), want)
