"""Pins the CPU oracle (oracle/march.c) to the reference's semantics.

Each test derives its expectation independently of the oracle's code: from
closed forms (constant fields, the encoding, camera geometry by rotation
matrices), from invariants the reference states (monotone alive, partial t
on exhaustion, one-step range overshoot then clamp, border clamping), or
from geometry with a known answer (a floor, a wall). Reference lines are
python/surfgym/vision.py unless stated.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle

D2R = np.pi / 180.0
F32 = np.float32


def _one(grid, mins, cell, eye, yaw, pitch, *, ducked=0.0, **kw):
    """Render one env; eye is the EYE position (origin + 17 standing)."""
    origin = np.array([[eye[0], eye[1], eye[2] - (12.0 if ducked else 17.0)]], np.float32)
    enc, loads = oracle.render(grid, np.asarray(mins, np.float32), cell, origin,
                               np.array([yaw], np.float32), np.array([pitch], np.float32),
                               np.array([ducked], np.float32), **kw)
    return enc[0], loads[0]


def _fp32_steps(step, k):
    t = F32(0.0)
    for _ in range(k):
        t = F32(t + F32(step))
    return t


# -------------------------------------------------------------- camera tables --
@pytest.mark.parametrize("w,fov", [(128, 120.0), (64, 90.0), (9, 120.0), (5, 90.0), (1, 90.0)])
def test_offset_tables_are_pixel_centres_of_the_fov(w, fov):
    """yoff/poff (vision.py:502-509, surfcore.h:29-34): pixel CENTRES of the
    fov, column 0 / row 0 at +fov/2 - half a pixel, symmetric, uniform."""
    yo, _ = oracle.offsets(w, 1, fov, 90.0)
    step = fov / w
    assert abs(yo[0] - math.radians(fov / 2 - step / 2)) < 1e-6        # left / up first
    assert np.allclose(yo, -yo[::-1], atol=1e-6)                      # symmetric
    if w > 1:
        assert np.allclose(np.diff(yo), -math.radians(step), atol=1e-6)
    # and rounded once from float64, so it equals the float64 value to half an ulp
    exact = np.radians(fov / 2 - step * (np.arange(w) + 0.5))
    assert np.all(np.abs(yo - exact) <= np.abs(np.spacing(yo)) * 0.5 + 1e-12)


def test_centre_and_axes_follow_the_camera_convention():
    """Odd sizes: the centre pixel is the view direction; col 0 looks left
    (+y at yaw 0), row 0 looks up (surfcore.h:29-34)."""
    for yaw, pitch in [(0.0, 0.0), (37.0, 0.0), (0.0, 25.0), (-140.0, -33.0), (270.0, 60.0)]:
        d = oracle.ray_dirs(9, 5, yaw, pitch)
        p, y = math.radians(pitch), math.radians(yaw)
        fwd = np.array([math.cos(p) * math.cos(y), math.cos(p) * math.sin(y), math.sin(p)])
        assert np.abs(d[2, 4] - fwd).max() < 1e-6
        assert np.abs(np.linalg.norm(d, axis=-1) - 1.0).max() < 1e-6
    d = oracle.ray_dirs(9, 5, 0.0, 0.0)
    assert d[2, 0][1] > 0 and d[2, -1][1] < 0
    assert d[0, 4][2] > 0 and d[-1, 4][2] < 0


def test_equiangular_corner_is_the_angle_composition():
    """The equiangular corner ray is yaw offset then pitch offset: its angle
    from forward is acos(cos(poff0) cos(yoff0))."""
    d = oracle.ray_dirs(9, 5, 0.0, 0.0)
    yo, po = oracle.offsets(9, 5)
    want = math.acos(math.cos(po[0]) * math.cos(yo[0]))
    got = math.acos(float(np.clip(d[0, 0] @ np.array([1.0, 0, 0]), -1, 1)))
    assert abs(got - want) < 1e-6


def test_pinhole_rays_are_the_tangent_grid_rotated_into_the_view():
    """Independent derivation (as tests/python/test_pinhole.py:91-118): the
    camera-space ray (1, -u, v) rotated by pitch about y, then yaw about z."""
    W, H = 7, 5
    tu, tv = math.tan(math.radians(60.0)), math.tan(math.radians(45.0))
    u = tu * (2.0 * np.arange(W) / (W - 1) - 1.0)
    v = tv * (1.0 - 2.0 * np.arange(H) / (H - 1))
    for yaw, pitch in [(0.0, 0.0), (41.0, 0.0), (0.0, -37.0), (41.0, -37.0), (-115.0, 62.0)]:
        got = oracle.ray_dirs(W, H, yaw, pitch, pinhole=True)
        y, p = math.radians(yaw), math.radians(pitch)
        rz = np.array([[math.cos(y), -math.sin(y), 0], [math.sin(y), math.cos(y), 0], [0, 0, 1]])
        ry = np.array([[math.cos(p), 0, -math.sin(p)], [0, 1, 0], [math.sin(p), 0, math.cos(p)]])
        for r in range(H):
            for c in range(W):
                cam = np.array([1.0, -u[c], v[r]])
                want = rz @ ry @ (cam / np.linalg.norm(cam))
                assert np.abs(got[r, c] - want).max() < 1e-6


def test_pinhole_corner_is_the_analytic_angle_and_one_pixel_is_the_centre():
    d = oracle.ray_dirs(9, 5, 0.0, 0.0, pinhole=True)
    want = math.atan(math.hypot(math.tan(math.radians(60)), math.tan(math.radians(45))))
    for r, c in ((0, 0), (0, 8), (4, 0), (4, 8)):
        assert abs(math.acos(float(np.clip(d[r, c][0], -1, 1))) - want) < 1e-6
    one = oracle.ray_dirs(1, 1, 30.0, -20.0, pinhole=True)[0, 0]
    p, y = math.radians(-20.0), math.radians(30.0)
    assert np.allclose(one, [math.cos(p) * math.cos(y), math.cos(p) * math.sin(y), math.sin(p)],
                       atol=1e-6)


# ------------------------------------------------------------------ encoding --
def test_encoding_closed_forms():
    """vision.py:112-116: linear up to near, then a tail bounded by 1.25."""
    assert oracle.encode(0.0, 2000.0) == 0.0
    assert oracle.encode(500.0, 2000.0) == F32(500.0) / F32(2000.0)
    assert oracle.encode(2000.0, 2000.0) == 1.0
    assert abs(oracle.encode(2000.0 + 2500.0, 2000.0) - (1.0 + 0.25 * (1 - math.exp(-1.0)))) < 1e-6
    assert abs(oracle.encode(1e9, 2000.0) - 1.25) < 1e-6
    # near == range is the legacy t/range
    for t in (0.0, 100.0, 1535.9):
        assert oracle.encode(t, 1536.0) == F32(t) / F32(1536.0)


# -------------------------------------------------------------------- march --
EMPTY = np.full((8, 8, 8), 999.0, np.float32)


def test_constant_field_runs_to_range_with_one_step_overshoot():
    """Constant d: every step is 0.9*d; `t < range` is tested before the step
    is added (vision.py:109-110), so t overshoots by up to one step and is
    clamped afterwards (:112). Loads = steps taken + the final check."""
    step = F32(F32(999.0) * F32(0.9))
    enc, loads = _one(EMPTY, (0, 0, 0), 16.0, (64, 64, 64), 10.0, -5.0, range_units=2000.0,
                      max_steps=64)
    k = math.ceil(2000.0 / float(step))          # steps until t >= range
    assert _fp32_steps(step, k - 1) < 2000.0 <= _fp32_steps(step, k)
    assert np.all(enc == 1.0)
    assert np.all(loads == k + 1)
    enc, _ = _one(EMPTY, (0, 0, 0), 16.0, (64, 64, 64), 10.0, -5.0, range_units=2000.0,
                  near_range=1000.0, max_steps=64)
    assert np.allclose(enc, 1.0 + 0.25 * (1.0 - math.exp(-1000.0 / 2500.0)), atol=1e-6)


def test_exhausted_rays_keep_their_partial_t():
    """A ray that runs out of steps reports t, not the range (vision.py:112)."""
    step = F32(F32(999.0) * F32(0.9))
    for m in (0, 1, 2, 5):
        enc, loads = _one(EMPTY, (0, 0, 0), 16.0, (64, 64, 64), 0.0, 0.0, range_units=1e6,
                          near_range=1e6, max_steps=m)
        t = _fp32_steps(step, m)
        assert np.all(enc == F32(t) / F32(1e6)), m
        assert np.all(loads == m)


def test_hit_epsilon_is_strict_and_min_step_floors_the_step():
    """alive needs d > hit_eps (strict, vision.py:109); step = max(0.9 d,
    min_step) (vision.py:110)."""
    eps = F32(9.6)
    g = np.full((8, 8, 8), eps, np.float32)
    enc, loads = _one(g, (0, 0, 0), 16.0, (64, 64, 64), 0.0, 0.0, hit_eps=float(eps))
    assert np.all(enc == 0.0) and np.all(loads == 1)
    just_above = np.nextafter(eps, F32(np.inf))
    g[:] = just_above
    enc, loads = _one(g, (0, 0, 0), 16.0, (64, 64, 64), 0.0, 0.0, hit_eps=float(eps),
                      range_units=2000.0, max_steps=3)
    step = F32(just_above * F32(0.9))
    assert np.all(loads == 3) and np.all(enc == _fp32_steps(step, 3) / F32(2000.0))
    # 0.9*5 = 4.5 < min_step 4.8: the floor takes over
    g[:] = 5.0
    enc, loads = _one(g, (0, 0, 0), 16.0, (64, 64, 64), 0.0, 0.0, hit_eps=1.0,
                      min_step=float(F32(4.8)), range_units=2000.0, max_steps=3)
    assert np.all(loads == 3) and np.all(enc == _fp32_steps(F32(4.8), 3) / F32(2000.0))


def test_floor_straight_down_hits_inside_the_floor_voxel():
    """A floor slab (as tests/python/test_surfmask.py:177-193): sdf = iz*cell.
    Straight down the march must stop inside voxel iz = 0, i.e. at a depth in
    (eye_z - cell, eye_z]; ducking lowers the eye by 5 u."""
    cell = 16.0
    g = (np.arange(16, dtype=np.float32) * cell)[:, None, None] * np.ones((1, 32, 32), np.float32)
    for ducked, eye_z in ((0.0, 200.0), (1.0, 195.0)):
        enc, loads = _one(g, (0, 0, 0), cell, (200, 200, eye_z), 0.0, -90.0, ducked=ducked,
                          width=1, height=1, range_units=2000.0, max_steps=64)
        t = float(enc[0, 0]) * 2000.0
        assert eye_z - cell < t <= eye_z + 1e-3, (ducked, t)
    # looking up: the grid's top layer is air, the clamp keeps reading it, the ray leaves
    enc, _ = _one(g, (0, 0, 0), cell, (200, 200, 200), 0.0, 80.0, range_units=2000.0)
    assert np.all(enc > 0.9)


def test_axis_order_and_yaw_sign_with_a_wall_at_plus_x():
    """A solid half-space x >= 512 in a [nz,ny,nx] grid: yaw 0 looks +x and
    hits at ~(512 - eye_x); yaw 180 looks -x into an air border and leaves.
    Also pins the grid order: the same wall stored along y is not seen."""
    cell = 8.0
    nx, ny, nz = 96, 64, 32
    cx = (np.arange(nx) + 0.5) * cell
    wall_x = np.maximum(512.0 - cx, 0.0).astype(np.float32)
    g = np.broadcast_to(wall_x[None, None, :], (nz, ny, nx)).copy()
    eye = (200.0, 256.0, 128.0)
    enc, _ = _one(g, (0, 0, 0), cell, eye, 0.0, 0.0, width=1, height=1, range_units=3000.0,
                  max_steps=64)
    assert abs(float(enc[0, 0]) * 3000.0 - (512.0 - 200.0)) <= cell
    enc, _ = _one(g, (0, 0, 0), cell, eye, 180.0, 0.0, width=1, height=1, range_units=3000.0,
                  max_steps=64)
    assert float(enc[0, 0]) == 1.0
    g2 = np.broadcast_to(np.maximum(512.0 - (np.arange(ny) + 0.5) * cell, 0.0)
                         .astype(np.float32)[None, :, None], (nz, ny, nx)).copy()
    enc, _ = _one(g2, (0, 0, 0), cell, eye, 90.0, 0.0, width=1, height=1, range_units=3000.0,
                  max_steps=64)
    assert abs(float(enc[0, 0]) * 3000.0 - (512.0 - 256.0)) <= cell
    enc, _ = _one(g2, (0, 0, 0), cell, eye, 0.0, 0.0, width=1, height=1, range_units=3000.0,
                  max_steps=64)
    assert float(enc[0, 0]) == 1.0


def test_samples_outside_the_grid_read_the_border_voxel():
    """Out-of-grid positions clamp to the nearest border voxel
    (vision.py:104-106): an eye far outside the grid, in line with a solid
    border voxel, stops at once; in line with air it marches."""
    g = np.full((4, 4, 4), 999.0, np.float32)
    g[1, 1, 0] = 0.0
    mins = (0.0, 0.0, 0.0)
    # eye at x = -500 (outside), y,z inside voxel (iy=1, iz=1): clamps to ix=0, solid
    enc, loads = _one(g, mins, 16.0, (-500.0, 24.0, 24.0), 0.0, 0.0, width=1, height=1)
    assert float(enc[0, 0]) == 0.0 and int(loads[0, 0]) == 1
    enc, loads = _one(g, mins, 16.0, (-500.0, 56.0, 24.0), 0.0, 0.0, width=1, height=1)
    assert float(enc[0, 0]) > 0.0 and int(loads[0, 0]) > 1


def test_mins_shift_the_grid():
    """Voxel i covers [mins + i*cell, mins + (i+1)*cell): shifting mins and
    the eye together changes nothing."""
    rng = np.random.default_rng(5)
    g = rng.uniform(0.0, 60.0, (8, 10, 12)).astype(np.float32)
    a, la = _one(g, (0, 0, 0), 16.0, (40.0, 50.0, 60.0), 33.0, -20.0, width=16, height=8,
                 hit_eps=1.0, range_units=400.0)
    b, lb = _one(g, (-1024.0, 512.0, -256.0), 16.0, (40.0 - 1024.0, 50.0 + 512.0, 60.0 - 256.0),
                 33.0, -20.0, width=16, height=8, hit_eps=1.0, range_units=400.0)
    # positions differ by exactly representable offsets, so most rays agree bit-for-bit
    assert (np.abs(a - b) < 1e-3).mean() > 0.95
    assert (la == lb).mean() > 0.95


def test_results_do_not_depend_on_the_batch():
    """Per-ray results are independent of N (test_lidar_march.py:161-169)."""
    from surfgym import synth
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, 6)
    kw = dict(range_units=w.range_units, near_range=w.near_range, hit_eps=w.hit_eps,
              max_steps=w.max_steps)
    full, lf = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked, **kw)
    for i in (0, 3, 5):
        one, lo = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin[i:i + 1], ps.yaw[i:i + 1],
                                ps.pitch[i:i + 1], ps.ducked[i:i + 1], **kw)
        assert np.array_equal(one[0], full[i]) and np.array_equal(lo[0], lf[i])


def test_march_invariants_on_a_ramp_scene():
    """On a real scene: a ray that stopped short of range and of max_steps
    stopped on a sample <= hit_eps; every depth is within [0, range]; the
    census never exceeds max_steps."""
    from surfgym import synth
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, 4)
    enc, loads = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                               range_units=w.range_units, near_range=w.near_range,
                               hit_eps=w.hit_eps, max_steps=w.max_steps)
    assert enc.min() >= 0.0 and enc.max() <= 1.0
    assert loads.min() >= 1 and loads.max() <= w.max_steps
    # re-sample the stop point of some hit rays and check it is (near) solid
    t = enc * w.range_units
    n_idx, r_idx, c_idx = np.nonzero((t < w.range_units - 1) & (loads < w.max_steps))
    pick = np.random.default_rng(0).choice(len(n_idx), 200, replace=False)
    for n, r, c in zip(n_idx[pick], r_idx[pick], c_idx[pick]):
        d = oracle.ray_dirs(w.width, w.height, ps.yaw[n], ps.pitch[n])[r, c]
        eye = ps.origin[n] + np.array([0, 0, 12.0 if ps.ducked[n] else 17.0], np.float32)
        p = eye + d * t[n, r, c]
        # the stop sample is within one fp32 rounding of p: it reads <= eps
        assert sc.grid_value(p[None])[0] <= w.hit_eps + 1e-6 or \
            sc.grid_value((p + d * 1e-2)[None])[0] <= w.hit_eps


def _remarch_f64(grid, mins, cell, eye, yaw_deg, pitch_deg, W, H, rng, near, eps, mstep, steps):
    """A float64 sphere trace of one env written from the algorithm's
    statement, not from the oracle: view rotations as matrices, nearest
    voxel by floor, the stop rule and the encoding as the reference states
    them (vision.py:59-116)."""
    nz, ny, nx = grid.shape
    img = np.empty((H, W))
    for r in range(H):
        for c in range(W):
            yw = math.radians(yaw_deg) + math.radians(120.0 * (0.5 - (c + 0.5) / W))
            pt = math.radians(pitch_deg) + math.radians(90.0 * (0.5 - (r + 0.5) / H))
            rz = np.array([[math.cos(yw), -math.sin(yw), 0], [math.sin(yw), math.cos(yw), 0],
                           [0, 0, 1]])
            ry = np.array([[math.cos(pt), 0, -math.sin(pt)], [0, 1, 0],
                           [math.sin(pt), 0, math.cos(pt)]])
            d = rz @ ry @ np.array([1.0, 0.0, 0.0])
            t = 0.0
            for _ in range(steps):
                q = (eye + d * t - mins) / cell
                i = np.clip(np.floor(q).astype(int), 0, [nx - 1, ny - 1, nz - 1])
                s = float(grid[i[2], i[1], i[0]])
                if not (s > eps and t < rng):
                    break
                t += max(0.9 * s, mstep)
            t = min(t, rng)
            img[r, c] = min(t, near) / near + 0.25 * (1.0 - math.exp(-max(t - near, 0.0) / 2500.0))
    return img


def test_oracle_agrees_with_an_independent_float64_march():
    """The oracle (fp32, the reference's operation order) against a float64
    re-march on small images of a real scene: a wrong axis, sign, index or
    step term would move most rays; fp32 against fp64 rounding moves only
    the rare ray whose sample sits on a voxel boundary."""
    from surfgym import synth
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, 6)
    W, H = 16, 8
    enc, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                           width=W, height=H, range_units=w.range_units,
                           near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps)
    mins = np.asarray(sc.mins, np.float64)
    close = total = 0
    for n in range(len(ps)):
        eye = np.asarray(ps.origin[n], np.float64) + [0, 0, 12.0 if ps.ducked[n] else 17.0]
        ref = _remarch_f64(np.asarray(sc.sdf, np.float64), mins, sc.cell, eye, float(ps.yaw[n]),
                           float(ps.pitch[n]), W, H, w.range_units, w.near_range, w.hit_eps,
                           0.3 * sc.cell, w.max_steps)
        close += int((np.abs(enc[n] - ref) <= 1e-3).sum())
        total += ref.size
    assert close / total >= 0.99, f"{close}/{total} rays agree"


# ------------------------------------------------------------------ SDF bake --
def test_bake_matches_brute_force_on_tiny_grids():
    """oracle.edt.bake is the reference's scipy call (vision.py:428-432); an
    exhaustive nearest-solid search pins it, padding shell included."""
    from oracle import edt
    rng = np.random.default_rng(3)
    for trial in range(12):
        shp = tuple(int(v) for v in rng.integers(1, 9, 3))
        occ = (rng.random(shp) < rng.uniform(0.0, 0.25)).astype(np.uint8)
        cell = (16.0, 32.0, 8.0)[trial % 3]
        assert np.allclose(edt.bake(occ, cell), edt.brute_force(occ, cell), rtol=0, atol=1e-9)
    # closed forms: an empty grid measures the distance to the padding shell
    occ = np.zeros((3, 4, 5), np.uint8)
    d = edt.bake(occ, 16.0)
    z, y, x = np.indices(occ.shape)
    shell = np.minimum.reduce([x + 1, 5 - x, y + 1, 4 - y, z + 1, 3 - z]) * 16.0
    assert np.array_equal(d, shell)
    assert edt.stored(d).dtype == np.float32


# ------------------------------------------------------------ surf-mask channel --
def test_surf_channel_closed_form_on_a_floor():
    """The second channel is |n_z| of the voxel the march stopped in, read at
    the clamped depth (vision.py:176-187, :658-665). Floor slab, |n_z| grid
    127 in the solid layers and 0 in the air: every ray that stops on the
    floor reads exactly 1.0 (127 / 127), every ray that runs out to the
    range reads the air's 0, and the depth channel equals the depth-only
    render bit for bit."""
    cell = 16.0
    nz = 16
    g = np.maximum((np.arange(nz, dtype=np.float32) - 3.0) * cell, 0.0)[:, None, None] \
        * np.ones((1, 32, 32), np.float32)                    # solid for iz <= 3
    snz = np.where(g == 0.0, 127, 0).astype(np.int8)
    origin = np.array([[256.0, 256.0, 150.0], [100.0, 400.0, 180.0]], np.float32)
    yaw = np.array([10.0, -140.0], np.float32)
    pitch = np.array([-30.0, 5.0], np.float32)
    duck = np.zeros(2, np.float32)
    kw = dict(width=32, height=16, range_units=1500.0, near_range=1500.0, max_steps=200)
    both, loads = oracle.render(g, np.zeros(3, np.float32), cell, origin, yaw, pitch, duck,
                                surf_nz=snz, **kw)
    depth, _ = oracle.render(g, np.zeros(3, np.float32), cell, origin, yaw, pitch, duck, **kw)
    assert both.shape == (2, 16, 32, 2)
    assert np.array_equal(both[..., 0], depth)
    hit = both[..., 0] < 1.0
    assert 0.2 < hit.mean() < 0.9
    assert np.all(both[..., 1][hit] == 1.0)
    assert np.all(both[..., 1][~hit] == 0.0)


def test_surf_channel_reads_the_stop_voxel_of_each_ray():
    """On a ramp scene with a distinct |n_z| code per voxel, each ray's
    second channel is the code of the voxel its own march (the sample by
    sample trace) stopped in, divided by 127 in fp32 as the CPU path does
    (``snz.float() / 127.0``). For a hit that is the last voxel sampled; for
    a ray clamped to the range it is the voxel at the range point. Reading
    the voxel of the sample before the stop (a plausible slip) disagrees on
    most hits."""
    from oracle import agreement
    from surfgym import synth
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, 3)
    rng = np.random.default_rng(11)
    snz = rng.integers(0, 128, sc.sdf.shape).astype(np.int8)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps)
    img, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                           surf_nz=snz, **kw)
    lib = oracle._load()
    mins = np.asarray(sc.mins, np.float32)
    inv = F32(1.0 / sc.cell)
    nz, ny, nx = sc.sdf.shape
    hits = slips = 0
    for e in range(3):
        eye = (F32(ps.origin[e, 0]), F32(ps.origin[e, 1]),
               F32(F32(ps.origin[e, 2]) + F32(12.0 if ps.ducked[e] else 17.0)))
        for r in range(0, w.height, 3):
            for c in range(0, w.width, 5):
                d = np.empty(3, np.float32)
                lib.oracle_ray_dir(0, r, c, w.width, w.height, 120.0, 90.0, 0.0, 0.0,
                                   float(ps.yaw[e]), float(ps.pitch[e]),
                                   d.ctypes.data_as(oracle.ctypes.c_void_p))
                tr = agreement.trace(sc.sdf, mins, sc.cell, eye, d,
                                     range_units=w.range_units, hit_eps=w.hit_eps,
                                     min_step=float(F32(0.3 * sc.cell)), max_steps=w.max_steps)
                if tr["why"] == "hit":
                    ix, iy, iz = tr["vox"][-1]
                    hits += 1
                    px, py, pz = tr["vox"][-2] if len(tr["vox"]) > 1 else tr["vox"][-1]
                    slips += snz[pz, py, px] != snz[iz, iy, ix]
                else:
                    t = min(F32(tr["t"]), F32(w.range_units))
                    idx = []
                    for a, n in ((0, nx), (1, ny), (2, nz)):
                        f = F32(F32(F32(eye[a] + F32(d[a] * t)) - mins[a]) * inv)
                        idx.append(0 if not f > 0 else min(int(f), n - 1))
                    ix, iy, iz = idx
                assert img[e, r, c, 1] == F32(snz[iz, iy, ix]) / F32(127.0), (e, r, c, tr["why"])
    assert hits > 50
    assert slips > 0.5 * hits


def test_the_sample_by_sample_trace_reproduces_the_render():
    """oracle_march_trace (the per-sample record the agreement classifier
    re-traces rays with) marches exactly as the render does: for 300 random
    rays of small_ramps its final depth encodes to the render's value, its
    sample count is the render's load count, its first sample is the eye's
    voxel, each recorded t is the previous one plus max(0.9 s, min_step),
    and the stop reason matches the last sample."""
    from oracle import agreement
    from surfgym import synth
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, 6)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps)
    img, loads = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                               **kw)
    lib = oracle._load()
    rng = np.random.default_rng(3)
    mstep = F32(0.3 * sc.cell)
    for _ in range(300):
        e, r, c = int(rng.integers(6)), int(rng.integers(w.height)), int(rng.integers(w.width))
        eye = (F32(ps.origin[e, 0]), F32(ps.origin[e, 1]),
               F32(F32(ps.origin[e, 2]) + F32(12.0 if ps.ducked[e] else 17.0)))
        d = agreement._dir(lib, w.width, w.height, 120.0, 90.0, ps.yaw[e], ps.pitch[e], r, c)
        tr = agreement.trace(sc.sdf, sc.mins, sc.cell, eye, d, range_units=w.range_units,
                             hit_eps=w.hit_eps, min_step=float(mstep), max_steps=w.max_steps)
        t = min(F32(tr["t"]), F32(w.range_units))
        assert F32(oracle.encode(float(t), w.near_range)) == img[e, r, c]
        assert len(tr["t_k"]) == loads[e, r, c]
        assert tr["t_k"][0] == 0.0
        for k in range(1, len(tr["t_k"])):
            step = max(F32(tr["s_k"][k - 1] * F32(0.9)), mstep)
            assert tr["t_k"][k] == F32(tr["t_k"][k - 1] + step)
        last = tr["s_k"][-1]
        if tr["why"] == "hit":
            assert not last > w.hit_eps
        elif tr["why"] == "range":
            assert last > w.hit_eps and not tr["t_k"][-1] < w.range_units
        else:
            assert len(tr["t_k"]) == w.max_steps
