"""Seeded synthetic surf scenes and poses for the depth renderer.

The reference renders baked maps (python/surfgym/vision.py build_sdf
:409-439). Its own renderer tests instead monkeypatch analytic grids in
(tests/python/test_pinhole.py:186-202, test_surfmask.py:177-193); this module
does the same at benchmark scale. A scene is a ground half-space, surf ramps
(triangular prisms with 45-60 degree faces, the geometry surf maps are made
of) and boxes; the grid holds the exact unsigned distance from each voxel
centre to the nearest solid, 0 inside (the reference's EDT convention,
vision.py:428-432), evaluated by ``csrc/synth.c``.

Named workloads (all 128x64 rays per env unless stated):

=================== ============================ ======== ======= ===========
name                grid (f32 unless stated)      envs     steps   range/near
=================== ============================ ======== ======= ===========
small_ramps         64x64x32 @16 u, plane+8 ramps 16       64      1536 / 1536
ramp_field          256x256x128 @16 u, 64 ramps   2048     96      6144 / 2000
                    + 16 boxes
winding_track       1024x1024x256 @16 u, track of 2048     96      23530 / 2000
                    300 ramp segments
sparse_grazing      256x256x128 @16 u, 16 ramps,  8192     256     6144 / 2000
                    pitch N(0,5 deg)
ramp_field_f16_bf16 ramp_field scene stored f16,  8192     96      6144 / 2000
                    bf16 output
ramp_field_r16_bf16 ramp_field scene stored as    8192     96      6144 / 2000
                    r16 bricks, bf16 output
map_scale           1536x1536x280 @32 u stored    2048     64      11500 / 2000
                    f16, track of 600 segments
=================== ============================ ======== ======= ===========

map_scale is no benchmark configuration: it is a map of the size the
reference's production map has (surf_src_cannonball, ~654 M voxels at 32 u,
fp16; python/surfgym/vision.py:433-437) with the reference's production
sensor (range 11500, near 2000, 64 steps; docs/perf-results.md:73).

hit_eps is 1 u in every workload. Scene seeds are 1000+k and pose seeds
2000+k (numpy PCG64) for the k-th row above; the two fused-output rows share
scene and poses (seed 2004) and differ only in the grid store.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

PKG_ROOT = Path(__file__).resolve().parents[1]
SYNTH_LIB = PKG_ROOT / "lib" / "libsurfsynth.so"

_PRISM = np.dtype([("cx", "<f4"), ("cy", "<f4"), ("z0", "<f4"), ("ax", "<f4"), ("ay", "<f4"),
                   ("half_len", "<f4"), ("half_base", "<f4"), ("height", "<f4")])
_BOX = np.dtype([("cx", "<f4"), ("cy", "<f4"), ("cz", "<f4"), ("hx", "<f4"), ("hy", "<f4"),
                 ("hz", "<f4"), ("cos_a", "<f4"), ("sin_a", "<f4")])

_lib = None


def _load():
    global _lib
    if _lib is None:
        if not SYNTH_LIB.exists():
            raise RuntimeError(f"{SYNTH_LIB} is not built: run __graft_entry__.build()")
        lib = ctypes.CDLL(str(SYNTH_LIB))
        p, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        lib.synth_eval.restype = i
        lib.synth_eval.argtypes = [p, i, i, i, p, f, i, f, p, i, p, i, f, i]
        lib.synth_eval_brute.restype = i
        lib.synth_eval_brute.argtypes = [p, i, i, i, p, f, i, f, p, i, p, i, f]
        lib.synth_query.restype = None
        lib.synth_query.argtypes = [p, i, i, f, p, i, p, i, f, p]
        _lib = lib
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None and a.size else None


@dataclass
class Scene:
    """Solids plus the sampled grid ([nz,ny,nx] f32, mins (3,) f32, cell)."""
    nx: int
    ny: int
    nz: int
    mins: np.ndarray
    cell: float
    ground_z: float | None
    prisms: np.ndarray
    boxes: np.ndarray
    trunc: float = 1.0e6
    sdf: np.ndarray | None = field(default=None, repr=False)

    @property
    def extent(self) -> np.ndarray:
        return np.array([self.nx, self.ny, self.nz], np.float64) * self.cell

    @property
    def diagonal(self) -> float:
        return float(np.linalg.norm(self.extent))

    def bake(self, threads: int = 0, brute: bool = False) -> np.ndarray:
        lib = _load()
        out = np.empty((self.nz, self.ny, self.nx), np.float32)
        mins = np.ascontiguousarray(self.mins, np.float32)
        has_ground = self.ground_z is not None
        gz = float(self.ground_z) if has_ground else 0.0
        pr = np.ascontiguousarray(self.prisms, _PRISM)
        bx = np.ascontiguousarray(self.boxes, _BOX)
        if brute:
            rc = lib.synth_eval_brute(_ptr(out), self.nx, self.ny, self.nz, _ptr(mins),
                                      float(self.cell), int(has_ground), gz, _ptr(pr), len(pr),
                                      _ptr(bx), len(bx), float(self.trunc))
        else:
            rc = lib.synth_eval(_ptr(out), self.nx, self.ny, self.nz, _ptr(mins),
                                float(self.cell), int(has_ground), gz, _ptr(pr), len(pr),
                                _ptr(bx), len(bx), float(self.trunc), int(threads))
        if rc != 0:
            raise RuntimeError("synth_eval failed")
        self.sdf = out
        return out

    def distance(self, xyz: np.ndarray) -> np.ndarray:
        """Exact distance to the nearest solid at arbitrary points (n,3)."""
        lib = _load()
        pts = np.ascontiguousarray(xyz, np.float32).reshape(-1, 3)
        out = np.empty(len(pts), np.float32)
        has_ground = self.ground_z is not None
        pr = np.ascontiguousarray(self.prisms, _PRISM)
        bx = np.ascontiguousarray(self.boxes, _BOX)
        lib.synth_query(_ptr(pts), len(pts), int(has_ground),
                        float(self.ground_z) if has_ground else 0.0, _ptr(pr), len(pr),
                        _ptr(bx), len(bx), float(self.trunc), _ptr(out))
        return out

    def grid_value(self, xyz: np.ndarray) -> np.ndarray:
        """The nearest-voxel grid value the march would read at points (n,3)."""
        assert self.sdf is not None, "bake() first"
        p = np.asarray(xyz, np.float32).reshape(-1, 3)
        idx = ((p - self.mins.astype(np.float32)) * np.float32(1.0 / self.cell))
        hi = np.array([self.nx - 1, self.ny - 1, self.nz - 1], np.float32)
        idx = np.clip(idx, 0.0, hi).astype(np.int64)
        return self.sdf[idx[:, 2], idx[:, 1], idx[:, 0]]


def _ramp(rng, cx, cy, z0, angle, half_len, half_base, slope_deg):
    h = half_base * math.tan(math.radians(slope_deg))
    return (cx, cy, z0, math.cos(angle), math.sin(angle), half_len, half_base, h)


def ramp_scene(nx, ny, nz, cell, n_prisms, n_boxes, seed, *, ground_frac=0.0625,
               len_range=(150.0, 600.0), base_range=(60.0, 220.0)) -> Scene:
    """A ground plane, ramps scattered at random heights and boxes."""
    rng = np.random.default_rng(seed)
    ext = np.array([nx, ny, nz], np.float64) * cell
    mins = np.array([-ext[0] / 2, -ext[1] / 2, -ext[2] / 4], np.float32)
    ground = float(mins[2] + ground_frac * ext[2])
    top = float(mins[2] + ext[2])
    pr = []
    for _ in range(n_prisms):
        hl = rng.uniform(*len_range)
        hb = rng.uniform(*base_range)
        slope = rng.uniform(45.0, 60.0)
        h = hb * math.tan(math.radians(slope))
        margin = 0.05 * ext[:2]
        cx = rng.uniform(mins[0] + margin[0], mins[0] + ext[0] - margin[0])
        cy = rng.uniform(mins[1] + margin[1], mins[1] + ext[1] - margin[1])
        zmax = max(ground, top - h - 0.3 * ext[2])
        z0 = ground if rng.random() < 0.25 else rng.uniform(ground, zmax)
        pr.append(_ramp(rng, cx, cy, z0, rng.uniform(0.0, math.pi), hl, hb, slope))
    bx = []
    for _ in range(n_boxes):
        hx, hy, hz = rng.uniform(64.0, 256.0), rng.uniform(64.0, 256.0), rng.uniform(16.0, 128.0)
        cx = rng.uniform(mins[0] + hx, mins[0] + ext[0] - hx)
        cy = rng.uniform(mins[1] + hy, mins[1] + ext[1] - hy)
        cz = rng.uniform(ground + hz, ground + 0.6 * (top - ground))
        a = rng.uniform(0.0, math.pi)
        bx.append((cx, cy, cz, hx, hy, hz, math.cos(a), math.sin(a)))
    return Scene(nx, ny, nz, mins, float(cell), ground,
                 np.array(pr, _PRISM).reshape(-1), np.array(bx, _BOX).reshape(-1))


def track_scene(nx, ny, nz, cell, n_segments, seed) -> Scene:
    """A long winding descending track of ramp segments above a ground plane."""
    rng = np.random.default_rng(seed)
    ext = np.array([nx, ny, nz], np.float64) * cell
    mins = np.array([-ext[0] / 2, -ext[1] / 2, -ext[2] / 4], np.float32)
    ground = float(mins[2] + 0.0625 * ext[2])
    lo = mins[:2].astype(np.float64) + 0.06 * ext[:2]
    hi = mins[:2].astype(np.float64) + 0.94 * ext[:2]
    pos = lo + rng.uniform(0.0, 0.2, 2) * (hi - lo)
    heading = rng.uniform(0.0, 2 * math.pi)
    z = float(mins[2] + 0.85 * ext[2])
    z_end = ground + 0.1 * ext[2]
    dz = (z - z_end) / n_segments
    pr = []
    for _ in range(n_segments):
        seg = rng.uniform(350.0, 700.0)
        heading += rng.normal(0.0, math.radians(18.0))
        nxt = pos + seg * np.array([math.cos(heading), math.sin(heading)])
        # turn back into the map instead of leaving it
        for _ in range(12):
            if np.all(nxt >= lo) and np.all(nxt <= hi):
                break
            heading += math.radians(35.0)
            nxt = pos + seg * np.array([math.cos(heading), math.sin(heading)])
        nxt = np.clip(nxt, lo, hi)
        c = 0.5 * (pos + nxt)
        hb = rng.uniform(90.0, 200.0)
        pr.append(_ramp(rng, c[0], c[1], z, heading, 0.5 * seg + 40.0, hb,
                        rng.uniform(45.0, 60.0)))
        pos = nxt
        z -= dz
    return Scene(nx, ny, nz, mins, float(cell), ground, np.array(pr, _PRISM).reshape(-1),
                 np.zeros(0, _BOX))


@dataclass
class Poses:
    origin: np.ndarray   # (N,3) f32
    yaw: np.ndarray      # (N,) f32 degrees
    pitch: np.ndarray    # (N,) f32 degrees
    ducked: np.ndarray   # (N,) f32 0/1

    def __len__(self):
        return len(self.yaw)


def _view_angles(rng, n, pitch_mode):
    yaw = rng.uniform(-180.0, 180.0, n)
    if pitch_mode == "grazing":
        pitch = np.clip(rng.normal(0.0, 5.0, n), -70.0, 30.0)
    else:
        pitch = rng.uniform(-70.0, 30.0, n)
    ducked = (rng.random(n) < 0.5).astype(np.float32)
    return yaw.astype(np.float32), pitch.astype(np.float32), ducked


def poses_free_space(scene: Scene, n, seed, *, clearance=32.0, pitch_mode="uniform") -> Poses:
    """Origins uniform over the grid box where the grid reads > clearance."""
    rng = np.random.default_rng(seed)
    lo = scene.mins.astype(np.float64)
    hi = lo + scene.extent
    out = np.empty((0, 3), np.float32)
    while len(out) < n:
        cand = rng.uniform(lo, hi, (4 * n + 16, 3)).astype(np.float32)
        ok = scene.grid_value(cand) > clearance
        eye = cand.copy()
        eye[:, 2] += 17.0
        ok &= scene.grid_value(eye) > clearance
        out = np.concatenate([out, cand[ok]])
    yaw, pitch, duck = _view_angles(rng, n, pitch_mode)
    return Poses(np.ascontiguousarray(out[:n]), yaw, pitch, duck)


def poses_above_ramps(scene: Scene, n, seed, *, lift=(400.0, 800.0), clearance=32.0,
                      pitch_mode="uniform") -> Poses:
    """Origins lift[0]..lift[1] u above a random point of a random ramp face,
    kept where the grid reads > clearance and inside the grid."""
    rng = np.random.default_rng(seed)
    pr = scene.prisms
    lo = scene.mins.astype(np.float64)
    hi = lo + scene.extent
    got = []
    while len(got) < n:
        m = 4 * (n - len(got)) + 16
        i = rng.integers(0, len(pr), m)
        p = pr[i]
        s = rng.uniform(-0.9, 0.9, m) * p["half_len"]
        u = rng.uniform(0.0, 1.0, m) * p["half_base"]
        side = np.where(rng.random(m) < 0.5, -1.0, 1.0)
        w = p["height"] * (1.0 - u / p["half_base"])
        x = p["cx"] + s * p["ax"] - side * u * p["ay"]
        y = p["cy"] + s * p["ay"] + side * u * p["ax"]
        z = p["z0"] + w + rng.uniform(lift[0], lift[1], m)
        cand = np.stack([x, y, z], 1).astype(np.float32)
        inside = np.all((cand >= lo + scene.cell) & (cand <= hi - 2 * scene.cell), axis=1)
        cand = cand[inside]
        if len(cand):
            ok = scene.grid_value(cand) > clearance
            got.extend(cand[ok])
    yaw, pitch, duck = _view_angles(rng, n, pitch_mode)
    return Poses(np.ascontiguousarray(np.array(got[:n], np.float32)), yaw, pitch, duck)


@dataclass
class Workload:
    """One render workload: a scene recipe, a pose recipe and the sensor."""
    name: str
    scene_fn: object
    pose_fn: object
    n_envs: int
    max_steps: int
    range_units: float
    near_range: float
    hit_eps: float = 1.0
    width: int = 128
    height: int = 64
    store: str = "f32"
    out_dtype: str = "f32"

    def scene(self) -> Scene:
        s = self.scene_fn()
        s.bake()
        return s

    def poses(self, scene: Scene, n_envs: int | None = None) -> Poses:
        return self.pose_fn(scene, self.n_envs if n_envs is None else n_envs)

    @property
    def rays(self) -> int:
        return self.n_envs * self.width * self.height


def _small_scene():
    return ramp_scene(64, 64, 32, 16.0, 8, 0, 1000, ground_frac=0.125,
                      len_range=(100.0, 300.0), base_range=(40.0, 120.0))


def _field_scene():
    return ramp_scene(256, 256, 128, 16.0, 64, 16, 1001)


def _track_scene():
    return track_scene(1024, 1024, 256, 16.0, 300, 1002)


def _sparse_scene():
    return ramp_scene(256, 256, 128, 16.0, 16, 0, 1003)


def _map_scale_scene():
    return track_scene(1536, 1536, 280, 32.0, 600, 1006)


SMALL_DIAG = float(np.linalg.norm(np.array([64, 64, 32]) * 16.0))       # 1536
TRACK_DIAG = float(np.linalg.norm(np.array([1024, 1024, 256]) * 16.0))  # 4096*sqrt(33)

WORKLOADS = {
    "small_ramps": Workload(
        "small_ramps", _small_scene, lambda s, n: poses_free_space(s, n, 2000),
        n_envs=16, max_steps=64, range_units=SMALL_DIAG, near_range=SMALL_DIAG),
    "ramp_field": Workload(
        "ramp_field", _field_scene, lambda s, n: poses_above_ramps(s, n, 2001),
        n_envs=2048, max_steps=96, range_units=6144.0, near_range=2000.0),
    "winding_track": Workload(
        "winding_track", _track_scene, lambda s, n: poses_above_ramps(s, n, 2002),
        n_envs=2048, max_steps=96, range_units=TRACK_DIAG, near_range=2000.0),
    "sparse_grazing": Workload(
        "sparse_grazing", _sparse_scene,
        lambda s, n: poses_above_ramps(s, n, 2003, pitch_mode="grazing"),
        n_envs=8192, max_steps=256, range_units=6144.0, near_range=2000.0),
    "ramp_field_f16_bf16": Workload(
        "ramp_field_f16_bf16", _field_scene, lambda s, n: poses_above_ramps(s, n, 2004),
        n_envs=8192, max_steps=96, range_units=6144.0, near_range=2000.0,
        store="f16", out_dtype="bf16"),
    "ramp_field_r16_bf16": Workload(
        "ramp_field_r16_bf16", _field_scene, lambda s, n: poses_above_ramps(s, n, 2004),
        n_envs=8192, max_steps=96, range_units=6144.0, near_range=2000.0,
        store="r16", out_dtype="bf16"),
    "map_scale": Workload(
        "map_scale", _map_scale_scene, lambda s, n: poses_above_ramps(s, n, 2006),
        n_envs=2048, max_steps=64, range_units=11500.0, near_range=2000.0, store="f16"),
}


# --------------------------------------------------------------- goal field --
def goal_zone(scene: Scene) -> dict:
    """A goal box ({"mins", "maxs"}, map units, the reference's zone format):
    96 x 96 x 64 u centred 80 u above the last ramp of a track scene, or over
    the ground near the far corner of a ramp scene."""
    if scene.boxes.size == 0 and len(scene.prisms) > 100:        # a track: its last segment
        p = scene.prisms[-1]
        c = np.array([p["cx"], p["cy"], p["z0"] + p["height"] + 80.0], np.float64)
    else:
        ext = scene.extent
        c = scene.mins.astype(np.float64) + np.array([0.92 * ext[0], 0.92 * ext[1], 0.0])
        c[2] = float(scene.ground_z) + 96.0
    h = np.array([48.0, 48.0, 32.0])
    return {"mins": (c - h).tolist(), "maxs": (c + h).tolist()}


def maze_occupancy(nx: int, ny: int, nz: int, seed: int, *, room: int = 8, storey: int = 16):
    """A 3-D labyrinth [nz, ny, nx] uint8 (1 = solid): walls every ``room``
    voxels along x and y with one 2x3-voxel doorway per wall segment, and a
    floor every ``storey`` voxels along z with one 2x2 hole per room — long
    winding geodesics for the goal-field bake."""
    rng = np.random.default_rng(seed)
    occ = np.zeros((nz, ny, nx), np.uint8)
    occ[:, :, ::room] = 1
    occ[:, ::room, :] = 1
    for z0 in range(0, nz, storey):
        occ[z0, :, :] = 1
    rx, ry = (nx + room - 1) // room, (ny + room - 1) // room
    for z0 in range(0, nz, storey):
        z1 = min(z0 + storey, nz)
        for j in range(ry):
            for i in range(rx):
                x0, y0 = i * room, j * room
                # doorway in the x-wall (plane x = x0) and in the y-wall (plane y = y0)
                if z1 - z0 > 4:
                    dz = int(rng.integers(z0 + 1, z1 - 3))
                    dy = int(rng.integers(y0 + 1, min(y0 + room - 2, ny - 2) + 1))
                    occ[dz:dz + 3, dy:dy + 2, x0] = 0
                    dx = int(rng.integers(x0 + 1, min(x0 + room - 2, nx - 2) + 1))
                    occ[dz:dz + 3, y0, dx:dx + 2] = 0
                if z0 > 0 and rng.random() < 0.5:
                    hx = int(rng.integers(x0 + 1, min(x0 + room - 2, nx - 2) + 1))
                    hy = int(rng.integers(y0 + 1, min(y0 + room - 2, ny - 2) + 1))
                    occ[z0, hy:hy + 2, hx:hx + 2] = 0
    return occ


@dataclass
class GoalWorkload:
    """An occupancy grid, its placement and a goal zone."""
    name: str
    occ: np.ndarray
    mins: np.ndarray
    cell: float
    zone: dict


def goal_workload(name: str) -> GoalWorkload:
    """ramp_field / winding_track: the render scenes' solid voxels with
    goal_zone(); maze: maze_occupancy(256, 256, 64) at 16 u, goal in the
    far top corner room."""
    if name in ("ramp_field", "winding_track", "small_ramps"):
        sc = WORKLOADS[name].scene()
        occ = (sc.sdf == 0).astype(np.uint8)
        return GoalWorkload(name, occ, sc.mins.astype(np.float64), sc.cell, goal_zone(sc))
    if name == "maze":
        occ = maze_occupancy(256, 256, 64, 3000)
        mins = np.zeros(3)
        c = np.array([252.0, 252.0, 60.0]) * 16.0
        return GoalWorkload(name, occ, mins, 16.0,
                            {"mins": (c - 24.0).tolist(), "maxs": (c + 24.0).tolist()})
    raise KeyError(f"unknown goal workload {name!r}")
