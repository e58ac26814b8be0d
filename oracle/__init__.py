"""CPU oracle for the SDF depth render — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg may
import this package: it is the oracle the GPU renderer is measured against,
never part of the product path.

Restatements of the reference's render (python/surfgym/vision.py) and of
its goal field:

* :func:`render` — per-ray C loop (``oracle/march.c``), the canonical oracle.
  It also returns the number of grid loads each ray issued (the census of
  tools/bench_lidar.py:45-88), which is the algorithmic-bytes count.
* :mod:`oracle.goal` — the goal-field bake and sampler
  (python/surfgym/goalfield.py), ``oracle/goal.c``.
* :mod:`oracle.agreement` — a render compared with the lockstep render
  (the reference's CPU arithmetic) at the accuracy bar (0.5 u, 1e-3), every
  ray outside it re-traced and classified.
* :mod:`oracle.lockstep` — the reference's CPU fallback shape
  (``_render_torch``, vision.py:626-666): torch tensors over all rays in
  lockstep, with a host ``any()`` check every 8 steps. It is the CPU
  baseline that bench.py times.
* :func:`as_stored` / :func:`r16_encode` / :func:`r16_decode` — the values
  the renderer reads from each grid store (fp32; fp16 as torch rounds it,
  vision.py:476; the r16 bricks, a storage format of this renderer).
* :mod:`oracle.edt` — the reference's scipy bake call (vision.py:428-438).

Where each is pinned (closed forms, invariants, brute force on tiny inputs,
an independent second implementation, planted mistakes):

* render (the surf-mask channel included), ray_dirs, offsets, encode —
  tests/test_oracle.py and the committed fixtures in tests/golden/
  (tests/test_golden.py);
* lockstep — tests/test_oracle_lockstep.py, against render;
* agreement — tests/test_oracle_lockstep.py: the grazing angle against a
  floor and a wall in closed form, each outlier's re-trace reproducing both
  renders, and planted mistakes (a yaw offset, corrupted pixels) caught;
* r16_encode / r16_decode — tests/test_oracle_store.py;
* edt — tests/test_oracle.py (exhaustive nearest-solid search);
* goal — tests/test_oracle_goal.py.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_march.so"

_lib = None


def build(verbose: bool = False) -> Path:
    """Compile march.c and goal.c with gcc (IEEE fp32, no contraction, OpenMP)."""
    import subprocess
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp",
           "-ffp-contract=off", "-fno-fast-math", "-fvisibility=hidden",
           str(HERE / "march.c"), str(HERE / "goal.c"), "-o", str(LIB_PATH) + ".tmp", "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(str(LIB_PATH) + ".tmp", LIB_PATH)
    return LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    f, i, d, p = ctypes.c_float, ctypes.c_int, ctypes.c_double, ctypes.c_void_p
    lib.oracle_equiangular_offset.restype = f
    lib.oracle_equiangular_offset.argtypes = [i, i, d]
    lib.oracle_pinhole_u.restype = f
    lib.oracle_pinhole_u.argtypes = [i, i, d]
    lib.oracle_pinhole_v.restype = f
    lib.oracle_pinhole_v.argtypes = [i, i, d]
    lib.oracle_ray_dir.restype = None
    lib.oracle_ray_dir.argtypes = [i, i, i, i, i, d, d, d, d, f, f, p]
    lib.oracle_encode.restype = f
    lib.oracle_encode.argtypes = [f, f]
    lib.oracle_march_ray.restype = f
    lib.oracle_march_ray.argtypes = [p, i, i, i, p, f, f, f, f, f, f, f, f, f, f, i, p]
    lib.oracle_march_trace.restype = i
    lib.oracle_march_trace.argtypes = [p, i, i, i, p, f, f, f, f, f, f, f, f, f, f, i, i,
                                       p, p, p, p, p, p]
    lib.oracle_render.restype = i
    lib.oracle_render.argtypes = [p, i, i, i, p, f, i, i, i, d, d, d, d, f, f, f, f, i,
                                  p, p, p, p, i, p, p, p, i]
    i64 = ctypes.c_int64
    lib.oracle_goal_distance.restype = i64
    lib.oracle_goal_distance.argtypes = [p, i, i, i, f, p, p, p]
    lib.oracle_goal_quantise.restype = i
    lib.oracle_goal_quantise.argtypes = [p, i64, f, p, p, p, p, p]
    lib.oracle_goal_sample.restype = None
    lib.oracle_goal_sample.argtypes = [p, i, i, i, p, d, d, p, i64, p]
    _lib = lib
    return lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def r16_encode(grid: np.ndarray):
    """The r16 brick store of a [nz,ny,nx] grid: (codes uint16 [bz,by,bx,64],
    base float32 [bz,by,bx], exponent int [bz,by,bx]).

    Per 4x4x4 brick of voxels (inner order x fastest, then y, then z; the
    brick grid padded up to whole bricks): base = the smallest value of the
    brick's voxels inside the grid; exponent e = the smallest integer >= -100
    with (max - base) <= 65535 * 2^e, at most 100 (for max > base, e is
    ilogb(max - base) - 15, plus one when that leaves the range above 65535
    units); code = round-half-even((value - base) * 2^-e) in fp64, clamped to
    [0, 65535] (NaN -> 0); padding voxels code 0. A storage format of this
    renderer (no reference counterpart): it gives the reference's fp32 grid
    values to within 2^(e-1) at two bytes per voxel.
    """
    g = np.ascontiguousarray(grid, dtype=np.float32)
    nz, ny, nx = g.shape
    bz, by, bx = (nz + 3) // 4, (ny + 3) // 4, (nx + 3) // 4
    pad = np.full((bz * 4, by * 4, bx * 4), np.nan, np.float64)
    pad[:nz, :ny, :nx] = g
    # [bz, 4(z), by, 4(y), bx, 4(x)] -> [bz, by, bx, 4z, 4y, 4x] -> 64 per brick
    b = pad.reshape(bz, 4, by, 4, bx, 4).transpose(0, 2, 4, 1, 3, 5).reshape(bz, by, bx, 64)
    inside = ~np.isnan(b)
    lo = np.where(inside, b, np.inf).min(axis=-1)
    hi = np.where(inside, b, -np.inf).max(axis=-1)
    rng = hi - lo                       # exact: differences of fp32 values in fp64
    e = np.full(rng.shape, -100, np.int64)
    pos = rng > 0
    _, ex = np.frexp(rng[pos])          # rng = m * 2^ex, m in [0.5, 1): ilogb = ex - 1
    ep = (ex - 1) - 15
    ep = ep + (np.ldexp(rng[pos], -ep) > 65535.0)
    e[pos] = np.clip(ep, -100, 100)
    q = np.rint((b - lo[..., None]) * np.ldexp(1.0, -e)[..., None])
    q = np.where(q >= 0.0, np.minimum(q, 65535.0), 0.0)   # NaN (padding) -> 0
    return q.astype(np.uint16), lo.astype(np.float32), e


def r16_decode(codes, base, exponent, shape) -> np.ndarray:
    """Voxel values the renderer reads from an r16 store, [nz,ny,nx] f32:
    f32(base + f32(code * 2^e)) (the product is exact in fp32)."""
    nz, ny, nx = shape
    bz, by, bx = base.shape
    scale = np.ldexp(np.float32(1.0), exponent).astype(np.float32)
    v = base[..., None] + codes.astype(np.float32) * scale[..., None]   # fp32 add, one rounding
    v = v.astype(np.float32).reshape(bz, by, bx, 4, 4, 4).transpose(0, 3, 1, 4, 2, 5)
    return np.ascontiguousarray(v.reshape(bz * 4, by * 4, bx * 4)[:nz, :ny, :nx])


def as_stored(grid: np.ndarray, store: str) -> np.ndarray:
    """The voxel values the renderer reads: f32 as given; rounded to f16
    (round to nearest even, as torch's ``.to(torch.float16)``, vision.py:476)
    and widened back; or through the r16 brick store (:func:`r16_encode`)."""
    g = np.ascontiguousarray(grid, dtype=np.float32)
    if store in ("f16", "float16"):
        return g.astype(np.float16).astype(np.float32)
    if store in ("f32", "float32"):
        return g
    if store == "r16":
        return r16_decode(*r16_encode(g), g.shape)
    raise ValueError(f"unknown store dtype {store!r}")


def render(grid, mins, cell, origin, yaw_deg, pitch_deg, ducked, *, width=128, height=64,
           hfov_deg=120.0, vfov_deg=90.0, range_units=2000.0, near_range=None,
           hit_eps=None, min_step=None, max_steps=64, pinhole=False, store="f32",
           surf_nz=None, threads=0):
    """Depth encodings (N,H,W) f32 and grid loads per ray (N,H,W) int32.

    With ``surf_nz`` (int8 [nz,ny,nx], |n_z|*127) the image is (N,H,W,2):
    depth and |n_z| at the voxel the march stopped in (vision.py:654-666).

    Defaults and derived constants follow GpuLidar (vision.py:457-509):
    near = range when not given, hit_eps = 0.6*cell, min_step = 0.3*cell
    (vision.py:87-88, 637-638), both rounded to fp32 as the comparison does.
    """
    lib = _load()
    g = as_stored(grid, store)
    nz, ny, nx = g.shape
    mins = np.ascontiguousarray(mins, dtype=np.float32).reshape(3)
    origin = np.ascontiguousarray(origin, dtype=np.float32).reshape(-1, 3)
    n = origin.shape[0]
    yaw = np.ascontiguousarray(yaw_deg, dtype=np.float32).reshape(n)
    pitch = np.ascontiguousarray(pitch_deg, dtype=np.float32).reshape(n)
    duck = np.ascontiguousarray(np.asarray(ducked, dtype=np.float64) != 0, dtype=np.float32).reshape(n)
    rng = float(range_units)
    near = float(near_range) if near_range else rng
    eps = float(np.float32(0.6 * cell)) if hit_eps is None else float(hit_eps)
    mstep = float(np.float32(0.3 * cell)) if min_step is None else float(min_step)
    tan_h = float(np.tan(0.5 * hfov_deg * (np.pi / 180.0)))
    tan_v = float(np.tan(0.5 * vfov_deg * (np.pi / 180.0)))
    nzg = None
    if surf_nz is not None:
        nzg = np.ascontiguousarray(surf_nz, dtype=np.int8)
        if nzg.shape != g.shape:
            raise ValueError(f"surf_nz grid {nzg.shape} != SDF grid {g.shape}")
    out = np.empty((n, height, width) + ((2,) if nzg is not None else ()), np.float32)
    loads = np.empty((n, height, width), np.int32)
    rc = lib.oracle_render(_ptr(g), nx, ny, nz, _ptr(mins), float(cell), width, height,
                           1 if pinhole else 0, float(hfov_deg), float(vfov_deg), tan_h, tan_v,
                           rng, near, eps, mstep, int(max_steps), _ptr(origin), _ptr(yaw),
                           _ptr(pitch), _ptr(duck), n, _ptr(out), _ptr(loads),
                           _ptr(nzg) if nzg is not None else None, int(threads))
    if rc != 0:
        raise ValueError("oracle_render rejected its arguments")
    return out, loads


def ray_dirs(width, height, yaw_deg, pitch_deg, *, hfov_deg=120.0, vfov_deg=90.0,
             pinhole=False):
    """(H,W,3) unit ray directions of one pose, as the oracle's march uses."""
    lib = _load()
    tan_h = float(np.tan(0.5 * hfov_deg * (np.pi / 180.0)))
    tan_v = float(np.tan(0.5 * vfov_deg * (np.pi / 180.0)))
    out = np.empty((height, width, 3), np.float32)
    buf = np.empty(3, np.float32)
    for r in range(height):
        for c in range(width):
            lib.oracle_ray_dir(1 if pinhole else 0, r, c, width, height, float(hfov_deg),
                               float(vfov_deg), tan_h, tan_v, float(yaw_deg),
                               float(pitch_deg), _ptr(buf))
            out[r, c] = buf
    return out


def encode(t: float, near: float) -> float:
    return float(_load().oracle_encode(float(t), float(near)))


def offsets(width, height, hfov_deg=120.0, vfov_deg=90.0):
    """The equiangular (yoff (W,), poff (H,)) tables as f32."""
    lib = _load()
    yo = np.array([lib.oracle_equiangular_offset(c, width, float(hfov_deg))
                   for c in range(width)], np.float32)
    po = np.array([lib.oracle_equiangular_offset(r, height, float(vfov_deg))
                   for r in range(height)], np.float32)
    return yo, po
