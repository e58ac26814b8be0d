"""Goal field on the GPU: geodesic distance-to-finish over a map's free space.

Drop-in for the reference's python/surfgym/goalfield.py ``GoalField`` and
``build_goal_field``. The bake (the reference's torch Bellman-Ford,
goalfield.py:159-298) and the trilinear honest-corner sampler
(GoalField.sample, :68-94) run in libsdfr.so (csrc/goal.hip, include/sdfr.h):

* the bake relaxes 8x8x8 tiles in LDS to local stability and keeps a queue of
  the tiles a wavefront still has to cross; it reaches the same fp32 fixpoint
  as the reference's whole-grid sweeps, then applies the reference's
  sentinel and uint16 quantisation, so a baked field equals the reference's
  cache file value for value;
* ``GoalField`` keeps its grid on the device and samples any number of
  positions per launch; given numpy positions it returns numpy, like the
  reference; given a device tensor it returns a device tensor without a host
  synchronisation.

There is no CPU path: a missing native library is an error.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import torch

from . import _sdfr, vision

__all__ = ["GoalField", "EuclidField", "build_goal_field", "goal_field_from_occupancy",
           "zone_seed_box", "seed_voxel_box", "goal_occupancy"]

# the reference's cache versioning (goalfield.py:44-47): a cache written here
# carries the same signature as one the reference wrote
_GOAL_BUILDER_VERSION = 4
MAX_SWEEPS = 1 << 20
_map_sig = vision._map_sig


def zone_seed_box(zone, cell: float):
    """The goal box inflated by max(0.75*cell, 20) u on every side
    (goalfield.py:148-156), float64 (mins, maxs)."""
    grow = max(0.75 * cell, 20.0)
    mins = np.asarray(zone["mins"], np.float64) - grow
    maxs = np.asarray(zone["maxs"], np.float64) + grow
    return mins, maxs


def seed_voxel_box(zone, mins, cell: float, dims):
    """Inclusive voxel box (lo, hi), (x, y, z) int32, of the voxel centres
    inside the inflated goal box, clipped to the grid (goalfield.py:228-231).
    ``dims`` is (nx, ny, nz)."""
    smin, smax = zone_seed_box(zone, cell)
    mins = np.asarray(mins, np.float64)
    nx, ny, nz = (int(v) for v in dims)
    lo = np.maximum(np.floor((smin - mins) / cell - 0.5), 0).astype(int)
    hi = np.minimum(np.ceil((smax - mins) / cell - 0.5), [nx - 1, ny - 1, nz - 1]).astype(int)
    return lo.astype(np.int32), hi.astype(np.int32)


def _grid_tensor(grid):
    """(tensor, SDFR dtype code): float32 distances, or uint16 quantised
    values held as int16 bits (torch's uint16 supports few operations)."""
    if torch.is_tensor(grid):
        if grid.dtype == torch.float32:
            return grid, _sdfr.F32
        if grid.dtype in (torch.int16, torch.uint16):
            return grid.view(torch.int16), _sdfr.U16
        raise ValueError(f"grid dtype must be float32 or uint16, got {grid.dtype}")
    a = np.asarray(grid)
    if a.dtype == np.float32:
        return torch.from_numpy(np.ascontiguousarray(a)), _sdfr.F32
    if a.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)), _sdfr.U16
    raise ValueError(f"grid dtype must be float32 or uint16, got {a.dtype}")


def _cuda_device(device) -> torch.device:
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError("the goal field runs on a ROCm GPU; there is no CPU path")
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


class GoalField:
    """Sampled geodesic distance-to-goal in map units, resident on the GPU.

    Same constructor and methods as the reference's GoalField
    (goalfield.py:50-107). ``grid`` [nz, ny, nx] is either the float32
    distance grid (numpy or torch) or the uint16 grid of the cache file with
    its ``quant``; values at or above ``reach_max + cell/2`` are not honest
    (solid or unreachable) and are skipped by :meth:`sample`.
    """

    def __init__(self, grid, mins, cell: float, reach_max: float, *, quant=None, device="cuda"):
        self.device = _cuda_device(device)
        g, self._kind = _grid_tensor(grid)
        if g.dim() != 3:
            raise ValueError(f"grid must be [nz, ny, nx], got shape {tuple(g.shape)}")
        if self._kind == _sdfr.U16 and quant is None:
            raise ValueError("a uint16 grid needs its quant")
        self.quant = float(np.float32(quant)) if quant is not None else 0.0
        self._grid = g.to(self.device).contiguous()
        self.mins = np.asarray(mins, np.float64)
        self.cell = float(cell)
        self.reach_max = float(reach_max)
        self.sentinel = float(self.reach_max + 2.0 * self.cell)
        self._valid_max = self.reach_max + 0.5 * self.cell
        self.dims = np.array(self._grid.shape[::-1])     # (nx, ny, nz)
        self._mins_c = (ctypes.c_double * 3)(*self.mins.tolist())
        self.bake_info: dict | None = None
        self.grid_q: torch.Tensor | None = None

    @property
    def grid(self) -> torch.Tensor:
        """The distance grid in map units, float32 on the device."""
        if self._kind == _sdfr.F32:
            return self._grid
        return (self._grid.to(torch.int32) & 0xFFFF).to(torch.float32) * np.float32(self.quant)

    def _positions(self, pos):
        """(tensor on the device (n, >=3) with unit inner stride, dtype code,
        row stride, was_numpy)."""
        if torch.is_tensor(pos):
            p = pos if pos.dim() == 2 else pos.reshape(-1, pos.shape[-1])
            if p.device != self.device:
                raise ValueError(f"positions on {p.device}, field on {self.device}")
            if p.dtype not in (torch.float32, torch.float64):
                p = p.to(torch.float64)
            if p.shape[1] < 3:
                raise ValueError("positions must have 3 columns")
            if p.stride(1) != 1 or p.stride(0) < 3:
                p = p[:, :3].contiguous()
            return p, (_sdfr.F32 if p.dtype == torch.float32 else _sdfr.F64), p.stride(0), False
        a = np.atleast_2d(np.asarray(pos, np.float64))
        if a.shape[-1] != 3:
            raise ValueError(f"positions must be (N, 3), got {a.shape}")
        p = torch.from_numpy(np.ascontiguousarray(a.reshape(-1, 3))).to(self.device)
        return p, _sdfr.F64, 3, True

    def _sample_dev(self, p, code, stride) -> torch.Tensor:
        lib = _sdfr.load()
        n = int(p.shape[0])
        out = torch.empty(n, dtype=torch.float32, device=self.device)
        if n == 0:
            return out
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            rc = lib.sdfr_goal_sample(self._grid.data_ptr(), self._kind, float(self.quant),
                                      int(self.dims[0]), int(self.dims[1]), int(self.dims[2]),
                                      self._mins_c, self.cell, self.reach_max,
                                      p.data_ptr(), code, int(stride), n, out.data_ptr(), stream)
        if rc != 0:
            raise _sdfr.SdfrError(f"sdfr_goal_sample failed ({rc}): "
                                  f"{lib.sdfr_goal_last_error().decode('utf-8', 'replace')}")
        return out

    def sample(self, pos):
        """Trilinear geodesic distance at ``pos`` (N, 3) -> (N,) float32 over
        honest corners only; ``sentinel`` where none is honest
        (goalfield.py:68-94). numpy in, numpy out; a device tensor in, a
        device tensor out (no host synchronisation)."""
        p, code, stride, was_np = self._positions(pos)
        out = self._sample_dev(p, code, stride)
        return out.cpu().numpy() if was_np else out

    def reachable(self, pos):
        """True where a finite path to the goal exists (goalfield.py:96-99)."""
        s = self.sample(pos)
        thr = np.float32(self.reach_max - 0.5 * self.cell)
        return s < thr if isinstance(s, np.ndarray) else s < float(thr)

    def descent_yaw(self, pos):
        """Yaw in degrees of the steepest horizontal descent
        (goalfield.py:101-107): one launch samples p +- cell along x and y."""
        p, _, _, was_np = self._positions(pos)
        p = p[:, :3].to(torch.float64)
        h = self.cell
        off = torch.tensor([[h, 0, 0], [-h, 0, 0], [0, h, 0], [0, -h, 0]], dtype=torch.float64,
                           device=self.device)
        q = (p[None, :, :] + off[:, None, :]).reshape(-1, 3).contiguous()
        s = self._sample_dev(q, _sdfr.F64, 3).view(4, -1)
        dx = s[0] - s[1]
        dy = s[2] - s[3]
        yaw = torch.remainder(torch.rad2deg(torch.atan2(-dy, -dx)), 360.0)
        return yaw.cpu().numpy() if was_np else yaw


class EuclidField:
    """Straight-line distance to the goal box, walls ignored
    (goalfield.py:110-137): the field of ``--race-dist euclid``, with no bake.
    Same methods as :class:`GoalField`; every position counts as reachable.
    Host numpy in and out, as the reference's; a handful of positions per
    tick is not worth a launch."""

    def __init__(self, zone):
        self.mins = np.asarray(zone["mins"], np.float64)
        self.maxs = np.asarray(zone["maxs"], np.float64)

    def _nearest(self, pos):
        p = np.atleast_2d(np.asarray(pos, np.float64))
        return p, np.minimum(np.maximum(p, self.mins), self.maxs)   # closest point of the box

    def sample(self, pos) -> np.ndarray:
        """(N,) float32 distance from each position to the box (0 inside)."""
        p, q = self._nearest(pos)
        return np.sqrt(((p - q) ** 2).sum(axis=1)).astype(np.float32)

    def reachable(self, pos) -> np.ndarray:
        return np.ones(len(np.atleast_2d(pos)), bool)

    def descent_yaw(self, pos) -> np.ndarray:
        """Yaw in degrees [0, 360) pointing at the box's closest point."""
        p, q = self._nearest(pos)
        return np.degrees(np.arctan2(q[:, 1] - p[:, 1], q[:, 0] - p[:, 0])) % 360.0


@torch.no_grad()
def goal_field_from_occupancy(occ, mins, zone, cell: float, device="cuda", *, keep_u16=False,
                              max_sweeps: int = MAX_SWEEPS) -> GoalField:
    """The bake of build_goal_field (goalfield.py:222-298) for a given
    occupancy grid ``occ`` [nz, ny, nx] (nonzero = solid, numpy or torch)
    placed at ``mins`` with voxel size ``cell``, toward ``zone``
    ({"mins": [...], "maxs": [...]} map units).

    The returned field holds the dequantised float32 grid (the reference's
    GoalField.grid), or with ``keep_u16`` the uint16 grid plus quant (half the
    memory, the same sampled values). ``field.bake_info`` reports the seed
    count, reach_max, the wavefront's sweeps and tile visits, and
    ``field.grid_q`` the uint16 grid the reference caches (as int16 bits:
    ``field.grid_q.cpu().numpy().view(np.uint16)``).
    """
    lib = _sdfr.load()
    dev = _cuda_device(device)
    o = occ if torch.is_tensor(occ) else torch.from_numpy(np.ascontiguousarray(occ))
    if o.dim() != 3:
        raise ValueError(f"occupancy must be [nz, ny, nx], got shape {tuple(o.shape)}")
    o = (o != 0).to(device=dev, dtype=torch.uint8).contiguous()
    nz, ny, nx = (int(v) for v in o.shape)
    lo, hi = seed_voxel_box(zone, mins, cell, (nx, ny, nz))
    if np.any(hi < lo):
        raise RuntimeError("goal zone contains no free voxel — wrong box?")
    need = int(lib.sdfr_goal_workspace_bytes(nx, ny, nz))
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    grid_q = torch.empty((nz, ny, nx), dtype=torch.int16, device=dev)   # uint16 bits
    grid = None if keep_u16 else torch.empty((nz, ny, nx), dtype=torch.float32, device=dev)
    info = _sdfr.GoalInfo()
    lo_c = (ctypes.c_int32 * 3)(*lo.tolist())
    hi_c = (ctypes.c_int32 * 3)(*hi.tolist())
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.sdfr_goal_bake(o.data_ptr(), nx, ny, nz, float(cell), lo_c, hi_c, int(max_sweeps),
                                grid_q.data_ptr(), grid.data_ptr() if grid is not None else None,
                                ctypes.byref(info), ws.data_ptr(), need, stream)
    del ws
    if rc != 0:
        msg = lib.sdfr_goal_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"goal field bake failed ({rc}): {msg}")
    reach_max = float(info.reach_max)
    if keep_u16:
        field = GoalField(grid_q, mins, cell, reach_max, quant=float(info.quant), device=dev)
    else:
        field = GoalField(grid, mins, cell, reach_max, device=dev)
    field.grid_q = grid_q          # int16 tensor holding the uint16 cache values
    field.bake_info = {"n_seed": int(info.n_seed), "reach_max": reach_max,
                       "sentinel": float(info.sentinel), "quant": float(info.quant),
                       "sweeps": int(info.sweeps), "tile_visits": int(info.tile_visits),
                       "seed_lo": lo.tolist(), "seed_hi": hi.tolist()}
    return field


def _goal_sig(bsp: Path, zone, mask_kill: bool) -> str:
    box = np.round(np.asarray(zone["mins"] + zone["maxs"], np.float64), 1)
    return (f"g{_GOAL_BUILDER_VERSION}_{'k1_' if mask_kill else ''}"
            f"{_map_sig(bsp)}_" + "_".join(f"{v:g}" for v in box))


def goal_occupancy(core, cell: float, cache_dir=None):
    """The goal graph's occupancy: the vision's slab-catching grid
    (goalfield.py:140-145)."""
    return vision.slab_occupancy(core, cell, cache_dir)


def _mask_kill_volumes(occ, mins, cell: float, bsp: Path):
    """Kill volumes as walls of the goal graph only (goalfield.py:188-219):
    the voxel centres inside each kill trigger's hull, classified by the
    package's BSP hull probe (``zones.kill_zones`` / ``zones.hull_probe``),
    become solid. The trigger's box (grown by 1 u) bounds the voxels tested."""
    zones = vision._sibling("zones")
    occ = np.array(occ, copy=True)
    gz, gy, gx = occ.shape
    inside_hull = zones.hull_probe(bsp)
    kills = zones.kill_zones(bsp)
    walled = 0
    for k in kills:
        lo_u = np.asarray(k["mins"], np.float64) - 1.0
        hi_u = np.asarray(k["maxs"], np.float64) + 1.0
        lo = np.maximum(np.floor((lo_u - mins) / cell - 0.5), 0).astype(int)
        hi = np.minimum(np.ceil((hi_u - mins) / cell - 0.5) + 1, [gx, gy, gz]).astype(int)
        if (hi <= lo).any():
            continue
        axes = [mins[a] + (np.arange(lo[a], hi[a]) + 0.5) * cell for a in range(3)]
        zz, yy, xx = np.meshgrid(axes[2], axes[1], axes[0], indexing="ij")
        pts = np.stack([xx.ravel(), yy.ravel(), zz.ravel()], 1)
        hit = inside_hull(int(k["model"][1:]), pts - np.asarray(k["origin"], np.float64))
        if hit.any():
            box = occ[lo[2]:hi[2], lo[1]:hi[1], lo[0]:hi[0]]
            m = np.asarray(hit).reshape(box.shape)
            walled += int((m & (box == 0)).sum())
            box[m] = 1
    print(f"[goalfield] {walled} free voxels inside {len(kills)} kill triggers made solid "
          "for the geodesic")
    return occ


def build_goal_field(core, zone, cell: float, cache_dir=None, device="cuda",
                     mask_kill: bool = False) -> GoalField:
    """Build (or load) the geodesic field toward ``zone`` (goalfield.py:159-298).

    Loads ``<map>.goal[k]_<cell>.npz`` when its signature is current, as the
    reference does. Otherwise bakes on the GPU from :func:`goal_occupancy`
    (with ``mask_kill``, kill volumes walled off first) and writes the goal
    cache in the reference's format.
    """
    bsp = Path(core.bsp_path)
    sig = _goal_sig(bsp, zone, mask_kill)
    cache = Path(cache_dir) if cache_dir else bsp.parent
    cache_file = cache / f"{bsp.stem}.goal{'k' if mask_kill else ''}_{cell:g}.npz"
    if cache_file.exists():
        z = np.load(cache_file, allow_pickle=False)
        if "sig" in z and str(z["sig"]) == sig:
            return GoalField(z["grid"], z["mins"], float(z["cell"]), float(z["reach_max"]),
                             quant=float(z["quant"]), device=device)
    occ, mins = goal_occupancy(core, cell, cache_dir)
    if mask_kill:
        occ = _mask_kill_volumes(occ, np.asarray(mins, np.float64), cell, bsp)
    field = goal_field_from_occupancy(occ, mins, zone, cell, device=device)
    info = field.bake_info
    print(f"[goalfield] GPU bake: {info['n_seed']} seed voxels, {info['sweeps']} wavefront "
          f"sweeps, farthest reachable voxel {field.reach_max:.0f} u")
    q = field.grid_q.cpu().numpy().view(np.uint16)
    np.savez_compressed(cache_file, grid=q, quant=np.float32(info["quant"]),
                        mins=mins, cell=np.float32(cell),
                        reach_max=np.float32(field.reach_max), sig=np.str_(sig))
    return field
