"""GPU lidar: batched depth images by sphere tracing a voxel SDF on MI355X.

Drop-in for the reference's ``surfgym.vision`` render path
(python/surfgym/vision.py): ``GpuLidar`` keeps the constructor, ``render``
signature and output contract (vision.py:457-462, :542-550), and
``grid_dims``/``pick_cell``/``build_sdf`` keep their meaning, so the
trainer's rollout loop (train_fast.py:1744-1765) calls it unchanged. The
render runs in libsdfr.so (hand-written HIP for gfx950, include/sdfr.h),
enqueued on the current torch stream with no host synchronisation.

Camera convention (src/surfcore.h:20-34): row 0 looks up (+vfov/2), column 0
looks left (+hfov/2), positive pitch is up, eye height 17 standing / 12
ducked. Output values: near-linear ``min(t,near)/near`` plus a bounded far
tail ``0.25*(1-exp(-(t-near)/2500))``; near == range is the legacy
``t/range`` clamped to 1 (vision.py:112-116, :468-472).

There is deliberately no CPU render: ``device`` must be a ROCm GPU, and a
missing native library is an error, not a fallback.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import torch

from . import _sdfr

__all__ = ["GpuLidar", "build_sdf", "sdf_from_occupancy", "map_occupancy", "slab_occupancy",
           "pick_cell", "grid_dims", "SOLID_ENT_CLASSES"]

# brush entities the reference's physics collides with (vision.py:301-307);
# thin ones are rasterised into the slab occupancy, and the surfability bake
# imports the name
SOLID_ENT_CLASSES = {"func_wall", "func_breakable", "func_pushable",
                     "func_button", "func_train", "func_conveyor",
                     "func_wall_toggle", "func_rotating",
                     "func_door_rotating", "func_door"}

_SDF_BUILDER_VERSION = 2
_SDF_SEMANTICS = "s4"
_OCC_SEMANTICS = "o2"

_DUCK_DTYPES = {torch.float32: _sdfr.F32, torch.float16: _sdfr.F16, torch.bfloat16: _sdfr.BF16,
                torch.int32: _sdfr.I32, torch.int64: _sdfr.I64, torch.uint8: _sdfr.U8,
                torch.bool: _sdfr.U8, torch.float64: _sdfr.F64}
# voxel storage of the device copy: a torch dtype, or "r16" (4x4x4 bricks of
# uint16 codes against a per-brick fp32 base and power-of-two scale)
_GRID_DTYPES = {torch.float32: _sdfr.F32, torch.float16: _sdfr.F16, "r16": _sdfr.R16}
_OUT_DTYPES = {torch.float32: _sdfr.F32, torch.bfloat16: _sdfr.BF16}
_LAYOUTS = {"linear": _sdfr.LAYOUT_LINEAR, "brick4": _sdfr.LAYOUT_BRICK4}
_SCHEDULES = {"persistent": _sdfr.SCHED_PERSISTENT, "tiles": _sdfr.SCHED_TILES}
_TILE_ORDERS = {"launch": _sdfr.ORDER_LAUNCH, "lookahead": _sdfr.ORDER_LOOKAHEAD}
_BORDER_FACES = {"auto": _sdfr.FACES_AUTO, "on": _sdfr.FACES_ON, "off": _sdfr.FACES_OFF}


# The grid geometry is computed in the dtype the map core returns its bounds
# in (float32 from the C core, core.py:869-878), as the reference computes it;
# widening the bounds first would move mins, and every origin handed back to
# the core's occupancy sampling, by up to half a float32 ulp.
def _bounds(core):
    mn, mx = core.map_bounds()
    return np.asarray(mn), np.asarray(mx)


def pick_cell(core, budget_voxels: float = 700e6) -> float:
    """Smallest power-of-two voxel size from 16 u whose padded grid fits the
    voxel budget (the reference's rule, vision.py:283-298): per axis the
    padded extent over the cell, rounded up, multiplied axis by axis from
    1.0 — all in the bounds' dtype, as there."""
    mn, mx = _bounds(core)
    cell = 16.0
    while cell < 256.0:
        voxels = 1.0
        for n_axis in np.ceil(((mx - mn) + 2.0 * (4.0 * cell)) / cell):
            voxels *= n_axis
        if voxels <= budget_voxels:
            break
        cell *= 2.0
    return cell


def grid_dims(core, cell: float):
    """(mins float64 (3,), nx, ny, nz): the map bounds padded by 4 cells and
    cut into whole voxels (vision.py:310-322). The padded minimum is taken in
    the bounds' dtype and then widened to float64; the far side is padded in
    the bounds' dtype too and measured from that float64 minimum."""
    mn, mx = _bounds(core)
    pad = 4.0 * cell
    mins = (mn - pad).astype(np.float64)
    nx, ny, nz = (int(np.ceil(e / cell)) for e in (mx + pad) - mins)
    return mins, nx, ny, nz


def _map_sig(bsp: Path) -> str:
    """The map part of every cache signature (vision.py:275-280)."""
    st = bsp.stat()
    return f"v{_SDF_BUILDER_VERSION}_{st.st_size}_{st.st_mtime_ns}"


def _cached(path: Path, sig: str, keys):
    """The arrays `keys` of the cache file `path` if it exists and carries
    signature `sig`, else None (the reference's cache test, vision.py:334-338)."""
    if path.exists():
        z = np.load(path, allow_pickle=False)
        if "sig" in z and str(z["sig"]) == sig:
            return tuple(z[k] for k in keys)
    return None


def _cache_file(core, cell, cache_dir, kind: str) -> Path:
    bsp = Path(core.bsp_path)
    cache = Path(cache_dir) if cache_dir else bsp.parent
    return cache / f"{bsp.stem}.{kind}_{cell:g}.npz"


def _sibling(name: str):
    """A module of the package this one is loaded in: the reference's own
    ``surfgym.<name>`` when this module is installed into the reference's
    package (surfgym_mi355x.install)."""
    import importlib
    try:
        return importlib.import_module(f"{__package__}.{name}")
    except ImportError as e:
        raise ImportError(
            f"{__package__}.{name} is needed to sample a map (it parses the BSP); install this "
            "renderer into the reference's surfgym package (surfgym_mi355x.install) or bake "
            "the map's caches with the reference") from e


def map_occupancy(core, cell: float = 16.0, cache_dir=None):
    """The map's voxel-centre solid occupancy, (occ uint8 [nz, ny, nx],
    mins float64 (3,)), cached as ``<map>.occ_<cell>.npz`` (vision.py:325-343).
    On a miss the map core samples it on grid_dims' voxels
    (``core.occupancy_grid``, the C core's surf_occupancy_grid)."""
    bsp = Path(core.bsp_path)
    sig = f"{_map_sig(bsp)}_{_OCC_SEMANTICS}"
    path = _cache_file(core, cell, cache_dir, "occ")
    hit = _cached(path, sig, ("occ", "mins"))
    if hit is not None:
        return hit[0], hit[1].astype(np.float64)
    mins, nx, ny, nz = grid_dims(core, cell)
    occ = core.occupancy_grid(mins, cell, nx, ny, nz)
    np.savez_compressed(path, occ=occ, mins=mins, sig=np.str_(sig))
    return occ, mins


# Thin solid brushes the slab occupancy rasterises exactly: a bounding box
# whose smallest side is at most this many units (vision.py:392-395).
_THIN_UNITS = 20.0


def slab_occupancy(core, cell: float = 16.0, cache_dir=None):
    """Occupancy that thin solids cannot slip through, cached as
    ``<map>.slabocc_<cell>.npz`` (vision.py:346-406): the voxel-centre
    occupancy ORed with twelve samplings whose origin is shifted by
    +-cell/4 and +-cell/2 along each axis, plus the bounding boxes of thin
    solid brush entities (smallest side <= 20 u; not-solid conveyors
    skipped) rasterised outright. On a miss the map core does the sampling
    and the package's BSP parser (``zones.parse_bsp``) lists the entities."""
    bsp = Path(core.bsp_path)
    sig = f"{_map_sig(bsp)}_{_SDF_SEMANTICS}"
    path = _cache_file(core, cell, cache_dir, "slabocc")
    hit = _cached(path, sig, ("occ", "mins"))
    if hit is not None:
        return hit[0], hit[1].astype(np.float64)
    base, mins = map_occupancy(core, cell, cache_dir)
    occ = np.array(base, copy=True)
    nz, ny, nx = occ.shape
    quarter = cell / 4.0
    for axis in range(3):
        for k in (-2, -1, 1, 2):
            shift = np.zeros(3)
            shift[axis] = k * quarter
            occ |= core.occupancy_grid(mins + shift, cell, nx, ny, nz)
    entities, bboxes = _sibling("zones").parse_bsp(bsp)
    dims = np.array([nx, ny, nz])
    n_thin = 0
    for ent in entities:
        cls, model = ent.get("classname"), ent.get("model", "")
        if cls not in SOLID_ENT_CLASSES or not model.startswith("*"):
            continue
        if cls == "func_conveyor" and int(float(ent.get("spawnflags", 0))) & 2:
            continue   # a not-solid conveyor (the core's solid set skips it)
        k = int(model[1:])
        if k >= len(bboxes):
            continue
        lo_u, hi_u = (np.asarray(v, np.float64) for v in bboxes[k])
        if float((hi_u - lo_u).min()) > _THIN_UNITS:
            continue
        lo = np.maximum(np.floor((lo_u - mins) / cell - 0.001), 0).astype(int)
        hi = np.minimum(np.ceil((hi_u - mins) / cell + 0.001), dims).astype(int)
        occ[lo[2]:hi[2], lo[1]:hi[1], lo[0]:hi[0]] = 1
        n_thin += 1
    if n_thin:
        print(f"[vision] {n_thin} thin solid brushes filled into the slab occupancy")
    np.savez_compressed(path, occ=occ, mins=mins, sig=np.str_(sig))
    return occ, mins


def build_sdf(core, cell: float = 16.0, cache_dir=None, device=None):
    """The map's distance field: (sdf [nz,ny,nx], mins (3,) f32, cell).

    Loads ``<map>.sdf_<cell>.npz`` (keys sdf, mins, cell, sig) when its
    signature is current (vision.py:409-426), so a bake the reference wrote is
    used as-is. Otherwise bakes it on the GPU (vision.py:428-439): the slab
    occupancy, padded with one layer of solid, through the exact distance
    transform of :func:`sdf_from_occupancy` (bit for bit the reference's scipy
    call for power-of-two cells), stored f16 above 100 M voxels, else f32,
    and writes the cache file in the reference's format. ``device``: the GPU
    of the bake (default: the current one). Tests replace this function on
    the module, as the reference's do.
    """
    bsp = Path(core.bsp_path)
    sig = f"{_map_sig(bsp)}_{_SDF_SEMANTICS}"
    path = _cache_file(core, cell, cache_dir, "sdf")
    hit = _cached(path, sig, ("sdf", "mins", "cell"))
    if hit is not None:
        return hit[0], hit[1], float(hit[2])
    occ, mins = slab_occupancy(core, cell, cache_dir)
    if device is None:
        device = torch.device("cuda", torch.cuda.current_device())
    sdf = sdf_from_occupancy(occ, cell, device=device).cpu().numpy()
    mins32 = np.asarray(mins).astype(np.float32)
    np.savez_compressed(path, sdf=sdf, mins=mins32, cell=np.float32(cell), sig=np.str_(sig))
    return sdf, mins32, cell


@torch.no_grad()
def sdf_from_occupancy(occ, cell: float, device="cuda", dtype=None) -> torch.Tensor:
    """The SDF bake on the GPU: exact Euclidean distance (map units) from
    every voxel centre to the nearest solid voxel centre, the grid padded with
    one layer of solid — what build_sdf computes with
    ``scipy.ndimage.distance_transform_edt`` (vision.py:428-438), bit for bit
    for power-of-two cells.

    ``occ``: [nz, ny, nx] solid occupancy (nonzero = solid), numpy or torch.
    ``dtype``: torch.float32 / torch.float16; None picks the reference's rule
    (float16 above 100 M voxels, vision.py:436-437). Returns a device tensor.
    """
    lib = _sdfr.load()
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("the SDF bake runs on a ROCm GPU")
    o = torch.as_tensor(np.asarray(occ) if not torch.is_tensor(occ) else occ)
    if o.dim() != 3:
        raise ValueError(f"occupancy must be [nz, ny, nx], got shape {tuple(o.shape)}")
    o = (o != 0).to(device=device, dtype=torch.uint8).contiguous()
    nz, ny, nx = (int(v) for v in o.shape)
    if dtype is None:
        dtype = torch.float16 if o.numel() > 100e6 else torch.float32
    if dtype not in (torch.float32, torch.float16):
        raise ValueError("dtype must be torch.float32 or torch.float16")
    need = int(lib.sdfr_edt_workspace_bytes(nx, ny, nz))
    ws = torch.empty(need, dtype=torch.uint8, device=device)
    out = torch.empty(nz, ny, nx, dtype=dtype, device=device)
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        rc = lib.sdfr_edt(o.data_ptr(), nx, ny, nz, float(cell), out.data_ptr(),
                          _sdfr.F32 if dtype == torch.float32 else _sdfr.F16, ws.data_ptr(),
                          need, stream)
    if rc != 0:
        raise _sdfr.SdfrError(f"sdfr_edt failed ({rc}): "
                              f"{lib.sdfr_edt_last_error().decode('utf-8', 'replace')}")
    return out


def _ducked_code(t: torch.Tensor) -> int:
    return _DUCK_DTYPES.get(t.dtype, -1)


# The current stream's raw handle for a device index: torch's own accessor
# (what torch.cuda.current_stream(...).cuda_stream reads, without building a
# Stream object per call), else the public route.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _current_stream(device: torch.device) -> int:
    if _raw_stream is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


class GpuLidar:
    """Batched depth-image renderer over a voxel SDF.

    ``render(origin, yaw_deg, pitch_deg, ducked) -> (N, H, W) float32`` on
    the lidar's device; values = hit distance / range, 1.0 = clear (plus the
    far tail when ``near_range`` < range).

    Keyword-only extensions (defaults reproduce the reference):

    * ``grid_dtype`` — voxel storage, torch.float16 as the reference stores
      it (vision.py:476-477), torch.float32, or ``"r16"``: 4x4x4 bricks of
      uint16 codes against a per-brick fp32 base and power-of-two scale,
      two bytes per voxel like fp16 but within scale/2 of the fp32 grid
      (2^-10 u at 16 u cells) at any distance;
    * ``layout`` — the device copy's order, "brick4" (4x4x4 bricks) or
      "linear";
    * ``hit_eps`` / ``min_step`` — the step rule's constants, 0.6*cell and
      0.3*cell by default (vision.py:87-88);
    * ``schedule`` / ``refill_lanes`` / ``rays_per_lane`` — how the kernel
      schedules rays: launch-scheduled waves of 16x4 pixel "tiles", each lane
      marching ``rays_per_lane`` rays at once (default None: each render
      picks 1 for grids above 192 MiB and for renders under 512 envs of
      128x64, else 2; see :meth:`effective_rays_per_lane`); or "persistent"
      waves that refill lanes with new rays once ``refill_lanes`` of them
      have finished. The results are identical;
    * ``tile_order`` — "lookahead" (default) or "launch": see
      :meth:`set_tile_order`.
    """

    def __init__(self, core, width: int = 128, height: int = 64,
                 hfov_deg: float = 120.0, vfov_deg: float = 90.0,
                 range_units: float = 2000.0, cell: float = 16.0,
                 max_steps: int = 64, near_range: float = None,
                 device="cuda", surf_mask: bool = False,
                 pinhole: bool = False, *, grid_dtype=torch.float16,
                 layout: str = "brick4", hit_eps: float = None,
                 min_step: float = None, schedule: str = "tiles",
                 refill_lanes: int = 16, rays_per_lane: int | None = None,
                 tile_order: str = "lookahead", _grid=None,
                 _surf_nz=None) -> None:
        if surf_mask and pinhole:
            raise ValueError(
                "pinhole=True with surf_mask=True: the surf-mask channel is rendered for the "
                "equiangular camera only; there is no combined kernel")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError(f"GpuLidar renders on a ROCm GPU (device='cuda'), got {device!r}; "
                             "this renderer has no CPU path")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        if grid_dtype not in _GRID_DTYPES:
            raise ValueError(f"grid_dtype must be torch.float16, torch.float32 or 'r16', "
                             f"got {grid_dtype!r}")
        if grid_dtype == "r16" and layout != "brick4":
            raise ValueError("the r16 store exists in the brick4 layout only")
        if layout not in _LAYOUTS:
            raise ValueError(f"layout must be one of {sorted(_LAYOUTS)}, got {layout!r}")
        if schedule not in _SCHEDULES:
            raise ValueError(f"schedule must be one of {sorted(_SCHEDULES)}, got {schedule!r}")
        self._lib = _sdfr.load()
        sdf, mins, cell = _grid if _grid is not None else build_sdf(core, cell)
        sdf = np.asarray(sdf)
        if sdf.ndim != 3:
            raise ValueError(f"the grid must be [nz, ny, nx], got shape {sdf.shape}")
        # the flat device grid the handle's copy is made from (an r16 copy is
        # encoded from the fp32 values); the handle keeps only its own
        # re-laid-out copy, and sdf_flat reads the stored values back on demand
        flat_dtype = torch.float32 if grid_dtype == "r16" else grid_dtype
        flat = torch.as_tensor(sdf, device=self.device).to(flat_dtype).reshape(-1)
        self.nz, self.ny, self.nx = (int(v) for v in sdf.shape)
        self.stride_z = self.ny * self.nx
        self.stride_y = self.nx
        mins = np.asarray(mins, np.float32).reshape(3)
        self.mins = torch.as_tensor(mins, device=self.device)
        self.mins_f = (float(mins[0]), float(mins[1]), float(mins[2]))
        self.cell = float(cell)
        # second channel: |n_z| of the hit surface (vision.py:482-497), on
        # exactly the SDF's voxels; nothing is allocated for it when off
        self.surf_mask = bool(surf_mask)
        self.channels = 2 if self.surf_mask else 1
        snz = None
        if self.surf_mask:
            if _surf_nz is not None:
                snz = np.asarray(_surf_nz)
            else:
                from . import surfmask
                snz, _ = surfmask.build_surfnz(core, cell)
                snz = np.asarray(snz)
            if snz.shape != sdf.shape:
                raise RuntimeError(
                    f"surf-mask grid {snz.shape} does not match the distance grid {sdf.shape}; "
                    "a single voxel index addresses both")
            self.snz_flat = torch.as_tensor(snz.astype(np.int8, copy=False),
                                            device=self.device).reshape(-1)
        self.W, self.H = int(width), int(height)
        self.range = float(range_units)
        self.near = float(near_range) if near_range else self.range
        self.max_steps = int(max_steps)
        self.hfov_deg, self.vfov_deg = float(hfov_deg), float(vfov_deg)
        # the march compares in fp32 (vision.py:87-88, 637-638)
        self.hit_eps = float(np.float32(0.6 * self.cell if hit_eps is None else hit_eps))
        self.min_step = float(np.float32(0.3 * self.cell if min_step is None else min_step))
        d2r = np.pi / 180.0
        # per-pixel angular offsets (surfcore.h convention); the kernel derives
        # the same float64-then-fp32 values in registers, these are for callers
        yoff = (self.hfov_deg * (0.5 - (np.arange(self.W) + 0.5) / self.W)) * d2r
        poff = (self.vfov_deg * (0.5 - (np.arange(self.H) + 0.5) / self.H)) * d2r
        self.yoff = torch.as_tensor(yoff, dtype=torch.float32, device=self.device)
        self.poff = torch.as_tensor(poff, dtype=torch.float32, device=self.device)
        self.pinhole = bool(pinhole)
        self._tan_h = float(np.tan(0.5 * self.hfov_deg * d2r))
        self._tan_v = float(np.tan(0.5 * self.vfov_deg * d2r))
        if self.pinhole:
            uo = self._tan_h * (2.0 * np.arange(self.W) / max(self.W - 1, 1) - 1.0)
            vo = self._tan_v * (1.0 - 2.0 * np.arange(self.H) / max(self.H - 1, 1))
            if self.W == 1:
                uo[:] = 0.0
            if self.H == 1:
                vo[:] = 0.0
            self.uoff = torch.as_tensor(uo, dtype=torch.float32, device=self.device)
            self.voff = torch.as_tensor(vo, dtype=torch.float32, device=self.device)
        self.layout = layout
        self.grid_dtype = grid_dtype
        desc = _sdfr.GridDesc(self.nx, self.ny, self.nz, (ctypes.c_float * 3)(*mins),
                              self.cell)
        err = ctypes.create_string_buffer(512)
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device)
            h = self._lib.sdfr_grid_create(ctypes.byref(desc), flat.data_ptr(),
                                           _GRID_DTYPES[flat_dtype], 1, _GRID_DTYPES[grid_dtype],
                                           _LAYOUTS[layout], stream.cuda_stream, err, len(err))
        # sdfr_grid_create has finished reading it when it returns (it waits
        # for its stream), so the flat grid can go back to torch's pool
        del flat
        if not h:
            raise _sdfr.SdfrError(err.value.decode("utf-8", "replace"))
        self._grid = h
        self._ws_retired = []   # workspaces captured renders still point at
        if self.surf_mask:
            with torch.cuda.device(self.device):
                stream = torch.cuda.current_stream(self.device).cuda_stream
                rc = self._lib.sdfr_grid_attach_surfnz(h, self.snz_flat.data_ptr(), 1, stream)
            _sdfr.check(rc, "sdfr_grid_attach_surfnz", self._lib)
        self.set_schedule(schedule, refill_lanes, rays_per_lane)
        self.set_tile_order(tile_order)
        self.border_faces = "auto"   # see set_border_faces

    def set_schedule(self, schedule: str = "tiles", refill_lanes: int = 16,
                     rays_per_lane: int | None = None) -> None:
        """Switch the ray schedule of later renders (results are unchanged).
        ``rays_per_lane=None`` lets each render choose (the library's
        default: 1 for grids above 192 MiB and for renders of fewer than
        65536 16x4 tiles, else 2); ``rays_per_lane`` then reads None."""
        if schedule not in _SCHEDULES:
            raise ValueError(f"schedule must be one of {sorted(_SCHEDULES)}, got {schedule!r}")
        rpl = 0 if rays_per_lane is None else int(rays_per_lane)
        _sdfr.check(self._lib.sdfr_grid_set_schedule(self._grid, _SCHEDULES[schedule],
                                                     int(refill_lanes), rpl),
                    "sdfr_grid_set_schedule", self._lib)
        self.schedule, self.refill_lanes = schedule, int(refill_lanes)
        self.rays_per_lane = None if rays_per_lane is None else rpl

    def effective_rays_per_lane(self, n_envs: int) -> int:
        """Rays per lane a render of ``n_envs`` images runs with (tiles
        schedule and surf-mask renders)."""
        r = int(self._lib.sdfr_render_rays_per_lane(self._grid, ctypes.byref(self._cam()),
                                                    int(n_envs)))
        if r < 0:
            _sdfr.check(r, "sdfr_render_rays_per_lane", self._lib)
        return r

    def set_tile_order(self, order: str = "lookahead", min_tiles: int | None = None) -> None:
        """The order the tiles schedule takes 16x4 pixel tiles in: "launch"
        (env by env) or "lookahead" (sorted by where each tile's centre ray
        is 1.2 x near units out, so each XCD's cache serves one part of the
        map). The sort costs two small launches, so "lookahead" applies to
        renders of at least ``min_tiles`` tiles (None: the library's
        default, 65536 = 512 envs of 128x64; 0: always). Results are
        unchanged."""
        if order not in _TILE_ORDERS:
            raise ValueError(f"tile_order must be one of {sorted(_TILE_ORDERS)}, got {order!r}")
        mt = -1 if min_tiles is None else int(min_tiles)
        if min_tiles is not None and mt < 0:
            raise ValueError(f"min_tiles must be >= 0, got {min_tiles}")
        _sdfr.check(self._lib.sdfr_grid_set_tile_order(self._grid, _TILE_ORDERS[order], mt),
                    "sdfr_grid_set_tile_order", self._lib)
        self.tile_order = order

    def set_border_faces(self, mode: str = "auto") -> None:
        """When the one-ray-per-lane march reads border voxels (every
        sample outside the grid clamps to one, vision.py:104-106) from the
        grid's 2D face copies instead of its bricks: "auto" (the default: on
        grids beyond the Infinity Cache, above 192 MiB, in renders of at
        least 128 envs of 128x64; smaller renders are latency-bound and the
        lookup lengthens every step), "on" or "off". The
        copies exist for fp32 and fp16 bricks; they hold the bricks'
        values, so results are unchanged."""
        if mode not in _BORDER_FACES:
            raise ValueError(f"border faces must be one of {sorted(_BORDER_FACES)}, got {mode!r}")
        _sdfr.check(self._lib.sdfr_grid_set_border_faces(self._grid, _BORDER_FACES[mode]),
                    "sdfr_grid_set_border_faces", self._lib)
        self.border_faces = mode

    def set_march_events(self, start: int | None, stop: int | None) -> None:
        """Measurement hook: raw hipEvent_t handles (ints) that every later
        render records right before and right after its march kernel, on its
        stream; None, None clears them. The caller owns the events."""
        _sdfr.check(self._lib.sdfr_grid_set_march_events(self._grid, start, stop),
                    "sdfr_grid_set_march_events", self._lib)

    @classmethod
    def from_grid(cls, sdf, mins, cell, surf_nz=None, **kwargs) -> "GpuLidar":
        """A lidar over an explicit [nz,ny,nx] distance grid (no map core);
        ``surf_nz`` (int8 |n_z|*127 on the same grid) enables the second
        channel."""
        kwargs = dict(kwargs)
        kwargs["cell"] = float(cell)
        if surf_nz is not None:
            kwargs["surf_mask"] = True
        return cls(None, _grid=(sdf, mins, float(cell)), _surf_nz=surf_nz, **kwargs)

    def __del__(self):
        h = getattr(self, "_grid", None)
        if h:
            self._grid = None
            try:
                torch.cuda.synchronize(self.device)
            except Exception:
                pass
            self._lib.sdfr_grid_destroy(h)

    # ------------------------------------------------------------------ args --
    def _workspace(self, cam, n: int) -> torch.Tensor:
        """The render's ray-table scratch, kept and grown with N. It is
        allocated outside the render call, so a render captured into a graph
        after one eager render of the same N allocates nothing. A buffer that
        a captured render has used stays alive for the lidar's lifetime when
        a larger render replaces it: the graph replays write to its address."""
        need = self._ws_need.get(n)
        if need is None:
            need = int(self._lib.sdfr_workspace_bytes(ctypes.byref(cam), n))
            if need < 0:
                _sdfr.check(need, "sdfr_workspace_bytes", self._lib)
            self._ws_need[n] = need
        ws = getattr(self, "_ws", None)
        if ws is None or ws.numel() < need:
            if ws is not None and getattr(self, "_ws_captured", False):
                self._ws_retired.append(ws)
            ws = torch.empty(need, dtype=torch.uint8, device=self.device)
            self._ws = ws
            self._ws_captured = False
        if not self._ws_captured and torch.cuda.is_current_stream_capturing():
            self._ws_captured = True
        return ws

    def _cam(self) -> _sdfr.Cam:
        """The sensor as the C ABI takes it, rebuilt only when an attribute
        it is made of has changed since the last render (callers may set
        range, near, max_steps and the like between renders)."""
        key = (self.W, self.H, self.hfov_deg, self.vfov_deg, self._tan_h, self._tan_v,
               self.range, self.near, self.hit_eps, self.min_step, self.max_steps, self.pinhole)
        if key != getattr(self, "_cam_key", None):
            self._cam_obj = _sdfr.Cam(*key[:-1], _sdfr.CAM_PINHOLE if key[-1] else _sdfr.CAM_EQUIANGULAR)
            self._cam_key = key
            self._ws_need = {}   # workspace bytes per N, for this sensor
        return self._cam_obj

    def _f32(self, t, name):
        t = torch.as_tensor(t)
        if t.device != self.device or t.dtype != torch.float32:
            t = t.to(self.device, torch.float32)
        return t

    def _poses(self, origin, yaw_deg, pitch_deg, ducked):
        dev = self.device
        if not (isinstance(origin, torch.Tensor) and origin.dtype == torch.float32
                and origin.device == dev):
            origin = self._f32(origin, "origin")
        if origin.dim() != 2 or origin.shape[1] != 3:
            raise ValueError(f"origin must be (N, 3), got {tuple(origin.shape)}")
        if origin.stride(1) != 1:
            origin = origin.contiguous()
        n = origin.shape[0]
        if n < 1:
            raise ValueError("render needs at least one env")
        yaw, pitch = yaw_deg, pitch_deg
        if not (isinstance(yaw, torch.Tensor) and yaw.dtype == torch.float32 and yaw.device == dev):
            yaw = self._f32(yaw, "yaw_deg")
        if not (isinstance(pitch, torch.Tensor) and pitch.dtype == torch.float32
                and pitch.device == dev):
            pitch = self._f32(pitch, "pitch_deg")
        if yaw.dim() != 1:
            yaw = yaw.reshape(-1)
        if pitch.dim() != 1:
            pitch = pitch.reshape(-1)
        if not (isinstance(ducked, torch.Tensor) and ducked.device == dev):
            ducked = torch.as_tensor(ducked).to(dev)
        if ducked.dim() != 1:
            ducked = ducked.reshape(-1)
        if _ducked_code(ducked) < 0:
            ducked = ducked.to(torch.int32)
        for name, t in (("yaw_deg", yaw), ("pitch_deg", pitch), ("ducked", ducked)):
            if t.shape[0] != n:
                raise ValueError(f"{name} has {t.shape[0]} entries for {n} envs")
        p = _sdfr.Poses(origin.data_ptr(), origin.stride(0), yaw.data_ptr(), yaw.stride(0),
                        pitch.data_ptr(), pitch.stride(0), ducked.data_ptr(), ducked.stride(0),
                        _ducked_code(ducked), n)
        return p, (origin, yaw, pitch, ducked)

    def _check_out(self, out: torch.Tensor, n: int) -> int:
        key = (out.shape, out.stride(), out.dtype, out.device, n, self.H, self.W, self.channels)
        if key == getattr(self, "_out_key", None):
            return self._out_stride
        stride = self._check_out_layout(out, n)
        self._out_key, self._out_stride = key, stride
        return stride

    def _check_out_layout(self, out: torch.Tensor, n: int) -> int:
        if out.device != self.device or out.dtype not in _OUT_DTYPES:
            raise ValueError("out must be a float32 or bfloat16 tensor on the lidar's device")
        per_env = self.H * self.W * self.channels
        if out.shape[0] != n or out[0].numel() != per_env:
            raise ValueError(f"out must hold N={n} images of {self.H}x{self.W}x{self.channels}, "
                             f"got {tuple(out.shape)}")
        # each env's image must be one dense row-major HxW block
        inner = out[0]
        expect = 1
        for size, stride in reversed(list(zip(inner.shape, inner.stride()))):
            if size != 1 and stride != expect:
                raise ValueError("each env's image in out must be contiguous")
            expect *= size
        return out.stride(0) if n > 1 else per_env

    # ---------------------------------------------------------------- render --
    # (no autograd context: the inputs are read by pointer and the output is
    # a fresh tensor without a graph either way)
    def render(self, origin, yaw_deg, pitch_deg, ducked, out=None, taps=None):
        """origin (N,3), yaw/pitch (N,) degrees, ducked (N,) bool/int/float ->
        (N, H, W) float32 depth encodings, or (N, H, W, 2) (depth, |n_z|)
        channel-fastest with the surf mask (vision.py:542-550).

        Inputs may be strided views (the trainer passes columns of its (N,6)
        pose tensor). ``out`` optionally names the destination — any float32
        or bfloat16 tensor whose dim 0 is N and whose per-env block is a dense
        HxW image (e.g. the image columns of an observation row); it is
        returned. ``taps`` optionally receives the grid loads each ray issued
        ((N,H,W) int32), for measurement."""
        poses, keep = self._poses(origin, yaw_deg, pitch_deg, ducked)
        n = poses.n_envs
        if out is None:
            shape = (n, self.H, self.W, 2) if self.surf_mask else (n, self.H, self.W)
            out = torch.empty(shape, device=self.device)
        env_stride = self._check_out(out, n)
        taps_ptr = None
        if taps is not None:
            if (taps.device != self.device or taps.dtype != torch.int32 or not taps.is_contiguous()
                    or taps.numel() != n * self.H * self.W):
                raise ValueError("taps must be a contiguous int32 (N,H,W) tensor on the device")
            taps_ptr = taps.data_ptr()
        img = _sdfr.Image(out.data_ptr(), env_stride, _OUT_DTYPES[out.dtype], self.channels,
                          taps_ptr)
        cam = self._cam()
        ws = self._workspace(cam, n)
        if torch.cuda.current_device() == self.device.index:
            rc = self._lib.sdfr_render(self._grid, ctypes.byref(cam), ctypes.byref(poses),
                                       ctypes.byref(img), ws.data_ptr(), ws.numel(),
                                       _current_stream(self.device))
        else:
            with torch.cuda.device(self.device):
                rc = self._lib.sdfr_render(self._grid, ctypes.byref(cam), ctypes.byref(poses),
                                           ctypes.byref(img), ws.data_ptr(), ws.numel(),
                                           _current_stream(self.device))
        if rc != 0:
            _sdfr.check(rc, "sdfr_render", self._lib)
        del keep
        return out

    @torch.no_grad()
    def ray_dirs(self, yaw_deg, pitch_deg, *, pinhole: bool | None = None) -> torch.Tensor:
        """(N, H, W, 3) unit ray directions exactly as the march casts them
        (``pinhole`` overrides the lidar's camera model)."""
        yaw = self._f32(yaw_deg, "yaw_deg").reshape(-1)
        pitch = self._f32(pitch_deg, "pitch_deg").reshape(-1)
        n = yaw.shape[0]
        zeros = torch.zeros(n, 3, device=self.device)
        duck = torch.zeros(n, dtype=torch.int32, device=self.device)
        poses, keep = self._poses(zeros, yaw, pitch, duck)
        out = torch.empty(n, self.H, self.W, 3, device=self.device)
        cam = _sdfr.Cam.from_buffer_copy(self._cam())
        if pinhole is not None:
            cam.camera = _sdfr.CAM_PINHOLE if pinhole else _sdfr.CAM_EQUIANGULAR
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            rc = self._lib.sdfr_ray_dirs(ctypes.byref(cam), ctypes.byref(poses), out.data_ptr(),
                                         stream)
        _sdfr.check(rc, "sdfr_ray_dirs", self._lib)
        del keep
        return out

    # The reference's CPU path keeps ray directions in (N, H, W) buffers that
    # its camera tests read (vision.py:531-540, :596-624; test_pinhole.py:
    # 36-41). The same names here fill device buffers from the kernel's own
    # ray setup.
    def _ensure_buffers(self, N):
        if getattr(self, "_buf_n", None) == N:
            return
        self._buf_n = N
        sh = (N, self.H, self.W)
        self._dx = torch.empty(sh, device=self.device)
        self._dy = torch.empty(sh, device=self.device)
        self._dz = torch.empty(sh, device=self.device)

    def _dirs_into(self, N, yaw_deg, pitch_deg, d2r, pinhole):
        if np.float32(d2r) != np.float32(np.pi / 180.0):
            raise ValueError("the kernel converts degrees with f32(pi/180); d2r must be pi/180")
        self._ensure_buffers(N)
        d = self.ray_dirs(torch.as_tensor(yaw_deg).reshape(N), torch.as_tensor(pitch_deg).reshape(N),
                          pinhole=pinhole)
        self._dx.copy_(d[..., 0])
        self._dy.copy_(d[..., 1])
        self._dz.copy_(d[..., 2])

    def _dirs_equiangular(self, N, yaw_deg, pitch_deg, d2r):
        """Equiangular directions into ``_dx/_dy/_dz`` (vision.py:596-607)."""
        self._dirs_into(N, yaw_deg, pitch_deg, d2r, False)

    def _dirs_pinhole(self, N, yaw_deg, pitch_deg, d2r):
        """Tangent-plane directions into ``_dx/_dy/_dz`` (vision.py:609-624)."""
        self._dirs_into(N, yaw_deg, pitch_deg, d2r, True)

    @property
    def sdf_flat(self) -> torch.Tensor:
        """The reference's flat device grid (vision.py:476-480): the values
        the march samples, [nz*ny*nx] in the store's dtype (fp32 holding the
        decoded values for r16). It is read back from the handle's copy on
        first access and kept; a lidar nobody asks holds only that copy."""
        t = self.__dict__.get("_sdf_flat")
        if t is None:
            dt = torch.float32 if self.grid_dtype == "r16" else self.grid_dtype
            t = self.stored_grid().to(dt).reshape(-1)
            self._sdf_flat = t
        return t

    @torch.no_grad()
    def stored_grid(self) -> torch.Tensor:
        """The device copy the march samples, read back as [nz, ny, nx]
        float32 (fp16 widened, r16 decoded)."""
        out = torch.empty(self.nz, self.ny, self.nx, device=self.device)
        with torch.cuda.device(self.device):
            rc = self._lib.sdfr_grid_read(self._grid, out.data_ptr(),
                                          torch.cuda.current_stream(self.device).cuda_stream)
        _sdfr.check(rc, "sdfr_grid_read", self._lib)
        return out

    @property
    def grid_bytes(self) -> int:
        """Device bytes of the re-laid-out grid the kernel reads."""
        return int(self._lib.sdfr_grid_bytes(self._grid))
