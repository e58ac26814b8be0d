"""ctypes binding of libsdfr.so (include/sdfr.h).

Written the way the reference binds its C core (python/surfgym/core.py:1-19,
:444-448): explicit argtypes for every entry point and a refusal to run
against a library whose ABI version differs from the one this file mirrors.

torch is imported before the library is opened so that the HIP runtime torch
already loaded is the one libsdfr.so binds to: device pointers and streams
then pass between the two unchanged.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime first, see above)

PKG_ROOT = Path(__file__).resolve().parents[1]
LIB_PATH = PKG_ROOT / "lib" / "libsdfr.so"

ABI_VERSION = 13
NOALLOC_SCRATCH_BYTES = 24 << 20   # SDFR_NOALLOC_SCRATCH_BYTES

# element types (SDFR_* in sdfr.h)
F32, F16, BF16, I32, I64, U8, F64, U16, R16 = 0, 1, 2, 3, 4, 5, 6, 7, 8
LAYOUT_LINEAR, LAYOUT_BRICK4 = 0, 1
CAM_EQUIANGULAR, CAM_PINHOLE = 0, 1
SCHED_PERSISTENT, SCHED_TILES = 0, 1
ORDER_LAUNCH, ORDER_LOOKAHEAD = 0, 1
FACES_AUTO, FACES_ON, FACES_OFF = 0, 1, 2

EXPORTS = ("sdfr_abi_version", "sdfr_last_error", "sdfr_grid_create", "sdfr_grid_destroy",
           "sdfr_grid_bytes", "sdfr_grid_attach_surfnz", "sdfr_grid_set_schedule",
           "sdfr_grid_set_tile_order", "sdfr_grid_set_border_faces", "sdfr_grid_set_march_events",
           "sdfr_render_rays_per_lane",
           "sdfr_workspace_bytes", "sdfr_render", "sdfr_render_noalloc", "sdfr_ray_dirs",
           "sdfr_grid_read",
           "sdfr_edt_workspace_bytes",
           "sdfr_edt", "sdfr_edt_last_error", "sdfr_goal_workspace_bytes", "sdfr_goal_bake",
           "sdfr_goal_sample", "sdfr_goal_last_error")


class GridDesc(ctypes.Structure):
    _fields_ = [("nx", ctypes.c_int32), ("ny", ctypes.c_int32), ("nz", ctypes.c_int32),
                ("mins", ctypes.c_float * 3), ("cell", ctypes.c_float)]


class Cam(ctypes.Structure):
    _fields_ = [("width", ctypes.c_int32), ("height", ctypes.c_int32),
                ("hfov_deg", ctypes.c_double), ("vfov_deg", ctypes.c_double),
                ("tan_half_h", ctypes.c_double), ("tan_half_v", ctypes.c_double),
                ("range", ctypes.c_float), ("near", ctypes.c_float),
                ("hit_eps", ctypes.c_float), ("min_step", ctypes.c_float),
                ("max_steps", ctypes.c_int32), ("camera", ctypes.c_int32)]


class Poses(ctypes.Structure):
    _fields_ = [("origin", ctypes.c_void_p), ("origin_stride", ctypes.c_int64),
                ("yaw_deg", ctypes.c_void_p), ("yaw_stride", ctypes.c_int64),
                ("pitch_deg", ctypes.c_void_p), ("pitch_stride", ctypes.c_int64),
                ("ducked", ctypes.c_void_p), ("ducked_stride", ctypes.c_int64),
                ("ducked_dtype", ctypes.c_int32), ("n_envs", ctypes.c_int32)]


class Image(ctypes.Structure):
    _fields_ = [("out", ctypes.c_void_p), ("env_stride", ctypes.c_int64),
                ("dtype", ctypes.c_int32), ("channels", ctypes.c_int32),
                ("taps", ctypes.c_void_p)]


class GoalInfo(ctypes.Structure):
    _fields_ = [("reach_max", ctypes.c_float), ("sentinel", ctypes.c_float),
                ("quant", ctypes.c_float), ("sweeps", ctypes.c_int32),
                ("n_seed", ctypes.c_int64), ("tile_visits", ctypes.c_int64)]


class SdfrError(RuntimeError):
    pass


_lib = None


def load(path: Path | str | None = None):
    """Open libsdfr.so once, declare its entry points, check the ABI."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise SdfrError(f"native renderer {p} is not built (run __graft_entry__.build()); "
                        "there is no fallback path")
    lib = ctypes.CDLL(str(p))
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    lib.sdfr_abi_version.restype = i32
    lib.sdfr_abi_version.argtypes = []
    lib.sdfr_last_error.restype = ctypes.c_char_p
    lib.sdfr_last_error.argtypes = []
    lib.sdfr_grid_create.restype = vp
    lib.sdfr_grid_create.argtypes = [ctypes.POINTER(GridDesc), vp, i32, i32, i32, i32, vp,
                                     ctypes.c_char_p, i32]
    lib.sdfr_grid_destroy.restype = None
    lib.sdfr_grid_destroy.argtypes = [vp]
    lib.sdfr_grid_bytes.restype = i64
    lib.sdfr_grid_bytes.argtypes = [vp]
    lib.sdfr_grid_attach_surfnz.restype = i32
    lib.sdfr_grid_attach_surfnz.argtypes = [vp, vp, i32, vp]
    lib.sdfr_grid_set_schedule.restype = i32
    lib.sdfr_grid_set_schedule.argtypes = [vp, i32, i32, i32]
    lib.sdfr_grid_set_tile_order.restype = i32
    lib.sdfr_grid_set_tile_order.argtypes = [vp, i32, i64]
    lib.sdfr_grid_set_border_faces.restype = i32
    lib.sdfr_grid_set_border_faces.argtypes = [vp, i32]
    lib.sdfr_grid_set_march_events.restype = i32
    lib.sdfr_render_rays_per_lane.restype = i32
    lib.sdfr_render_rays_per_lane.argtypes = [vp, ctypes.POINTER(Cam), i32]
    lib.sdfr_grid_set_march_events.argtypes = [vp, vp, vp]
    lib.sdfr_workspace_bytes.restype = i64
    lib.sdfr_workspace_bytes.argtypes = [ctypes.POINTER(Cam), i32]
    lib.sdfr_render.restype = i32
    lib.sdfr_render.argtypes = [vp, ctypes.POINTER(Cam), ctypes.POINTER(Poses),
                                ctypes.POINTER(Image), vp, i64, vp]
    lib.sdfr_render_noalloc.restype = i32
    lib.sdfr_render_noalloc.argtypes = [vp, ctypes.POINTER(Cam), ctypes.POINTER(Poses),
                                        ctypes.POINTER(Image), vp]
    lib.sdfr_grid_read.restype = i32
    lib.sdfr_grid_read.argtypes = [vp, vp, vp]
    lib.sdfr_ray_dirs.restype = i32
    lib.sdfr_ray_dirs.argtypes = [ctypes.POINTER(Cam), ctypes.POINTER(Poses), vp, vp]
    lib.sdfr_edt_workspace_bytes.restype = i64
    lib.sdfr_edt_workspace_bytes.argtypes = [i32, i32, i32]
    lib.sdfr_edt.restype = i32
    lib.sdfr_edt.argtypes = [vp, i32, i32, i32, ctypes.c_float, vp, i32, vp, i64, vp]
    lib.sdfr_edt_last_error.restype = ctypes.c_char_p
    lib.sdfr_edt_last_error.argtypes = []
    lib.sdfr_goal_workspace_bytes.restype = i64
    lib.sdfr_goal_workspace_bytes.argtypes = [i32, i32, i32]
    lib.sdfr_goal_bake.restype = i32
    lib.sdfr_goal_bake.argtypes = [vp, i32, i32, i32, ctypes.c_float, ctypes.POINTER(ctypes.c_int32),
                                   ctypes.POINTER(ctypes.c_int32), i32, vp, vp,
                                   ctypes.POINTER(GoalInfo), vp, i64, vp]
    lib.sdfr_goal_sample.restype = i32
    lib.sdfr_goal_sample.argtypes = [vp, i32, ctypes.c_float, i32, i32, i32,
                                     ctypes.POINTER(ctypes.c_double), ctypes.c_double,
                                     ctypes.c_double, vp, i32, i64, i64, vp, vp]
    lib.sdfr_goal_last_error.restype = ctypes.c_char_p
    lib.sdfr_goal_last_error.argtypes = []
    got = lib.sdfr_abi_version()
    if got != ABI_VERSION:
        raise SdfrError(f"{p} reports ABI {got}, this binding mirrors ABI {ABI_VERSION}: "
                        "rebuild the library")
    if path is None:
        _lib = lib
    return lib


def last_error(lib=None) -> str:
    lib = lib or load()
    return lib.sdfr_last_error().decode("utf-8", "replace")


def check(rc: int, what: str, lib=None) -> None:
    if rc != 0:
        raise SdfrError(f"{what} failed ({rc}): {last_error(lib)}")
