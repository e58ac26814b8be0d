"""The C-ABI boundary without a GPU: the library loads, exports every entry
point include/sdfr.h declares, reports its ABI version, and rejects bad
arguments before touching the device (surfcore.h-style error returns)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "sdfr.h").read_text()
    return set(re.findall(r"SDFR_API\s+[\w\s\*]+?\b(sdfr_\w+)\s*\(", text))


def test_every_declared_symbol_is_exported_and_bound():
    from surfgym import _sdfr
    lib = ctypes.CDLL(str(_sdfr.LIB_PATH))
    declared = _declared()
    assert declared == set(_sdfr.EXPORTS), declared ^ set(_sdfr.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version_matches_the_binding():
    from surfgym import _sdfr
    lib = _sdfr.load()
    text = (ROOT / "include" / "sdfr.h").read_text()
    assert int(re.search(r"#define SDFR_ABI_VERSION (\d+)", text).group(1)) == _sdfr.ABI_VERSION
    assert lib.sdfr_abi_version() == _sdfr.ABI_VERSION
    m = re.search(r"#define SDFR_NOALLOC_SCRATCH_BYTES \((\d+)ll << (\d+)\)", text)
    assert int(m.group(1)) << int(m.group(2)) == _sdfr.NOALLOC_SCRATCH_BYTES


def test_binding_structs_match_the_header_layout(tmp_path):
    """Every field offset and struct size gcc gives the header's structs
    equals what the ctypes mirror uses."""
    import subprocess
    from surfgym import _sdfr
    structs = {"SdfrGridDesc": _sdfr.GridDesc, "SdfrCam": _sdfr.Cam,
               "SdfrPoses": _sdfr.Poses, "SdfrImage": _sdfr.Image,
               "SdfrGoalInfo": _sdfr.GoalInfo}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "sdfr.h"', "int main(void){"]
    for cname, cls in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    for line in got.splitlines():
        cname, field, value = line.split()
        cls = structs[cname]
        want = ctypes.sizeof(cls) if field == "size" else getattr(cls, field).offset
        assert int(value) == want, line


def _cam(**kw):
    from surfgym import _sdfr
    c = _sdfr.Cam(128, 64, 120.0, 90.0, 1.7, 1.0, 2000.0, 2000.0, 9.6, 4.8, 64, 0)
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def _poses(**kw):
    from surfgym import _sdfr
    p = _sdfr.Poses(8, 3, 16, 1, 24, 1, 32, 1, _sdfr.F32, 4)   # dummy non-null pointers
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_grid_create_rejects_bad_descriptors_without_a_device():
    from surfgym import _sdfr
    lib = _sdfr.load()
    err = ctypes.create_string_buffer(256)
    src = np.zeros(8, np.float32)
    for desc, dtype, store, layout, needle in [
        (_sdfr.GridDesc(0, 2, 2, (ctypes.c_float * 3)(), 16.0), 0, 0, 0, "positive"),
        (_sdfr.GridDesc(2, 2, 2, (ctypes.c_float * 3)(), 0.0), 0, 0, 0, "cell"),
        (_sdfr.GridDesc(2, 2, 2, (ctypes.c_float * 3)(), 16.0), 42, 0, 0, "source dtype"),
        (_sdfr.GridDesc(2, 2, 2, (ctypes.c_float * 3)(), 16.0), 0, 2, 0, "store dtype"),
        (_sdfr.GridDesc(2, 2, 2, (ctypes.c_float * 3)(), 16.0), 0, 0, 9, "layout"),
        (_sdfr.GridDesc(2, 2, 2, (ctypes.c_float * 3)(), 16.0), 0, _sdfr.R16,
         _sdfr.LAYOUT_LINEAR, "brick4 layout only"),
        (_sdfr.GridDesc(2, 2, 2, (ctypes.c_float * 3)(), 16.0), 0, 9, 1, "store dtype"),
    ]:
        h = lib.sdfr_grid_create(ctypes.byref(desc), src.ctypes.data, dtype, 0, store, layout,
                                 None, err, len(err))
        assert not h
        assert needle in err.value.decode(), err.value
    assert not lib.sdfr_grid_create(None, None, 0, 0, 0, 0, None, err, len(err))
    assert b"null" in err.value


def test_schedule_and_tile_order_reject_a_null_handle_without_a_device():
    from surfgym import _sdfr
    lib = _sdfr.load()
    assert lib.sdfr_grid_read(None, None, None) == -1
    assert "null grid" in _sdfr.last_error()
    assert lib.sdfr_render_noalloc(None, None, None, None, None) == -1
    assert "null grid" in _sdfr.last_error()
    assert lib.sdfr_grid_set_schedule(None, 2, 16, 0) == -1      # no slot schedule any more
    assert lib.sdfr_grid_set_tile_order(None, _sdfr.ORDER_LOOKAHEAD, -1) == -1
    assert "null grid" in _sdfr.last_error()
    assert lib.sdfr_grid_set_schedule(None, _sdfr.SCHED_TILES, 16, 2) == -1
    assert "null grid" in _sdfr.last_error()
    assert lib.sdfr_grid_set_march_events(None, None, None) == -1
    assert "null grid" in _sdfr.last_error()
    assert lib.sdfr_grid_set_border_faces(None, _sdfr.FACES_ON) == -1
    assert "null grid" in _sdfr.last_error()


def test_border_face_modes_match_the_header():
    from surfgym import _sdfr
    text = (ROOT / "include" / "sdfr.h").read_text()
    for name, value in (("AUTO", _sdfr.FACES_AUTO), ("ON", _sdfr.FACES_ON),
                        ("OFF", _sdfr.FACES_OFF)):
        assert re.search(rf"SDFR_FACES_{name} = {value}\b", text), name


def test_render_rejects_bad_arguments_without_a_device():
    from surfgym import _sdfr
    lib = _sdfr.load()
    img = _sdfr.Image(64, 128 * 64, _sdfr.F32, 1, None)
    rc = lib.sdfr_render(None, ctypes.byref(_cam()), ctypes.byref(_poses()), ctypes.byref(img),
                         None, 0, None)
    assert rc == -1 and "grid" in _sdfr.last_error()
    # ray tables, then an int32, a uint16 and a uint32 per 16x4 tile (parts 256-byte aligned)
    assert lib.sdfr_workspace_bytes(ctypes.byref(_cam()), 2048) == (
        2048 * (128 + 64 + 4) * 8 + 2048 * 128 * 4 + 2048 * 128 * 2 + 2048 * 128 * 4)
    c = _cam(width=9, height=5)
    assert lib.sdfr_workspace_bytes(ctypes.byref(c), 3) == 512 + 256 + 256 + 256
    # tiles come in 2x2 quads of 32x8 pixels: 40x9 is 2 x 2 quads, 16 tiles per env
    c = _cam(width=40, height=9)
    a256 = lambda v: (v + 255) // 256 * 256   # noqa: E731
    assert lib.sdfr_workspace_bytes(ctypes.byref(c), 100) == (
        a256(100 * (40 + 9 + 4) * 8) + a256(1600 * 4) + a256(1600 * 2) + a256(1600 * 4))
    assert lib.sdfr_workspace_bytes(ctypes.byref(_cam()), 0) < 0
    # the grid check comes first; the argument checks are shared with sdfr_ray_dirs
    cases = [
        (dict(width=0), {}, "image size"),
        (dict(max_steps=-1), {}, "max_steps"),
        (dict(near=0.0), {}, "near"),
        (dict(camera=5), {}, "camera"),
        ({}, dict(n_envs=0), "n_envs"),
        (dict(width=8192, height=4096), {}, "image too large"),
        ({}, dict(n_envs=262144), "too many rays"),   # 2^31 rays of 128x64
        ({}, dict(origin=None), "null pose"),
        ({}, dict(ducked_dtype=42), "ducked dtype"),
    ]
    out = (ctypes.c_float * 3)()
    for ck, pk, needle in cases:
        rc = lib.sdfr_ray_dirs(ctypes.byref(_cam(**ck)), ctypes.byref(_poses(**pk)),
                               ctypes.addressof(out), None)
        assert rc < 0 and needle in _sdfr.last_error(), (ck, pk, _sdfr.last_error())
    rc = lib.sdfr_ray_dirs(ctypes.byref(_cam()), ctypes.byref(_poses()), None, None)
    assert rc == -1 and "output" in _sdfr.last_error()


def test_lidar_refuses_the_cpu_instead_of_falling_back():
    from surfgym import vision
    with pytest.raises(ValueError, match="no CPU path"):
        vision.GpuLidar.from_grid(np.full((4, 4, 4), 99.0, np.float32), np.zeros(3), 16.0,
                                  device="cpu")
    with pytest.raises(ValueError, match="no combined kernel"):
        vision.GpuLidar(None, surf_mask=True, pinhole=True)
    with pytest.raises(ValueError, match="no CPU path"):
        vision.GpuLidar.from_grid(np.full((4, 4, 4), 99.0, np.float32), np.zeros(3), 16.0,
                                  surf_nz=np.zeros((4, 4, 4), np.int8), device="cpu")


def test_missing_library_is_an_error(tmp_path):
    from surfgym import _sdfr
    with pytest.raises(_sdfr.SdfrError, match="not built"):
        _sdfr.load(tmp_path / "libsdfr.so")


def test_grid_contract_helpers():
    """grid_dims / pick_cell arithmetic (vision.py:283-322) on a fake core."""
    from surfgym import vision

    class Core:
        def map_bounds(self):
            return np.array([-1000.0, -500.0, -64.0]), np.array([1000.0, 1500.0, 900.0])

    mins, nx, ny, nz = vision.grid_dims(Core(), 16.0)
    assert np.allclose(mins, [-1064.0, -564.0, -128.0])
    assert (nx, ny, nz) == (133, 133, 69)
    assert vision.pick_cell(Core()) == 16.0
    assert vision.pick_cell(Core(), budget_voxels=1e5) == 64.0


def test_goal_entry_points_reject_bad_arguments_without_a_device():
    from surfgym import _sdfr
    lib = _sdfr.load()
    assert lib.sdfr_goal_workspace_bytes(0, 4, 4) < 0
    ws = lib.sdfr_goal_workspace_bytes(17, 9, 8)
    tiles = 3 * 2 * 1
    assert ws >= 17 * 9 * 8 * 4 + 4 * tiles * 4
    info = _sdfr.GoalInfo()
    lo = (ctypes.c_int32 * 3)(0, 0, 0)
    hi = (ctypes.c_int32 * 3)(1, 1, 1)
    fake = 64 * 1024   # never dereferenced: every case fails before a launch
    cases = [
        (dict(occ=None), -1, "null"),
        (dict(grid_q=None, grid=None), -1, "null"),
        (dict(nx=0), -2, "positive"),
        (dict(cell=0.0), -2, "cell"),
        (dict(max_sweeps=0), -2, "max_sweeps"),
        (dict(size=16), -2, "workspace"),
        (dict(ws=fake + 4), -2, "aligned"),
        (dict(hi=(ctypes.c_int32 * 3)(-1, 1, 1)), -5, "no free voxel"),
    ]
    for kw, code, needle in cases:
        a = dict(occ=fake, nx=17, ny=9, nz=8, cell=16.0, lo=lo, hi=hi, max_sweeps=100,
                 grid_q=fake, grid=None, ws=fake, size=ws)
        a.update(kw)
        rc = lib.sdfr_goal_bake(a["occ"], a["nx"], a["ny"], a["nz"], a["cell"], a["lo"], a["hi"],
                                a["max_sweeps"], a["grid_q"], a["grid"], ctypes.byref(info),
                                a["ws"], a["size"], None)
        msg = lib.sdfr_goal_last_error().decode()
        assert rc == code and needle in msg, (kw, rc, msg)
    mins = (ctypes.c_double * 3)(0.0, 0.0, 0.0)
    for args, code, needle in [
        ((fake, 42, 1.0, 4, 4, 4, mins, 16.0, 100.0, fake, _sdfr.F64, 3, 1, fake), -3, "grid dtype"),
        ((fake, _sdfr.F32, 1.0, 4, 4, 4, mins, 16.0, 100.0, fake, _sdfr.I32, 3, 1, fake), -3,
         "position dtype"),
        ((fake, _sdfr.F32, 1.0, 4, 4, 4, mins, 16.0, 100.0, fake, _sdfr.F64, 2, 1, fake), -2,
         "stride"),
        ((fake, _sdfr.F32, 1.0, 0, 4, 4, mins, 16.0, 100.0, fake, _sdfr.F64, 3, 1, fake), -2,
         "dims"),
        ((None, _sdfr.F32, 1.0, 4, 4, 4, mins, 16.0, 100.0, fake, _sdfr.F64, 3, 1, fake), -1,
         "null"),
    ]:
        rc = lib.sdfr_goal_sample(*args, None)
        msg = lib.sdfr_goal_last_error().decode()
        assert rc == code and needle in msg, (rc, msg)
    assert lib.sdfr_goal_sample(fake, _sdfr.F32, 1.0, 4, 4, 4, mins, 16.0, 100.0, None, _sdfr.F64,
                                3, 0, fake, None) == 0


def test_goal_seed_box_and_cache_contract(tmp_path):
    """The seed box rounding (goalfield.py:148-156, :228-231) by hand, the
    cache signature format (:173-177), and the refusals of the host layer."""
    from surfgym import goalfield
    # a zone shrunk to the centre of voxel 5 (88 u at cell 16): grown by 20 u
    # to [68, 108] -> floor(68/16 - .5) = 3, ceil(108/16 - .5) = 7
    z = {"mins": [88.0, 88.0, 88.0], "maxs": [88.0, 88.0, 88.0]}
    lo, hi = goalfield.seed_voxel_box(z, np.zeros(3), 16.0, (20, 20, 20))
    assert lo.tolist() == [3, 3, 3] and hi.tolist() == [7, 7, 7]
    # cell 64 grows by 48 u: [40, 136] -> floor(.125) = 0, ceil(1.625) = 2; clipped to the grid
    lo, hi = goalfield.seed_voxel_box(z, np.zeros(3), 64.0, (2, 9, 9))
    assert lo.tolist() == [0, 0, 0] and hi.tolist() == [1, 2, 2]
    # below the grid: lo clips to 0, hi stays negative (an empty box)
    lo, hi = goalfield.seed_voxel_box({"mins": [-900.0] * 3, "maxs": [-800.0] * 3},
                                      np.zeros(3), 16.0, (8, 8, 8))
    assert lo.tolist() == [0, 0, 0] and np.all(hi < 0)

    bsp = tmp_path / "surf_x.bsp"
    bsp.write_bytes(b"BSP" * 10)
    st = bsp.stat()
    zone = {"mins": [1.04, -2.0, 3.0], "maxs": [10.0, 20.0, 30.55]}
    sig = goalfield._goal_sig(bsp, zone, False)
    assert sig == f"g4_v2_{st.st_size}_{st.st_mtime_ns}_1_-2_3_10_20_30.6"
    assert goalfield._goal_sig(bsp, zone, True).startswith("g4_k1_v2_")

    with pytest.raises(ValueError, match="no CPU path"):
        goalfield.GoalField(np.zeros((2, 2, 2), np.float32), np.zeros(3), 16.0, 10.0,
                            device="cpu")
    with pytest.raises(ValueError, match="no CPU path"):
        goalfield.goal_field_from_occupancy(np.zeros((2, 2, 2)), np.zeros(3), zone, 16.0,
                                            device="cpu")


