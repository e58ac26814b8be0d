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


def test_binding_structs_match_the_header_layout(tmp_path):
    """Every field offset and struct size gcc gives the header's structs
    equals what the ctypes mirror uses."""
    import subprocess
    from surfgym import _sdfr
    structs = {"SdfrGridDesc": _sdfr.GridDesc, "SdfrCam": _sdfr.Cam,
               "SdfrPoses": _sdfr.Poses, "SdfrImage": _sdfr.Image}
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
        (_sdfr.GridDesc(2, 2, 2, (ctypes.c_float * 3)(), 16.0), 7, 0, 0, "source dtype"),
        (_sdfr.GridDesc(2, 2, 2, (ctypes.c_float * 3)(), 16.0), 0, 2, 0, "store dtype"),
        (_sdfr.GridDesc(2, 2, 2, (ctypes.c_float * 3)(), 16.0), 0, 0, 9, "layout"),
    ]:
        h = lib.sdfr_grid_create(ctypes.byref(desc), src.ctypes.data, dtype, 0, store, layout,
                                 None, err, len(err))
        assert not h
        assert needle in err.value.decode(), err.value
    assert not lib.sdfr_grid_create(None, None, 0, 0, 0, 0, None, err, len(err))
    assert b"null" in err.value


def test_render_rejects_bad_arguments_without_a_device():
    from surfgym import _sdfr
    lib = _sdfr.load()
    img = _sdfr.Image(64, 128 * 64, _sdfr.F32, 1, None)
    rc = lib.sdfr_render(None, ctypes.byref(_cam()), ctypes.byref(_poses()), ctypes.byref(img),
                         None, 0, None)
    assert rc == -1 and "grid" in _sdfr.last_error()
    assert lib.sdfr_workspace_bytes(ctypes.byref(_cam()), 2048) == 2048 * (128 + 64 + 4) * 8
    assert lib.sdfr_workspace_bytes(ctypes.byref(_cam()), 0) < 0
    # the grid check comes first; the argument checks are shared with sdfr_ray_dirs
    cases = [
        (dict(width=0), {}, "image size"),
        (dict(max_steps=-1), {}, "max_steps"),
        (dict(near=0.0), {}, "near"),
        (dict(camera=5), {}, "camera"),
        ({}, dict(n_envs=0), "n_envs"),
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
