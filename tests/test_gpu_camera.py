"""End-to-end camera properties of the reference's renderer, on the GPU.

The reference's pinhole tests (tests/python/test_pinhole.py:180-243)
photograph one straight world edge: under the pinhole camera (a regular grid
on the tangent plane, vision.py:609-624) a straight line perpendicular to
the view axis images to a single pixel row; under the equiangular camera
(angles added to the view, vision.py:596-607) the same edge bows, highest in
the middle of the frame; and both cameras cast the same ray through the
image centre. Its march test (tests/python/test_lidar_march.py:150-158)
checks that the poses it uses actually exercise the march: some rays hit
close, some run past the near range, and neither kind is all of them.

Here the edge is the rim of a shelf of this file's own making, rendered by
the HIP kernels and cross-checked against the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from surfgym import synth, vision

pytestmark = pytest.mark.gpu

CELL = 8.0
NX, NY, NZ = 128, 160, 64            # 1024 x 1280 x 512 u
RIM_X, TOP_Z, DEPTH = 600.0, 240.0, 12.0
EYE = (260.0, 640.0, 440.0)          # eye position (origin z + 17)
RANGE = 2500.0


def _shelf():
    """Exact distance from each voxel centre to a shelf: the slab
    TOP_Z - DEPTH <= z <= TOP_Z for every x >= RIM_X (all y). Its rim is the
    straight line x = RIM_X, z = TOP_Z, at right angles to a view along +x."""
    x = (np.arange(NX) + 0.5) * CELL
    z = (np.arange(NZ) + 0.5) * CELL
    dx = np.clip(RIM_X - x, 0.0, None)
    dz = np.clip(np.maximum(z - TOP_Z, (TOP_Z - DEPTH) - z), 0.0, None)
    d = np.sqrt(dz[:, None] ** 2 + dx[None, :] ** 2)
    return np.repeat(d[:, None, :], NY, axis=1).astype(np.float32)


@pytest.fixture(scope="module")
def shelf():
    return _shelf()


# The view pitch puts the rim's image between two image rows' rays at both
# sizes (pitches within half a degree of it do too), so no row grazes it:
# nearest-voxel sampling near the rim would otherwise decide per column.
PITCH = -11.0


def _render(dev, sdf, size, pinhole, pitch=PITCH):
    lid = vision.GpuLidar.from_grid(sdf, np.zeros(3), CELL, width=size, height=size,
                                    range_units=RANGE, pinhole=pinhole, device=dev,
                                    grid_dtype=torch.float32)
    origin = np.array([[EYE[0], EYE[1], EYE[2] - 17.0]], np.float32)
    args = (origin, np.zeros(1, np.float32), np.array([pitch], np.float32),
            np.zeros(1, np.float32))
    got = lid.render(*[torch.as_tensor(a, device=dev) for a in args])[0].cpu().numpy()
    want, _ = oracle.render(sdf, np.zeros(3), CELL, *args, width=size, height=size,
                            range_units=RANGE, pinhole=pinhole)
    assert np.array_equal(got, want[0]), "kernel and oracle disagree on the shelf"
    return got


def _rim_rows(img):
    """Per image column, the lowest image row whose ray meets the shelf:
    looking slightly down from above the shelf, rows above the rim's image
    land on the shelf top (or its front face), rows below it pass under the
    shelf and run to range."""
    hit = img < 0.99
    assert 0.1 < hit.mean() < 0.9, f"the frame is degenerate ({hit.mean():.2f} hit)"
    rows = np.array([np.flatnonzero(hit[:, c]).max() if hit[:, c].any() else -1
                     for c in range(img.shape[1])])
    assert (rows >= 0).all(), "some column never sees the shelf"
    return rows


@pytest.mark.parametrize("size", [32, 33])
def test_the_rim_is_one_image_row_under_the_pinhole_camera(dev, shelf, size):
    print(f"case camera: pinhole rim {size}", flush=True)
    rows = _rim_rows(_render(dev, shelf, size, pinhole=True))
    assert rows.min() == rows.max(), f"rim spread over rows {rows.min()}..{rows.max()}"


@pytest.mark.parametrize("size", [32, 33])
def test_the_rim_bows_under_the_equiangular_camera(dev, shelf, size):
    """The control for the test above: the same rim, equiangular, crosses
    several rows, lowest (largest row index) at the centre columns and
    falling off symmetrically to both edges."""
    print(f"case camera: equiangular rim {size}", flush=True)
    rows = _rim_rows(_render(dev, shelf, size, pinhole=False))
    mid = size // 2
    assert rows.max() - rows.min() >= 3, rows
    assert rows[mid] > rows[0] and rows[mid] > rows[-1], rows
    assert rows[mid] == rows.max()
    assert np.abs(rows - rows[::-1]).max() <= 1, rows


def test_both_cameras_share_the_centre_ray_only(dev, shelf):
    """At an odd size the centre pixel is the view ray itself in both
    cameras; elsewhere the images differ."""
    print("case camera: centre ray", flush=True)
    a = _render(dev, shelf, 33, pinhole=False)
    b = _render(dev, shelf, 33, pinhole=True)
    assert a[16, 16] == b[16, 16]
    assert float(np.abs(a - b).max()) > 0.05


def test_the_bench_poses_exercise_the_march(dev):
    """ramp_field's poses (400-800 u above the ramps, pitch U[-70, 30]):
    near hits, rays past the near range, and neither all of them."""
    w = synth.WORKLOADS["ramp_field"]
    sc = w.scene()
    ps = w.poses(sc, 256)
    print("case camera: poses exercise the march", flush=True)
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, width=w.width, height=w.height,
                                    range_units=w.range_units, near_range=w.near_range,
                                    max_steps=w.max_steps, hit_eps=w.hit_eps,
                                    grid_dtype=torch.float32, device=dev)
    d = lid.render(*[torch.as_tensor(v, device=dev)
                     for v in (ps.origin, ps.yaw, ps.pitch, ps.ducked)])
    far = float((d > 1.0).float().mean())
    print(f"min {d.min().item():.4f} max {d.max().item():.4f} past near {far:.3f}", flush=True)
    assert d.min().item() < 0.05, "no near hits"
    assert d.max().item() > 1.0, "nothing beyond the near range"
    assert 0.02 < far < 0.98, far


def test_the_pinhole_flag_allocates_only_its_tables(dev, shelf):
    """Equiangular lidars hold the grid, mins and the two angle tables as
    tensors; the pinhole flag adds exactly the tangent-plane tables
    (u = tan(hfov/2) * (2c/(W-1) - 1), v = tan(vfov/2) * (1 - 2r/(H-1)),
    vision.py:510-529), and an equiangular render is unchanged by the
    feature existing (tests/python/test_pinhole.py:251-263)."""
    off = vision.GpuLidar.from_grid(shelf, np.zeros(3), CELL, width=8, height=4, device=dev)
    on = vision.GpuLidar.from_grid(shelf, np.zeros(3), CELL, width=8, height=4, pinhole=True,
                                   device=dev)
    base = {k for k, v in vars(off).items() if torch.is_tensor(v)}
    # sdf_flat is read back from the handle's copy on first access
    assert base == {"mins", "yoff", "poff"}
    assert {k for k, v in vars(on).items() if torch.is_tensor(v)} - base == {"uoff", "voff"}
    assert torch.equal(off.sdf_flat.cpu(), torch.as_tensor(shelf, dtype=torch.float16).reshape(-1))
    assert {k for k, v in vars(off).items() if torch.is_tensor(v)} == base | {"_sdf_flat"}
    assert off.pinhole is False and on.pinhole is True
    th, tv = np.tan(np.radians(60.0)), np.tan(np.radians(45.0))
    assert np.allclose(on.uoff.cpu().numpy(), th * (2 * np.arange(8) / 7 - 1), atol=1e-6)
    assert np.allclose(on.voff.cpu().numpy(), tv * (1 - 2 * np.arange(4) / 3), atol=1e-6)
    args = [torch.as_tensor(a, device=dev) for a in
            (np.array([[300.0, 600.0, 300.0]], np.float32), np.zeros(1, np.float32),
             np.array([-20.0], np.float32), np.zeros(1, np.float32))]
    assert off.render(*args).shape == (1, 4, 8) and on.render(*args).shape == (1, 4, 8)


def test_the_lidar_holds_one_device_copy_of_the_grid(dev):
    """Only the handle's re-laid-out copy stays resident: the flat grid the
    copy is made from is released, and torch holds just the small tables
    until sdf_flat is first read, which then equals the grid as stored."""
    g = (np.random.default_rng(3).random((64, 128, 128), dtype=np.float32) * 100.0)
    torch.cuda.synchronize(dev)
    base = torch.cuda.memory_allocated(dev)
    lid = vision.GpuLidar.from_grid(g, np.zeros(3), CELL, width=8, height=4,
                                    grid_dtype=torch.float32, device=dev)
    torch.cuda.synchronize(dev)
    assert torch.cuda.memory_allocated(dev) - base < 64 * 1024
    assert lid.grid_bytes >= g.nbytes
    assert torch.equal(lid.sdf_flat.cpu(), torch.as_tensor(g).reshape(-1))
    assert torch.cuda.memory_allocated(dev) - base >= g.nbytes   # now kept


@pytest.mark.parametrize("W,H", [(1, 9), (9, 1), (1, 1)])
def test_a_one_pixel_axis_looks_along_the_view(dev, shelf, W, H):
    """A one-pixel axis has its single ray on the view's centre line in both
    cameras (pinhole u = 0 / v = 0, equiangular offset 0;
    tests/python/test_pinhole.py:266-273)."""
    for pin in (False, True):
        lid = vision.GpuLidar.from_grid(shelf, np.zeros(3), CELL, width=W, height=H,
                                        pinhole=pin, device=dev)
        d = lid.ray_dirs(torch.tensor([30.0]), torch.tensor([-12.0]))[0].cpu().numpy()
        y, p = np.radians(30.0), np.radians(-12.0)
        view = np.array([np.cos(p) * np.cos(y), np.cos(p) * np.sin(y), np.sin(p)])
        if W == 1:
            col = d[:, 0, :]
            # every ray of the single column lies in the vertical plane of the view
            assert np.abs(col[:, 0] * np.sin(y) - col[:, 1] * np.cos(y)).max() < 1e-6
        if H == 1:
            row = d[0, :, :]
            if pin:
                # the single row of the pinhole camera lies in the view's
                # horizontal-tilted plane through the centre ray
                assert np.abs(row @ np.cross(view, [-np.sin(y), np.cos(y), 0.0])).max() < 1e-6
            else:
                assert np.allclose(row[:, 2], np.sin(p), atol=1e-7)
        if W % 2 == 1 and H % 2 == 1:
            assert np.abs(d[H // 2, W // 2] - view).max() < 1e-6
