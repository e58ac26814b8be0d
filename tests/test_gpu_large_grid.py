"""A grid above 2 GiB renders exactly.

sdfr_grid_create accepts device copies up to 4 GiB: the march addresses its
copy with unsigned 32-bit byte offsets through one buffer descriptor whose
32-bit record count spans the whole copy, face copies included. The
reference keeps map-scale grids of this size (surf_src_cannonball: 654 M
voxels, python/surfgym/vision.py:433-437, 2.6 GB as fp32). This renders a
1024x1024x640 fp32 grid (2.5 GiB of bricks) with the eyes high in it, so
that the samples near the top of the grid and every ray that leaves through
the top (clamped to the last layer, vision.py:104-106) read bricks past the
2 GiB offset, and compares the image with the oracle's bit for bit, with
the border voxels read from the bricks and from the face copies. A map of
the reference's production size, stored fp16 as the reference stores it,
renders exactly as well.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from surfgym import synth, vision

pytestmark = pytest.mark.gpu

NX, NY, NZ, CELL = 1024, 1024, 640, 16.0


def test_a_grid_above_2_gib_renders_equal_to_the_oracle(dev):
    sc = synth.track_scene(NX, NY, NZ, CELL, 300, 1012)
    sc.bake()
    ps = synth.poses_above_ramps(sc, 256, 3012)
    top = np.argsort(ps.origin[:, 2])[-16:]             # the 16 highest eyes
    origin, yaw, pitch, duck = (np.ascontiguousarray(v[top]) for v in
                                (ps.origin, ps.yaw, ps.pitch, ps.ducked))
    kw = dict(width=128, height=64, range_units=float(np.linalg.norm([NX, NY, NZ]) * CELL),
              near_range=2000.0, max_steps=96, hit_eps=1.0)
    print(f"case large grid {NX}x{NY}x{NZ} f32, 16 envs", flush=True)
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, grid_dtype=torch.float32,
                                    device=dev, **kw)
    assert lid.grid_bytes > 2 ** 31 + 2 ** 28
    want, _ = oracle.render(sc.sdf, sc.mins, sc.cell, origin, yaw, pitch, duck, threads=16, **kw)
    args = [torch.as_tensor(v, device=dev) for v in (origin, yaw, pitch, duck)]
    for faces in ("off", "on"):
        lid.set_border_faces(faces)
        got = lid.render(*args).cpu().numpy()
        print(f"faces {faces}: {int((got != want).sum())} rays differ", flush=True)
        assert np.array_equal(got, want), faces
    # where the rays ended: a brick layer at or above voxel z 512 lies past the
    # 2 GiB offset (256 x 256 bricks of 256 B per layer of 4 voxels)
    d = lid.ray_dirs(args[1], args[2]).cpu().numpy().astype(np.float64)
    enc = want.astype(np.float64)
    t = np.where(enc <= 1.0, enc * 2000.0,
                 2000.0 - 2500.0 * np.log(np.clip(1.0 - (enc - 1.0) / 0.25, 1e-12, None)))
    eye_z = origin[:, 2] + np.where(duck != 0, 12.0, 17.0)
    z_end = eye_z[:, None, None] + d[..., 2] * t
    iz = np.clip(np.floor((z_end - sc.mins[2]) / CELL), 0, NZ - 1)
    assert (iz >= 512).mean() > 0.2, (iz >= 512).mean()


def test_a_map_of_the_references_production_size_renders_exactly(dev):
    """map_scale: 661 M voxels at 32 u (the size of the reference's
    production map, vision.py:433-437) with its production sensor (range
    11500, near 2000, 64 steps), in the reference's fp16 store: 16 envs
    equal the oracle's render of the fp16-rounded grid bit for bit."""
    store = "f16"
    w = synth.WORKLOADS["map_scale"]
    sc = w.scene()
    ps = w.poses(sc, 16)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, max_steps=w.max_steps, hit_eps=w.hit_eps)
    print(f"case map_scale {sc.nx}x{sc.ny}x{sc.nz} {store}, 16 envs", flush=True)
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, device=dev,
                                    grid_dtype=torch.float16, **kw)
    want, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                            store=store, threads=16, **kw)
    got = lid.render(*[torch.as_tensor(v, device=dev)
                       for v in (ps.origin, ps.yaw, ps.pitch, ps.ducked)]).cpu().numpy()
    assert np.array_equal(got, want), int((got != want).sum())
