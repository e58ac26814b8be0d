"""Seeded random renders against the oracle.

Each case draws a grid (shape, cell, origin, a distance-like field), a
camera (size, field of view, equiangular or pinhole, optionally the
surf-mask channel), the step rule (range, near, hit_eps, min_step,
max_steps), a batch of poses inside and outside the grid, and a library
configuration (store, layout, schedule, rays per lane, tile order, output
dtype, census, border faces). The image must equal the oracle's on the grid as stored bit
for bit (bf16: the oracle's fp32 encodings rounded to nearest even), and the
census its per-ray load counts. The sweep reaches combinations the fixed
tests do not: odd image sizes against the 16x4 tiles, step budgets from 0 to
200, cells that are not powers of two, near beyond the range.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from surfgym import vision

pytestmark = pytest.mark.gpu

N_CASES = 600


def _field(rng, shape, cell):
    """Distance (in units) from each voxel centre to a few random solid
    voxels, 0 on them; optionally a solid floor."""
    nz, ny, nx = shape
    zz, yy, xx = np.meshgrid(np.arange(nz), np.arange(ny), np.arange(nx), indexing="ij")
    pts = rng.integers(0, [nz, ny, nx], (max(1, int(np.prod(shape)) // 60), 3))
    d = np.full(shape, np.inf)
    for z, y, x in pts:
        d = np.minimum(d, np.sqrt((zz - z) ** 2 + (yy - y) ** 2 + (xx - x) ** 2))
    if rng.random() < 0.5:
        d = np.minimum(d, zz)   # a floor at z = 0
    return (d * cell).astype(np.float32)


def _case(seed):
    rng = np.random.default_rng(9000 + seed)
    shape = tuple(int(v) for v in rng.integers(1, 40, 3))
    cell = float(rng.choice([8.0, 12.0, 16.0, 24.0, 32.0]))
    mins = rng.uniform(-300.0, 300.0, 3).astype(np.float32)
    grid = _field(rng, shape, cell)
    ext = np.array(shape[::-1], np.float64) * cell
    n = int(rng.integers(1, 25))
    origin = (mins + rng.uniform(-0.3, 1.3, (n, 3)) * ext).astype(np.float32)
    pinhole = bool(rng.random() < 0.3)
    surf = (not pinhole) and rng.random() < 0.2
    rng_units = float(rng.uniform(0.3, 2.0) * np.linalg.norm(ext))
    cam = dict(width=int(rng.integers(1, 150)), height=int(rng.integers(1, 70)),
               hfov_deg=float(rng.uniform(30.0, 170.0)), vfov_deg=float(rng.uniform(20.0, 120.0)),
               range_units=rng_units,
               near_range=float(rng_units * rng.choice([1.0, rng.uniform(0.2, 1.5)])),
               max_steps=int(rng.integers(0, 3) if rng.random() < 0.15 else rng.integers(3, 201)),
               hit_eps=float(rng.choice([0.6 * cell, rng.uniform(0.05, 1.5) * cell])),
               min_step=float(rng.choice([0.3 * cell, rng.uniform(0.05, 1.0) * cell])),
               pinhole=pinhole)
    poses = (origin, rng.uniform(-180.0, 180.0, n).astype(np.float32),
             rng.uniform(-89.0, 89.0, n).astype(np.float32),
             (rng.random(n) < 0.5).astype(np.float32))
    store = str(rng.choice(["f32", "f16", "r16"]))
    layout = "brick4" if store == "r16" else str(rng.choice(["brick4", "linear"]))
    lib = dict(schedule=str(rng.choice(["tiles", "tiles", "persistent"])),
               rays_per_lane=[None, 1, 2][int(rng.integers(0, 3))],
               order=str(rng.choice(["launch", "lookahead"])),
               out=str(rng.choice(["f32", "bf16"])), census=bool(rng.random() < 0.5),
               faces=str(rng.choice(["auto", "on", "off"])) if store != "r16" and layout == "brick4"
               else "auto")
    snz = rng.integers(0, 128, shape).astype(np.int8) if surf else None
    return grid, mins, cell, poses, cam, store, layout, lib, snz


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_render_equals_the_oracle(dev, seed):
    grid, mins, cell, poses, cam, store, layout, lib, snz = _case(seed)
    n = len(poses[0])
    print(f"case random seed={seed} grid={grid.shape} cell={cell} n={n} "
          f"{cam['width']}x{cam['height']} pinhole={cam['pinhole']} surf={snz is not None} "
          f"steps={cam['max_steps']} store={store}/{layout} {lib}", flush=True)
    want, loads = oracle.render(grid, mins, cell, *poses, store=store, surf_nz=snz, **cam)
    gdt = {"f32": torch.float32, "f16": torch.float16, "r16": "r16"}[store]
    lid = vision.GpuLidar.from_grid(grid, mins, cell, surf_nz=snz, grid_dtype=gdt, layout=layout,
                                    device=dev, **cam)
    lid.set_schedule(lib["schedule"], rays_per_lane=lib["rays_per_lane"])
    lid.set_tile_order(lib["order"], min_tiles=0)
    lid.set_border_faces(lib["faces"])
    ch = (2,) if snz is not None else ()
    odt = torch.bfloat16 if lib["out"] == "bf16" else torch.float32
    out = torch.full((n, cam["height"], cam["width"]) + ch, -1.0, dtype=odt, device=dev)
    taps = (torch.full((n, cam["height"], cam["width"]), -1, dtype=torch.int32, device=dev)
            if lib["census"] else None)
    lid.render(*[torch.as_tensor(a, device=dev) for a in poses], out=out, taps=taps)
    if odt == torch.float32:
        assert np.array_equal(out.cpu().numpy(), want)
    else:
        assert torch.equal(out.cpu(), torch.as_tensor(want).to(torch.bfloat16))
    if taps is not None:
        assert np.array_equal(taps.cpu().numpy(), loads)
