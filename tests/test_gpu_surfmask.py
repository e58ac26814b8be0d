"""The surf-mask channel (GpuLidar(surf_mask=True), reference
python/surfgym/vision.py:118-191, 558-570, 658-666) on the GPU.

The reference checks its mask renderer on an analytic world
(tests/python/test_surfmask.py:174-240): the channel must not disturb the
depth, must report the |n_z| of the voxel a ray stops in (1 on a flat floor,
0 where a ray runs out into the sky), and must come out interleaved with the
depth, channel fastest. The same three properties are checked here on a
terrace world of this file's own, then both channels against the CPU
oracle ray for ray, in every schedule.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from surfgym import synth, vision

pytestmark = pytest.mark.gpu

CELL = 16.0
NX, NY, NZ = 40, 24, 20
SLOPE_X = 20          # columns ix >= SLOPE_X carry a sloped surface's |n_z|
SLOPE_NZ = 90         # |n_z| * 127 of that surface (about 45 degrees)


def _terrace():
    """Ground below z = 0: each voxel's distance is its centre height, the
    bottom layer is the surface, flat (127) west of SLOPE_X and tilted
    (SLOPE_NZ) east of it; every voxel above the bottom layer reads 0."""
    sdf = np.broadcast_to(((np.arange(NZ) + 0.5) * CELL).astype(np.float32)[:, None, None],
                          (NZ, NY, NX)).copy()
    sdf[0] = 0.0
    snz = np.zeros((NZ, NY, NX), np.int8)
    snz[0, :, :SLOPE_X] = 127
    snz[0, :, SLOPE_X:] = SLOPE_NZ
    return sdf, snz


# eye = origin + 17; (x, y, z, yaw, pitch, ducked)
_VIEWS = np.array([[120.0, 190.0, 133.0, 0.0, -90.0, 0.0],     # down onto the flat part
                   [520.0, 190.0, 128.0, 0.0, -90.0, 1.0],     # down onto the slope, ducked
                   [300.0, 190.0, 133.0, 90.0, 65.0, 0.0]],    # up, out of the grid
                  np.float32)


def _views(dev):
    v = torch.as_tensor(_VIEWS, device=dev)
    return v[:, 0:3], v[:, 3], v[:, 4], v[:, 5]


def _lidar(dev, snz=None, **kw):
    sdf, _ = _terrace()
    return vision.GpuLidar.from_grid(sdf, np.zeros(3), CELL, width=12, height=6,
                                     range_units=1200.0, surf_nz=snz, device=dev, **kw)


def test_the_mask_channel_leaves_the_depth_channel_alone(dev):
    print("case surf-mask: depth channel unchanged", flush=True)
    _, snz = _terrace()
    plain, masked = _lidar(dev), _lidar(dev, snz)
    assert (plain.surf_mask, plain.channels) == (False, 1)
    assert (masked.surf_mask, masked.channels) == (True, 2)
    base = {k for k, v in vars(plain).items() if torch.is_tensor(v)}
    extra = {k for k, v in vars(masked).items() if torch.is_tensor(v)} - base
    assert extra == {"snz_flat"}, extra
    d = plain.render(*_views(dev))
    both = masked.render(*_views(dev))
    assert d.shape == (3, 6, 12) and both.shape == (3, 6, 12, 2)
    assert torch.equal(both[..., 0], d)


def test_the_mask_channel_reports_the_surface_under_the_hit(dev):
    print("case surf-mask: surface under the hit", flush=True)
    _, snz = _terrace()
    out = _lidar(dev, snz).render(*_views(dev)).cpu()
    flat, slope, sky = out[0], out[1], out[2]
    assert float(flat[..., 0].max()) < 0.2 and float(slope[..., 0].max()) < 0.2
    assert torch.all(flat[..., 1] == 1.0)
    assert torch.all(slope[..., 1] == torch.tensor(SLOPE_NZ / 127.0))
    assert torch.all(sky[..., 0] == 1.0)          # ran to range, encoding clamps at 1
    assert torch.all(sky[..., 1] == 0.0)


def test_the_two_channels_are_interleaved(dev):
    print("case surf-mask: interleaved layout", flush=True)
    _, snz = _terrace()
    lid = _lidar(dev, snz)
    out = lid.render(*_views(dev))
    assert out.is_contiguous() and out.stride()[-1] == 1 and out.shape[-1] == 2
    flat = out.reshape(3, -1)
    assert torch.equal(flat[:, 0::2].reshape(3, 6, 12), out[..., 0])
    assert torch.equal(flat[:, 1::2].reshape(3, 6, 12), out[..., 1])
    row = torch.full((3, 15 + flat.shape[1] + 4), -3.0, device=dev)
    lid.render(*_views(dev), out=row[:, 15:15 + flat.shape[1]])
    assert torch.equal(row[:, 15:15 + flat.shape[1]], flat)
    assert torch.all(row[:, :15] == -3.0) and torch.all(row[:, -4:] == -3.0)


@pytest.mark.parametrize("schedule,rpl", [("persistent", None), ("persistent", 2),
                                          ("tiles", 1), ("tiles", 2)])
def test_every_pixel_is_written_whatever_the_schedule(dev, schedule, rpl):
    """The mask renders with the tiles kernel whatever schedule the handle is
    set to; every pixel of a -1-filled output is written and equals the
    oracle's, sorted or not."""
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc)
    snz = np.random.default_rng(3).integers(0, 128, sc.sdf.shape).astype(np.int8)
    print(f"case surf-mask schedule={schedule} rpl={rpl}", flush=True)
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, surf_nz=snz,
                                    range_units=w.range_units, near_range=w.near_range,
                                    max_steps=w.max_steps, hit_eps=w.hit_eps,
                                    grid_dtype=torch.float32, schedule=schedule,
                                    rays_per_lane=rpl, device=dev)
    want, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                            range_units=w.range_units, near_range=w.near_range,
                            hit_eps=w.hit_eps, max_steps=w.max_steps, surf_nz=snz, threads=16)
    args = [torch.as_tensor(v, device=dev) for v in (ps.origin, ps.yaw, ps.pitch, ps.ducked)]
    for min_tiles in (0, None):
        lid.set_tile_order("lookahead", min_tiles=min_tiles)
        out = torch.full((len(ps), w.height, w.width, 2), -1.0, device=dev)
        lid.render(*args, out=out)
        assert np.array_equal(out.cpu().numpy(), want), min_tiles


@pytest.mark.parametrize("layout,out_dtype,rpl", [("brick4", torch.float32, None),
                                                  ("linear", torch.float32, None),
                                                  ("brick4", torch.bfloat16, None),
                                                  ("brick4", torch.float32, 2)])
def test_both_channels_match_the_oracle(dev, layout, out_dtype, rpl):
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc)
    rng = np.random.default_rng(7)
    snz = rng.integers(0, 128, sc.sdf.shape).astype(np.int8)
    print(f"case surf-mask parity layout={layout} out={out_dtype} rpl={rpl}", flush=True)
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, surf_nz=snz,
                                    range_units=w.range_units, near_range=w.near_range,
                                    max_steps=w.max_steps, hit_eps=w.hit_eps,
                                    grid_dtype=torch.float32, layout=layout, device=dev,
                                    rays_per_lane=rpl)
    n = len(ps)
    out = torch.empty(n, w.height, w.width, 2, dtype=out_dtype, device=dev)
    taps = torch.empty(n, w.height, w.width, dtype=torch.int32, device=dev)
    lid.render(torch.as_tensor(ps.origin, device=dev), torch.as_tensor(ps.yaw, device=dev),
               torch.as_tensor(ps.pitch, device=dev), torch.as_tensor(ps.ducked, device=dev),
               out=out, taps=taps)
    want, loads = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                                range_units=w.range_units, near_range=w.near_range,
                                hit_eps=w.hit_eps, max_steps=w.max_steps, surf_nz=snz,
                                threads=16)
    if out_dtype == torch.bfloat16:
        want = torch.as_tensor(want).to(torch.bfloat16).float().numpy()
    got = out.float().cpu().numpy()
    exact = (got == want).all(axis=-1).mean()
    print(f"surf-mask {layout}/{out_dtype}: both channels exact on {exact:.6f} of rays", flush=True)
    assert exact >= 0.999
    assert (taps.cpu().numpy() == loads).mean() >= 0.999
