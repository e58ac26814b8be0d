"""The surf-mask channel (GpuLidar(surf_mask=True), reference
python/surfgym/vision.py:118-191, 558-570, 658-666) on the GPU.

The first three tests restate the reference's renderer tests of the mask
(tests/python/test_surfmask.py:174-240) — a floor-slab world with an
analytic SDF — against this renderer; the last compares both channels with
the CPU oracle ray for ray.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from surfgym import synth, vision

pytestmark = pytest.mark.gpu

RCELL = 16.0
RNX, RNY, RNZ = 32, 32, 16


def _floor_world():
    sdf = (np.arange(RNZ, dtype=np.float32) * RCELL)[:, None, None] \
        * np.ones((1, RNY, RNX), dtype=np.float32)
    snz = np.zeros((RNZ, RNY, RNX), dtype=np.int8)
    snz[0] = 127                                        # the floor is flat
    return sdf, snz


def _poses(dev):
    #                x      y      z (eye = z + 17)  yaw  pitch duck
    a = np.array([[200.0, 200.0, 183.0, 0.0, -90.0, 0],    # straight down
                  [200.0, 200.0, 183.0, 0.0, 80.0, 0],     # up into the sky
                  [200.0, 200.0, 183.0, 45.0, -30.0, 0]], dtype=np.float32)
    return (torch.as_tensor(a[:, 0:3], device=dev), torch.as_tensor(a[:, 3], device=dev),
            torch.as_tensor(a[:, 4], device=dev), torch.as_tensor(a[:, 5], device=dev))


def test_flag_off_changes_nothing(dev):
    print("case surf-mask flag off", flush=True)
    sdf, snz = _floor_world()
    off = vision.GpuLidar.from_grid(sdf, np.zeros(3), RCELL, width=8, height=4, device=dev)
    on = vision.GpuLidar.from_grid(sdf, np.zeros(3), RCELL, width=8, height=4, device=dev,
                                   surf_nz=snz)
    tensors = {k for k, v in vars(off).items() if torch.is_tensor(v)}
    assert tensors == {"sdf_flat", "mins", "yoff", "poff"}
    assert {k for k, v in vars(on).items() if torch.is_tensor(v)} - tensors == {"snz_flat"}
    assert (off.surf_mask, off.channels) == (False, 1)
    assert (on.surf_mask, on.channels) == (True, 2)
    d = off.render(*_poses(dev))
    both = on.render(*_poses(dev))
    assert d.shape == (3, 4, 8) and both.shape == (3, 4, 8, 2)
    assert torch.equal(both[..., 0], d), "the mask perturbed the depth channel"


def test_mask_channel_reads_the_hit_surface(dev):
    print("case surf-mask reads the surface", flush=True)
    sdf, snz = _floor_world()
    lid = vision.GpuLidar.from_grid(sdf, np.zeros(3), RCELL, width=8, height=4, device=dev,
                                    surf_nz=snz)
    out = lid.render(*_poses(dev))
    down, up = out[0], out[1]
    assert down[..., 0].max() < 0.2, "the floor should be close below"
    assert torch.all(down[..., 1] == 1.0), "flat floor must read |n_z| = 1"
    assert torch.all(up[..., 0] > 0.9), "the sky pixels should run to range"
    assert torch.all(up[..., 1] == 0.0), "open sky must read 0"


def test_flat_image_is_channel_fastest(dev):
    print("case surf-mask layout", flush=True)
    sdf, snz = _floor_world()
    lid = vision.GpuLidar.from_grid(sdf, np.zeros(3), RCELL, width=8, height=4, device=dev,
                                    surf_nz=snz)
    out = lid.render(*_poses(dev))
    flat = out.reshape(3, -1)
    assert torch.equal(flat.reshape(-1, 4, 8, 2), out)
    im = flat.reshape(-1, 4, 8, 2).permute(0, 3, 1, 2)
    assert im.stride()[1] == 1, "channel stride must be 1 (NHWC)"
    # and it can be written straight into an observation row
    obs = torch.full((3, 15 + 4 * 8 * 2), -3.0, device=dev)
    lid.render(*_poses(dev), out=obs[:, 15:])
    assert torch.equal(obs[:, 15:], flat) and torch.all(obs[:, :15] == -3.0)


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
