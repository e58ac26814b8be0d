"""Every march kernel the library instantiates, against the oracle.

The render is a family of kernels: grid store (fp32, fp16, r16) x layout
(bricks, the reference's linear order) x camera (equiangular, pinhole) x
output (f32, bf16) x census (load counts on or off) x schedule (tiles with
one or two tiles per wave, persistent) x tile order (launch, lookahead),
plus the surf-mask channel. One tile per wave in launch order is a small
render's path, where each wave builds its tile's ray-table entries itself;
the other schedules and the sorted order read the tables the ray-setup
launch writes. Each combination renders the same small scene on
an image that leaves quads of tiles partly outside it, and must equal the
oracle on the grid as stored: depth encodings bit for bit (bf16: the oracle's
fp32 encodings rounded to nearest even), per-ray load counts exactly.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from surfgym import synth, vision

pytestmark = pytest.mark.gpu

W, H, N = 40, 22, 6
_STORES = [("f32", "brick4", torch.float32), ("f32", "linear", torch.float32),
           ("f16", "brick4", torch.float16), ("f16", "linear", torch.float16),
           ("r16", "brick4", "r16")]
_SCHEDULES = [("tiles", 1), ("tiles", 2), ("persistent", None)]


@pytest.fixture(scope="module")
def scene():
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, N)
    snz = np.random.default_rng(5).integers(0, 128, sc.sdf.shape).astype(np.int8)
    return w, sc, ps, snz


def _kw(w):
    return dict(width=W, height=H, range_units=w.range_units, near_range=w.near_range,
                max_steps=w.max_steps, hit_eps=w.hit_eps)


def _want(w, sc, ps, store, pinhole=False, surf_nz=None):
    return oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                         store=store, pinhole=pinhole, surf_nz=surf_nz, **_kw(w))


def _args(ps, dev):
    return [torch.as_tensor(a, device=dev) for a in (ps.origin, ps.yaw, ps.pitch, ps.ducked)]


@pytest.mark.parametrize("store,layout,gdt", _STORES)
@pytest.mark.parametrize("camera", ["equiangular", "pinhole"])
def test_every_depth_kernel_matches_the_oracle(dev, scene, store, layout, gdt, camera):
    w, sc, ps, _ = scene
    pin = camera == "pinhole"
    want, loads = _want(w, sc, ps, store, pinhole=pin)
    want_bf = torch.as_tensor(want).to(torch.bfloat16)
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, grid_dtype=gdt, layout=layout,
                                    pinhole=pin, device=dev, **_kw(w))
    args = _args(ps, dev)
    for schedule, rpl in _SCHEDULES:
        lid.set_schedule(schedule, rays_per_lane=rpl)
        for order in ("launch", "lookahead"):
            lid.set_tile_order(order, min_tiles=0)
            for odt in (torch.float32, torch.bfloat16):
                for census in (False, True):
                    case = f"{store}/{layout} {camera} {schedule} rpl={rpl} {order} {odt} census={census}"
                    print(f"case matrix {case}", flush=True)
                    out = torch.full((N, H, W), -1.0, dtype=odt, device=dev)
                    taps = (torch.full((N, H, W), -1, dtype=torch.int32, device=dev)
                            if census else None)
                    lid.render(*args, out=out, taps=taps)
                    if odt == torch.float32:
                        assert np.array_equal(out.cpu().numpy(), want), case
                    else:
                        assert torch.equal(out.cpu(), want_bf), case
                    if census:
                        assert np.array_equal(taps.cpu().numpy(), loads), case


@pytest.mark.parametrize("store,layout,gdt", _STORES)
def test_every_surf_mask_kernel_matches_the_oracle(dev, scene, store, layout, gdt):
    """The surf-mask channel runs the tiles schedule whatever the lidar's
    setting (persistent included)."""
    w, sc, ps, snz = scene
    want, loads = _want(w, sc, ps, store, surf_nz=snz)
    want_bf = torch.as_tensor(want).to(torch.bfloat16)
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, surf_nz=snz, grid_dtype=gdt,
                                    layout=layout, device=dev, **_kw(w))
    args = _args(ps, dev)
    for schedule, rpl in _SCHEDULES:
        lid.set_schedule(schedule, rays_per_lane=rpl)
        for order in ("launch", "lookahead"):
            lid.set_tile_order(order, min_tiles=0)
            for odt in (torch.float32, torch.bfloat16):
                for census in (False, True):
                    case = f"surf {store}/{layout} {schedule} rpl={rpl} {order} {odt} census={census}"
                    print(f"case matrix {case}", flush=True)
                    out = torch.full((N, H, W, 2), -1.0, dtype=odt, device=dev)
                    taps = (torch.full((N, H, W), -1, dtype=torch.int32, device=dev)
                            if census else None)
                    lid.render(*args, out=out, taps=taps)
                    if odt == torch.float32:
                        assert np.array_equal(out.cpu().numpy(), want), case
                    else:
                        assert torch.equal(out.cpu(), want_bf), case
                    if census:
                        assert np.array_equal(taps.cpu().numpy(), loads), case
