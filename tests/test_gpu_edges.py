"""GPU edge cases of the render against the oracle: degenerate grid shapes
(one voxel thick along any axis, a single voxel, partial bricks) in every
store and layout, eyes outside the grid on every side (every sample then
reads the clamped border voxel first, vision.py:644-646), and grids whose
cell or origin keeps the voxel index in subtract-then-scale form; where the
grid keeps border face copies, with the march reading them and not."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from surfgym import vision

pytestmark = pytest.mark.gpu

_STORES = [(torch.float32, "f32", "brick4"), (torch.float32, "f32", "linear"),
           (torch.float16, "f16", "brick4"), ("r16", "r16", "brick4")]


def _field(shape, seed):
    """A distance-like field: distance (16 u cells) to a few random solid
    voxels, 0 on them."""
    rng = np.random.default_rng(seed)
    nz, ny, nx = shape
    zz, yy, xx = np.meshgrid(np.arange(nz), np.arange(ny), np.arange(nx), indexing="ij")
    pts = rng.integers(0, [nz, ny, nx], (max(1, int(np.prod(shape)) // 40), 3))
    d = np.full(shape, np.inf)
    for z, y, x in pts:
        d = np.minimum(d, np.sqrt((zz - z) ** 2 + (yy - y) ** 2 + (xx - x) ** 2))
    return (d * 16.0).astype(np.float32)


def _has_faces(store, layout):
    return store in ("f32", "f16") and layout == "brick4"


def _poses(shape, n, seed, outside=False):
    rng = np.random.default_rng(seed)
    ext = np.array(shape[::-1], np.float64) * 16.0
    if outside:
        # eyes beyond each face of the grid (and beyond corners)
        o = rng.uniform(-0.5, 1.5, (n, 3)) * ext
        o[:, rng.integers(0, 3)] = np.where(rng.random(n) < 0.5, -200.0, ext.max() + 200.0)
    else:
        o = rng.uniform(0.0, 1.0, (n, 3)) * ext
    o[:, 2] -= 17.0
    yaw = rng.uniform(-180, 180, n).astype(np.float32)
    pitch = rng.uniform(-70, 30, n).astype(np.float32)
    duck = (rng.random(n) < 0.5).astype(np.float32)
    return o.astype(np.float32), yaw, pitch, duck


@pytest.mark.parametrize("shape", [(1, 1, 1), (1, 5, 3), (4, 1, 9), (7, 6, 1), (5, 9, 13),
                                   (2, 33, 2)])
@pytest.mark.parametrize("gdt,store,layout", _STORES)
def test_degenerate_grid_shapes(dev, shape, gdt, store, layout):
    g = _field(shape, sum(shape))
    n = 5
    o, yaw, pitch, duck = _poses(shape, n, 7)
    print(f"case edges shape={shape} store={store} layout={layout}", flush=True)
    kw = dict(width=24, height=10, range_units=900.0, near_range=400.0, max_steps=48)
    lid = vision.GpuLidar.from_grid(g, np.zeros(3), 16.0, grid_dtype=gdt, layout=layout,
                                    device=dev, **kw)
    want, _ = oracle.render(g, np.zeros(3), 16.0, o, yaw, pitch, duck, store=store, **kw)
    faces = ("off", "on") if _has_faces(store, layout) else ("auto",)
    for mode in faces:
        lid.set_border_faces(mode)
        for order in ("lookahead", "launch"):
            lid.set_tile_order(order, min_tiles=0)
            got = lid.render(*[torch.as_tensor(a, device=dev) for a in (o, yaw, pitch, duck)])
            assert np.array_equal(got.cpu().numpy(), want), (mode, order)


@pytest.mark.parametrize("gdt,store,layout", _STORES)
def test_eyes_outside_the_grid(dev, gdt, store, layout):
    shape = (20, 24, 28)
    g = _field(shape, 3)
    n = 64
    o, yaw, pitch, duck = _poses(shape, n, 11, outside=True)
    print(f"case edges eyes outside store={store} layout={layout}", flush=True)
    kw = dict(width=32, height=16, range_units=1500.0, near_range=600.0, max_steps=64)
    lid = vision.GpuLidar.from_grid(g, np.full(3, -8.0), 16.0, grid_dtype=gdt, layout=layout,
                                    device=dev, **kw)
    want, _ = oracle.render(g, np.full(3, -8.0), 16.0, o, yaw, pitch, duck, store=store, **kw)
    for mode in (("off", "on") if _has_faces(store, layout) else ("auto",)):
        lid.set_border_faces(mode)
        for rpl in (1, 2):
            lid.set_schedule("tiles", rays_per_lane=rpl)
            got = lid.render(*[torch.as_tensor(a, device=dev) for a in (o, yaw, pitch, duck)])
            assert np.array_equal(got.cpu().numpy(), want), (mode, rpl)


def test_border_faces_exist_for_f32_and_f16_bricks(dev):
    """set_border_faces("on") is refused where the grid keeps no face
    copies (r16 bricks, the linear layout); "auto" and "off" are accepted."""
    g = _field((6, 7, 9), 2)
    for gdt, layout in (("r16", "brick4"), (torch.float32, "linear"), (torch.float16, "linear")):
        lid = vision.GpuLidar.from_grid(g, np.zeros(3), 16.0, grid_dtype=gdt, layout=layout,
                                        device=dev, width=8, height=8)
        lid.set_border_faces("auto")
        lid.set_border_faces("off")
        with pytest.raises(Exception, match="face copies"):
            lid.set_border_faces("on")
    with pytest.raises(ValueError):
        lid.set_border_faces("always")


@pytest.mark.parametrize("cell,mins", [(12.0, (-8.0, -8.0, -8.0)), (24.0, (3.0, -5.0, 0.0)),
                                       (16.0, (1e-40, -8.0, 2.5))])
@pytest.mark.parametrize("gdt,store,layout", _STORES)
def test_grids_without_the_single_rounding_index(dev, cell, mins, gdt, store, layout):
    """The march forms a sample's voxel coordinate as one fma when inv_cell
    is a power of two and mins * inv_cell is exact, and as the reference's
    subtract-then-scale otherwise (vision.py:104-106). Cells of 12 and 24 u,
    and a 16 u cell whose x origin is subnormal (so its scaled value is not
    exact), take the second form: one and two rays per lane, both tile
    orders, against the oracle."""
    shape = (9, 14, 17)
    g = _field(shape, 5)
    mins = np.array(mins, np.float32)
    n = 12
    o, yaw, pitch, duck = _poses(shape, n, 13)
    kw = dict(width=40, height=12, range_units=1200.0, near_range=500.0, max_steps=64)
    want, _ = oracle.render(g, mins, cell, o, yaw, pitch, duck, store=store, **kw)
    lid = vision.GpuLidar.from_grid(g, mins, cell, grid_dtype=gdt, layout=layout, device=dev, **kw)
    args = [torch.as_tensor(a, device=dev) for a in (o, yaw, pitch, duck)]
    if _has_faces(store, layout):
        lid.set_border_faces("on")
    for rpl in (1, 2):
        lid.set_schedule("tiles", rays_per_lane=rpl)
        for order in ("launch", "lookahead"):
            lid.set_tile_order(order, min_tiles=0)
            print(f"case edges cell={cell} mins={mins.tolist()} store={store} layout={layout} "
                  f"rpl={rpl} order={order}", flush=True)
            got = lid.render(*args)
            assert np.array_equal(got.cpu().numpy(), want), (cell, rpl, order)


@pytest.mark.parametrize("eps", [16.0, 16.003, 0.0, -3.0, 70000.0, 1e-6, float("inf")])
def test_fp16_samples_against_hit_eps_at_every_rounding(dev, eps):
    """fp16 bricks widen each sample to fp32 and compare it with hit_eps,
    as the reference compares its fp16 gathers (vision.py:107-109). Grid
    values at and a few
    fp16 steps either side of hit_eps (and of its fp16 floor), with hit_eps
    exact in fp16, between two fp16 values, zero, negative, beyond the fp16
    range and infinite: every image equals the oracle's on the f16-rounded
    grid, one and two rays per lane."""
    rng = np.random.default_rng(17)
    shape = (6, 7, 8)
    e16 = np.float16(np.clip(eps, -65504.0, 65504.0)) if np.isfinite(eps) else np.float16(60000.0)
    steps = np.arange(-3, 4)
    bits = (e16.view(np.uint16).astype(np.int32) + np.where(e16 < 0, -steps, steps)).astype(np.uint16)
    near = bits.view(np.float16).astype(np.float32)
    near = near[np.isfinite(near)]
    g = rng.choice(np.concatenate([near, np.float32([0.0, 40.0, 300.0])]), size=shape).astype(np.float32)
    n = 6
    o, yaw, pitch, duck = _poses(shape, n, 19)
    kw = dict(width=24, height=8, range_units=700.0, near_range=300.0, max_steps=24, hit_eps=eps,
              min_step=4.0)
    want, _ = oracle.render(g, np.zeros(3), 16.0, o, yaw, pitch, duck, store="f16", **kw)
    lid = vision.GpuLidar.from_grid(g, np.zeros(3), 16.0, grid_dtype=torch.float16, device=dev, **kw)
    args = [torch.as_tensor(a, device=dev) for a in (o, yaw, pitch, duck)]
    for rpl in (1, 2):
        lid.set_schedule("tiles", rays_per_lane=rpl)
        print(f"case edges fp16 hit_eps={eps} rpl={rpl}", flush=True)
        got = lid.render(*args)
        assert np.array_equal(got.cpu().numpy(), want), (eps, rpl)


def test_the_largest_batch_renders_every_env(dev):
    """The largest batch the library accepts at 128x64 (2^31 - 1 rays):
    262,140 envs, four distinct poses repeated, so the image offsets reach
    the top of the int32 range. Every env must equal the oracle's image of
    its pose (batch independence, tests/python/test_lidar_march.py:161-169,
    at the size limit)."""
    from surfgym import synth
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, 4)
    n = 262_140
    assert n * w.width * w.height <= 2 ** 31 - 1 < (n + 4) * w.width * w.height
    print(f"case edges largest batch n={n}", flush=True)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units, near_range=w.near_range,
              max_steps=w.max_steps, hit_eps=w.hit_eps)
    want, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked, **kw)
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, grid_dtype=torch.float32, device=dev,
                                    **kw)
    rep = lambda a: torch.as_tensor(a, device=dev).repeat((n // 4,) + (1,) * (a.ndim - 1))  # noqa: E731
    got = lid.render(rep(ps.origin), rep(ps.yaw), rep(ps.pitch), rep(ps.ducked))
    assert got.shape == (n, w.height, w.width)
    ref = torch.as_tensor(want, device=dev)
    assert torch.equal(got.view(n // 4, 4, w.height, w.width)[-1], ref)
    assert bool((got.view(n // 4, 4, w.height, w.width) == ref).all())
    del got
    torch.cuda.empty_cache()
