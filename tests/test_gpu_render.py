"""GPU parity: the HIP renderer (through the C ABI) against the CPU oracle.

Bar (per ray, same seeded inputs): at least 99.9% of rays within 0.5 u of
the oracle's depth and encodings within 1e-3; in practice the two agree
bit-for-bit on nearly every ray because both evaluate the same fp32
operation sequence. Reference semantics: python/surfgym/vision.py:59-116,
:596-666.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from surfgym import synth, vision

pytestmark = pytest.mark.gpu

DEPTH_TOL_U = 0.5
ENC_TOL = 1e-3
MIN_AGREE = 0.999


def _say(msg):
    print(msg, flush=True)


_SCENES = {}


def _scene(name):
    if name not in _SCENES:
        w = synth.WORKLOADS[name]
        _SCENES[name] = (w, w.scene())
    return _SCENES[name]


def _depth(enc, near, rng):
    """Invert the encoding to depth in units (both branches are monotone)."""
    enc = np.asarray(enc, np.float64)
    lin = enc * near
    tail = near - 2500.0 * np.log(np.clip(1.0 - (enc - 1.0) / 0.25, 1e-12, None))
    return np.where(enc <= 1.0, lin, np.minimum(tail, rng))


def _lidar(dev, w, sc, **kw):
    args = dict(width=w.width, height=w.height, range_units=w.range_units,
                near_range=w.near_range, max_steps=w.max_steps, hit_eps=w.hit_eps,
                grid_dtype=torch.float32, device=dev)
    args.update(kw)
    return vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, **args)


def _gpu_render(lid, ps, dev, **kw):
    return lid.render(torch.as_tensor(ps.origin, device=dev), torch.as_tensor(ps.yaw, device=dev),
                      torch.as_tensor(ps.pitch, device=dev),
                      torch.as_tensor(ps.ducked, device=dev), **kw)


def _oracle(w, sc, ps, store="f32", **kw):
    args = dict(width=w.width, height=w.height, range_units=w.range_units,
                near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps, store=store,
                threads=16)
    args.update(kw)
    return oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked, **args)


def _assert_parity(got, want, w, label):
    got = np.asarray(got, np.float32)
    d_enc = np.abs(got - want)
    d_u = np.abs(_depth(got, w.near_range, w.range_units) - _depth(want, w.near_range,
                                                                   w.range_units))
    ok = (d_enc <= ENC_TOL) & (d_u <= DEPTH_TOL_U)
    exact = float((got == want).mean())
    _say(f"{label}: {got.size} rays, exact {exact:.6f}, within tol {ok.mean():.6f}, "
         f"max|d enc| {d_enc.max():.3e}")
    assert ok.mean() >= MIN_AGREE, f"{label}: only {ok.mean():.5f} of rays within tolerance"
    return ok


@pytest.mark.parametrize("layout", ["linear", "brick4"])
def test_small_ramps_matches_the_oracle(dev, layout):
    w, sc = _scene("small_ramps")
    ps = w.poses(sc)
    _say(f"case small_ramps layout={layout} envs={len(ps)}")
    lid = _lidar(dev, w, sc, layout=layout)
    taps = torch.empty(len(ps), w.height, w.width, dtype=torch.int32, device=dev)
    got = _gpu_render(lid, ps, dev, taps=taps).cpu().numpy()
    want, loads = _oracle(w, sc, ps)
    ok = _assert_parity(got, want, w, f"small_ramps/{layout}")
    # the census counts the same loads the oracle counts, ray for ray
    assert (taps.cpu().numpy()[ok] == loads[ok]).mean() > 0.999


@pytest.mark.parametrize("layout,rpl", [("linear", None), ("brick4", None), ("brick4", 2)])
def test_ramp_field_matches_the_oracle(dev, layout, rpl):
    """256 envs: one ray per lane by default (a small render), and two."""
    w, sc = _scene("ramp_field")
    ps = w.poses(sc, 256)
    _say(f"case ramp_field layout={layout} rpl={rpl} envs={len(ps)}")
    lid = _lidar(dev, w, sc, layout=layout, rays_per_lane=rpl)
    assert lid.effective_rays_per_lane(len(ps)) == (rpl or 1)
    got = _gpu_render(lid, ps, dev).cpu().numpy()
    want, _ = _oracle(w, sc, ps)
    _assert_parity(got, want, w, f"ramp_field/{layout}")


def test_f16_store_matches_the_oracle_on_the_rounded_grid(dev):
    """The reference's device grid is f16 (vision.py:476-477): rounding to
    nearest even, then widening, is what both sides read."""
    w, sc = _scene("ramp_field")
    ps = w.poses(sc, 128)
    _say("case ramp_field f16 store envs=128")
    lid = _lidar(dev, w, sc, grid_dtype=torch.float16)
    got = _gpu_render(lid, ps, dev).cpu().numpy()
    want, _ = _oracle(w, sc, ps, store="f16")
    _assert_parity(got, want, w, "ramp_field/f16")


@pytest.mark.parametrize("name,n,size", [("ramp_field", 96, None), ("small_ramps", 16, None),
                                         ("ramp_field", 23, (37, 19)), ("small_ramps", 9, (8, 8))])
def test_f16_slot_packing_is_exact(dev, name, n, size):
    """fp16 grids march with slot packing (a wave's two tiles merged into one
    slot once their live rays fit 64 lanes): images and per-ray load counts
    equal the oracle's on the f16-rounded grid bit for bit, in both tile
    orders. 37x19 images give quads of tiles partly outside the image
    (lanes and whole tiles without a pixel); 8x8 images give one quad per
    env, half of it outside."""
    w, sc = _scene(name)
    ps = w.poses(sc, n)
    W, H = size if size else (w.width, w.height)
    _say(f"case f16 packing {name} n={n} {W}x{H}")
    lid = _lidar(dev, w, sc, grid_dtype=torch.float16, width=W, height=H, rays_per_lane=2)
    assert lid.rays_per_lane == 2 and lid.effective_rays_per_lane(n) == 2
    want, want_taps = _oracle(w, sc, ps, store="f16", width=W, height=H)
    for order in ("lookahead", "launch"):
        lid.set_tile_order(order, min_tiles=0)
        taps = torch.full((n, H, W), -1, dtype=torch.int32, device=dev)
        got = torch.full((n, H, W), -1.0, device=dev)
        _gpu_render(lid, ps, dev, out=got, taps=taps)
        assert np.array_equal(got.cpu().numpy(), want), order
        assert np.array_equal(taps.cpu().numpy(), want_taps), order


def test_bf16_output_is_the_rounded_f32_output(dev):
    w, sc = _scene("small_ramps")
    ps = w.poses(sc)
    _say("case small_ramps bf16 out")
    lid = _lidar(dev, w, sc)
    f32 = _gpu_render(lid, ps, dev)
    bf = torch.empty(len(ps), w.height, w.width, dtype=torch.bfloat16, device=dev)
    _gpu_render(lid, ps, dev, out=bf)
    assert torch.equal(bf, f32.to(torch.bfloat16))


def test_batch_size_is_irrelevant_to_the_result(dev):
    """tests/python/test_lidar_march.py:161-169."""
    w, sc = _scene("small_ramps")
    ps = w.poses(sc)
    _say("case batch independence")
    lid = _lidar(dev, w, sc)
    full = _gpu_render(lid, ps, dev)
    for i in (0, 3, 7, 15):
        one = lid.render(torch.as_tensor(ps.origin[i:i + 1], device=dev),
                         torch.as_tensor(ps.yaw[i:i + 1], device=dev),
                         torch.as_tensor(ps.pitch[i:i + 1], device=dev),
                         torch.as_tensor(ps.ducked[i:i + 1], device=dev))
        assert torch.equal(one[0], full[i]), i


def test_strided_pose_views_and_ducked_dtypes(dev):
    """The trainer passes columns of a packed (N,6) tensor
    (train_fast.py:1749-1757) with float ducked."""
    w, sc = _scene("small_ramps")
    ps = w.poses(sc)
    _say("case strided inputs")
    lid = _lidar(dev, w, sc)
    ref = _gpu_render(lid, ps, dev)
    packed = torch.as_tensor(np.concatenate([ps.origin, ps.yaw[:, None], ps.pitch[:, None],
                                             ps.ducked[:, None]], 1), device=dev)
    got = lid.render(packed[:, 0:3], packed[:, 3], packed[:, 4], packed[:, 5])
    assert torch.equal(got, ref)
    for dt in (torch.bool, torch.int32, torch.int64, torch.uint8, torch.float64):
        got = lid.render(packed[:, 0:3], packed[:, 3], packed[:, 4], packed[:, 5].to(dt))
        assert torch.equal(got, ref), dt


def test_render_into_an_observation_row(dev):
    """Fused epilogue: write straight into the image columns of the
    trainer's (N, 15 + H*W) observation buffer (train_fast.py:1760)."""
    w, sc = _scene("small_ramps")
    ps = w.poses(sc)
    _say("case obs-row output")
    lid = _lidar(dev, w, sc)
    ref = _gpu_render(lid, ps, dev)
    obs = torch.full((len(ps), 15 + w.height * w.width), -7.0, device=dev)
    lid.render(torch.as_tensor(ps.origin, device=dev), torch.as_tensor(ps.yaw, device=dev),
               torch.as_tensor(ps.pitch, device=dev), torch.as_tensor(ps.ducked, device=dev),
               out=obs[:, 15:])
    assert torch.equal(obs[:, 15:].reshape(-1, w.height, w.width), ref)
    assert torch.all(obs[:, :15] == -7.0)


def test_settings_changed_between_renders_take_effect(dev):
    """render keeps the C-ABI camera and the output-layout check of its last
    call; sensor attributes set between renders, a new output layout and a
    bad output after a good one must all still be honoured."""
    w, sc = _scene("small_ramps")
    ps = w.poses(sc)
    _say("case settings changed between renders")
    lid = _lidar(dev, w, sc)
    want, _ = _oracle(w, sc, ps)
    assert np.array_equal(_gpu_render(lid, ps, dev).cpu().numpy(), want)
    lid.max_steps, lid.range, lid.near = 12, 900.0, 600.0
    want2, _ = _oracle(w, sc, ps, max_steps=12, range_units=900.0, near_range=600.0)
    assert not np.array_equal(want2, want)
    assert np.array_equal(_gpu_render(lid, ps, dev).cpu().numpy(), want2)
    obs = torch.full((len(ps), 15 + w.height * w.width), -7.0, device=dev)
    _gpu_render(lid, ps, dev, out=obs[:, 15:])
    assert np.array_equal(obs[:, 15:].reshape(-1, w.height, w.width).cpu().numpy(), want2)
    with pytest.raises(ValueError):
        _gpu_render(lid, ps, dev, out=obs[:, 14:])
    with pytest.raises(ValueError):
        _gpu_render(lid, ps, dev, out=obs[:, 15:].to(torch.float16))
    lid.pinhole = True
    want3, _ = _oracle(w, sc, ps, max_steps=12, range_units=900.0, near_range=600.0,
                       pinhole=True)
    assert np.array_equal(_gpu_render(lid, ps, dev).cpu().numpy(), want3)
    lid.pinhole = False
    assert np.array_equal(_gpu_render(lid, ps, dev).cpu().numpy(), want2)


@pytest.mark.parametrize("W,H", [(9, 5), (33, 33), (1, 1), (128, 64), (20, 12)])
def test_ray_directions_equal_the_oracle(dev, W, H):
    """sdfr_ray_dirs exposes the march's own ray setup; the oracle restates
    _dirs_equiangular / _dirs_pinhole (vision.py:596-624)."""
    _say(f"case dirs {W}x{H}")
    w, sc = _scene("small_ramps")
    for pin in (False, True):
        lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, width=W, height=H,
                                        pinhole=pin, grid_dtype=torch.float32, device=dev)
        for yaw, pitch in [(0.0, 0.0), (123.0, -41.0), (-140.0, -33.0), (270.0, 60.0)]:
            got = lid.ray_dirs(torch.tensor([yaw]), torch.tensor([pitch]))[0].cpu().numpy()
            want = oracle.ray_dirs(W, H, yaw, pitch, pinhole=pin)
            assert np.abs(got - want).max() <= 1e-7, (pin, yaw, pitch)


def test_reference_ray_buffer_helpers(dev):
    """_ensure_buffers + _dirs_equiangular / _dirs_pinhole fill _dx/_dy/_dz
    the way the reference's camera tests read them (test_pinhole.py:36-41)."""
    W, H = 9, 5
    w, sc = _scene("small_ramps")
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, width=W, height=H,
                                    grid_dtype=torch.float32, device=dev)
    d2r = np.pi / 180.0
    for pin, f in ((False, lid._dirs_equiangular), (True, lid._dirs_pinhole)):
        lid._ensure_buffers(1)
        f(1, torch.tensor([123.0]), torch.tensor([-41.0]), d2r)
        got = torch.stack((lid._dx[0], lid._dy[0], lid._dz[0]), -1).cpu().numpy()
        want = oracle.ray_dirs(W, H, 123.0, -41.0, pinhole=pin)
        assert np.abs(got - want).max() <= 1e-7, pin
    with pytest.raises(ValueError, match="pi/180"):
        lid._dirs_equiangular(1, torch.tensor([0.0]), torch.tensor([0.0]), 1.0)


def test_pinhole_render_matches_the_oracle(dev):
    w, sc = _scene("small_ramps")
    ps = w.poses(sc)
    _say("case pinhole render")
    lid = _lidar(dev, w, sc, pinhole=True)
    got = _gpu_render(lid, ps, dev).cpu().numpy()
    want, _ = _oracle(w, sc, ps, pinhole=True)
    _assert_parity(got, want, w, "small_ramps/pinhole")


def test_closed_form_constant_field(dev):
    """Empty world: every ray runs to range in ceil(range/step) steps
    (vision.py:109-112), or keeps its partial t when steps run out."""
    _say("case constant field")
    g = np.full((8, 8, 8), 999.0, np.float32)
    step = np.float32(np.float32(999.0) * np.float32(0.9))
    for max_steps, rng, want_t in [(64, 2000.0, 2000.0), (2, 1e6, None), (0, 1e6, 0.0)]:
        lid = vision.GpuLidar.from_grid(g, np.zeros(3), 16.0, width=16, height=8,
                                        range_units=rng, max_steps=max_steps,
                                        grid_dtype=torch.float32, device=dev)
        out = lid.render(torch.tensor([[64.0, 64.0, 47.0]]), torch.tensor([10.0]),
                         torch.tensor([-5.0]), torch.tensor([0.0])).cpu().numpy()
        if want_t is None:
            want_t = np.float32(step + step)
        assert np.all(out == np.float32(want_t) / np.float32(rng)), (max_steps, out.ravel()[:3])


@pytest.mark.parametrize("max_steps,hit_eps,rng", [
    (0, 1.0, 1536.0), (1, 1.0, 1536.0), (2, 1.0, 1536.0), (3, -1.0, 1536.0),
    (64, 0.0, 1536.0), (64, 1.0, 0.0), (64, 1.0, -5.0), (64, -1.0, 300.0)])
def test_step_rule_corners_are_exact_in_every_schedule(dev, max_steps, hit_eps, rng):
    """The step rule at its edges (vision.py:100-112): no steps, the first
    step only (taken from the eye sample), a hit_eps that nothing reaches or
    that 0 distance does not pass, a range that ends every ray at t = 0 or
    that the march overshoots. Images and per-ray load counts equal the
    oracle's bit for bit in every schedule, both tile orders and on f16
    grids (slot packing)."""
    w, sc = _scene("small_ramps")
    n = 6
    ps = w.poses(sc, n)
    _say(f"case step corners max_steps={max_steps} hit_eps={hit_eps} range={rng}")
    kw = dict(range_units=rng, near_range=1000.0, max_steps=max_steps, hit_eps=hit_eps)
    for store, gdt in (("f32", torch.float32), ("f16", torch.float16)):
        want, want_taps = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch,
                                        ps.ducked, width=w.width, height=w.height, store=store,
                                        threads=8, **kw)
        lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, width=w.width,
                                        height=w.height, grid_dtype=gdt, device=dev, **kw)
        for sched, rpl, order in (("tiles", 2, "lookahead"), ("tiles", 2, "launch"),
                                  ("tiles", 1, "lookahead"), ("persistent", None, "launch")):
            lid.set_schedule(sched, rays_per_lane=rpl)
            lid.set_tile_order(order, min_tiles=0)
            taps = torch.full((n, w.height, w.width), -1, dtype=torch.int32, device=dev)
            got = torch.full((n, w.height, w.width), -1.0, device=dev)
            _gpu_render(lid, ps, dev, out=got, taps=taps)
            label = (store, sched, rpl, order)
            assert np.array_equal(got.cpu().numpy(), want), label
            assert np.array_equal(taps.cpu().numpy(), want_taps), label


@pytest.mark.parametrize("W,H,n", [(9, 5, 3), (33, 33, 2), (1, 1, 5), (20, 12, 7)])
def test_ragged_images_match_the_oracle(dev, W, H, n):
    """Image sizes that do not fill whole 16x4 tiles, and tiny N."""
    w, sc = _scene("small_ramps")
    ps = w.poses(sc, n)
    _say(f"case ragged {W}x{H} n={n}")
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, width=W, height=H,
                                    range_units=w.range_units, max_steps=w.max_steps,
                                    hit_eps=w.hit_eps, grid_dtype=torch.float32, device=dev)
    got = _gpu_render(lid, ps, dev).cpu().numpy()
    want, _ = _oracle(w, sc, ps, width=W, height=H)
    assert (np.abs(got - want) <= ENC_TOL).mean() >= 0.99


@pytest.mark.parametrize("refill,rpl", [(1, 1), (16, 2), (48, 2), (64, 1)])
def test_schedules_give_identical_results(dev, refill, rpl):
    """Persistent waves with ray refill and one-wave-per-tile launches march
    the same rays: outputs and censuses must be bit-identical, whatever the
    refill threshold."""
    w, sc = _scene("ramp_field")
    ps = w.poses(sc, 96)
    _say(f"case schedules refill={refill} rays_per_lane={rpl}")
    lid = _lidar(dev, w, sc)
    n = len(ps)
    lid.set_schedule("tiles", rays_per_lane=rpl)
    ta = torch.empty(n, w.height, w.width, dtype=torch.int32, device=dev)
    a = _gpu_render(lid, ps, dev, taps=ta)
    lid.set_schedule("persistent", refill)
    tb = torch.empty_like(ta)
    b = _gpu_render(lid, ps, dev, taps=tb)
    assert torch.equal(a, b)
    assert torch.equal(ta, tb)


def test_schedule_arguments_are_checked(dev):
    from surfgym import _sdfr
    w, sc = _scene("small_ramps")
    lid = _lidar(dev, w, sc)
    # by render size on a cache-resident grid: one ray per lane below 65536
    # tiles (512 envs of 128x64), two from there on
    assert lid.rays_per_lane is None
    assert [lid.effective_rays_per_lane(n) for n in (1, 16, 511, 512, 2048)] == [1, 1, 1, 2, 2]
    lid.set_schedule("tiles", rays_per_lane=2)
    assert lid.rays_per_lane == 2 and lid.effective_rays_per_lane(1) == 2
    with pytest.raises(_sdfr.SdfrError, match="rays_per_lane"):
        lid.set_schedule("tiles", rays_per_lane=3)
    with pytest.raises(_sdfr.SdfrError, match="rays_per_lane"):
        lid.set_schedule("tiles", rays_per_lane=-1)
    with pytest.raises(_sdfr.SdfrError, match="refill_lanes"):
        lid.set_schedule("persistent", refill_lanes=0)
    with pytest.raises(ValueError, match="schedule"):
        lid.set_schedule("bogus")
    with pytest.raises(ValueError, match="schedule"):
        lid.set_schedule("slots")      # the slot schedule measured slower and is gone
    lid.set_schedule("persistent", refill_lanes=8, rays_per_lane=2)
    assert (lid.schedule, lid.rays_per_lane) == ("persistent", 2)


@pytest.mark.parametrize("name,n,rpl", [("ramp_field", 256, None), ("ramp_field", 256, 2),
                                        ("winding_track", 64, None), ("small_ramps", 16, 2)])
def test_tile_order_is_a_permutation_and_changes_nothing(dev, name, n, rpl):
    """The lookahead tile order (default) sorts the tiles in runs of one
    workgroup's tiles (two waves x rays per lane); the sorted list in the
    workspace is a permutation of all runs, and images and censuses are
    bit-identical to env-order launches."""
    w, sc = _scene(name)
    ps = w.poses(sc, n)
    _say(f"case tile order {name} n={n} rpl={rpl}")
    lid = _lidar(dev, w, sc, rays_per_lane=rpl)
    assert lid.tile_order == "lookahead"
    lid.set_tile_order("lookahead", min_tiles=0)      # sort however small the render
    # a tile the sorted schedule never marched would keep these fills
    ta = torch.full((n, w.height, w.width), -1, dtype=torch.int32, device=dev)
    a = torch.full((n, w.height, w.width), -1.0, device=dev)
    _gpu_render(lid, ps, dev, taps=ta, out=a)
    torch.cuda.synchronize()
    tiles = n * (w.width // 8) * (w.height // 8)
    unit = 2 * lid.effective_rays_per_lane(n)
    units = (tiles + unit - 1) // unit
    rt_bytes = -(-(n * (w.width + w.height + 4) * 8) // 256) * 256
    perm = lid._ws[rt_bytes:rt_bytes + 4 * units].view(torch.int32).cpu().numpy()
    assert np.array_equal(np.sort(perm), np.arange(units))
    assert not np.array_equal(perm, np.arange(units))       # it did reorder
    lid.set_tile_order("launch")
    tb = torch.empty_like(ta)
    b = _gpu_render(lid, ps, dev, taps=tb)
    assert torch.equal(a, b)
    assert torch.equal(ta, tb)
    with pytest.raises(ValueError):
        lid.set_tile_order("zigzag")
    with pytest.raises(ValueError):
        lid.set_tile_order("lookahead", min_tiles=-2)


def test_small_renders_skip_the_sort_by_default(dev):
    """Below 65536 tiles the lookahead order leaves the sort out (its two
    launches cost more than they save); min_tiles moves the threshold."""
    w, sc = _scene("small_ramps")
    n = 16
    ps = w.poses(sc, n)
    _say("case tile order threshold")
    lid = _lidar(dev, w, sc)
    tiles = n * (w.width // 8) * (w.height // 8)
    rt_bytes = -(-(n * (w.width + w.height + 4) * 8) // 256) * 256
    want = _gpu_render(lid, ps, dev).clone()
    units = tiles // (2 * lid.effective_rays_per_lane(n))
    for min_tiles, sorted_ in ((None, False), (tiles + 1, False), (tiles, True), (0, True)):
        lid.set_tile_order("lookahead", min_tiles=min_tiles)
        lid._ws[rt_bytes:rt_bytes + 4 * units].fill_(255)       # perm slots read -1
        got = _gpu_render(lid, ps, dev)
        torch.cuda.synchronize()
        perm = lid._ws[rt_bytes:rt_bytes + 4 * units].view(torch.int32).cpu().numpy()
        assert torch.equal(got, want), min_tiles
        assert bool((perm >= 0).all()) == sorted_, min_tiles


def test_tile_order_with_pinhole_ragged_and_surf_mask(dev):
    w, sc = _scene("small_ramps")
    ps = w.poses(sc, 5)
    _say("case tile order variants")
    o, y = torch.as_tensor(ps.origin, device=dev), torch.as_tensor(ps.yaw, device=dev)
    p, d = torch.as_tensor(ps.pitch, device=dev), torch.as_tensor(ps.ducked, device=dev)
    snz = np.random.default_rng(3).integers(0, 128, sc.sdf.shape).astype(np.int8)
    # 37x19 and 8x8 over 5 envs leave quads of tiles partly (8x8: half)
    # outside the image: tiles without a pixel are ordered and marched as
    # empty, and every pixel must still be marched once
    for kw in (dict(pinhole=True, rays_per_lane=2), dict(width=37, height=19, rays_per_lane=2),
               dict(width=8, height=8, rays_per_lane=2),
               dict(width=37, height=19, rays_per_lane=1), dict(width=8, height=8, rays_per_lane=1),
               dict(surf_nz=snz, rays_per_lane=2), dict(surf_nz=snz)):
        kw.setdefault("width", w.width)
        kw.setdefault("height", w.height)
        lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, range_units=w.range_units,
                                        near_range=w.near_range, max_steps=w.max_steps,
                                        hit_eps=w.hit_eps, grid_dtype=torch.float32, device=dev,
                                        **kw)
        shape = (5, kw["height"], kw["width"]) + ((2,) if "surf_nz" in kw else ())
        lid.set_tile_order("lookahead", min_tiles=0)
        a = torch.full(shape, -1.0, device=dev)   # a tile never marched stays -1
        lid.render(o, y, p, d, out=a)
        lid.set_tile_order("launch")
        b = lid.render(o, y, p, d)
        assert torch.equal(a, b), sorted(kw)
        assert bool((b >= 0).all()) and bool((b <= 1.25).all()), sorted(kw)


def test_persistent_relaunches_reuse_their_counters(dev):
    """The persistent kernel's last wave clears its tile counters: renders
    of different sizes back to back on one handle must each be complete."""
    w, sc = _scene("small_ramps")
    ps = w.poses(sc)
    _say("case persistent relaunch")
    lid = _lidar(dev, w, sc)
    full = _gpu_render(lid, ps, dev)
    for n in (16, 3, 1, 16, 7):
        out = torch.full((n, w.height, w.width), -1.0, device=dev)
        lid.render(torch.as_tensor(ps.origin[:n], device=dev), torch.as_tensor(ps.yaw[:n], device=dev),
                   torch.as_tensor(ps.pitch[:n], device=dev), torch.as_tensor(ps.ducked[:n], device=dev),
                   out=out)
        assert torch.equal(out, full[:n]), n


@pytest.mark.parametrize("sort,grid_dtype,rpl", [(False, torch.float32, None),
                                                 (True, torch.float32, 2),
                                                 (True, torch.float16, 2)])
def test_render_inside_a_captured_graph(dev, sort, grid_dtype, rpl):
    """A hipGraph of one render replays correctly, again and again, with
    eager work between replays (the kernels clear their own counters: the
    persistent schedule's tile counters, the tile order's bucket counts)."""
    w, sc = _scene("small_ramps")
    ps = w.poses(sc)
    _say(f"case graph capture sort={sort} grid={grid_dtype} rpl={rpl}")
    lid = _lidar(dev, w, sc, grid_dtype=grid_dtype, rays_per_lane=rpl)
    if sort:
        lid.set_tile_order("lookahead", min_tiles=0)   # sort even this small batch
    origin = torch.as_tensor(ps.origin, device=dev)
    yaw = torch.as_tensor(ps.yaw, device=dev)
    pitch = torch.as_tensor(ps.pitch, device=dev)
    duck = torch.as_tensor(ps.ducked, device=dev)
    want = lid.render(origin, yaw, pitch, duck).clone()
    out = torch.empty_like(want)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        lid.render(origin, yaw, pitch, duck, out=out)     # warm up on the side stream
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lid.render(origin, yaw, pitch, duck, out=out)
    for i in range(4):
        out.fill_(-1.0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        # eager work between replays
        eager = lid.render(origin, yaw, pitch, duck)
        assert torch.equal(eager, want)
    # new poses copied into the captured inputs are rendered by the replay
    yaw.add_(30.0)
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, lid.render(origin, yaw, pitch, duck))


def test_ramp_field_full_batch_matches_the_oracle(dev):
    """The headline workload at its full size: 2048 envs x 128x64 rays."""
    w, sc = _scene("ramp_field")
    ps = w.poses(sc)
    _say(f"case ramp_field full envs={len(ps)}")
    lid = _lidar(dev, w, sc)
    taps = torch.empty(len(ps), w.height, w.width, dtype=torch.int32, device=dev)
    got = _gpu_render(lid, ps, dev, taps=taps)
    again = _gpu_render(lid, ps, dev)
    assert torch.equal(got, again), "two launches differ"
    want, loads = _oracle(w, sc, ps)
    ok = _assert_parity(got.cpu().numpy(), want, w, "ramp_field/full")
    t = taps.cpu().numpy()
    assert (t[ok] == loads[ok]).mean() > 0.999
    assert abs(int(t.sum()) - int(loads.sum())) <= 1e-4 * int(loads.sum())


def test_winding_track_matches_the_oracle(dev):
    """1 GiB grid (1024x1024x256 f32): gathers that miss the caches."""
    w, sc = _scene("winding_track")
    ps = w.poses(sc, 96)
    _say(f"case winding_track envs={len(ps)}")
    lid = _lidar(dev, w, sc)
    # a grid beyond the Infinity Cache: one tile per wave at any batch size
    assert lid.effective_rays_per_lane(len(ps)) == 1 and lid.effective_rays_per_lane(2048) == 1
    got = _gpu_render(lid, ps, dev).cpu().numpy()
    want, _ = _oracle(w, sc, ps)
    _assert_parity(got, want, w, "winding_track")


def test_sparse_grazing_matches_the_oracle(dev):
    """Near-horizontal views, 256-step cap: the long-tail workload."""
    w, sc = _scene("sparse_grazing")
    ps = w.poses(sc, 256)
    _say(f"case sparse_grazing envs={len(ps)}")
    lid = _lidar(dev, w, sc)
    for sched in ("tiles", "persistent"):
        lid.set_schedule(sched)
        got = _gpu_render(lid, ps, dev).cpu().numpy()
        want, _ = _oracle(w, sc, ps)
        _assert_parity(got, want, w, f"sparse_grazing/{sched}")


def test_f16_bricks_against_the_f32_oracle(dev):
    """f16 storage (the reference's device dtype) against the f32 grid.

    Rounding a stored distance to f16 (ulp 1 u at 1024-2048 u, 2 u above)
    changes step lengths, so a ray can stop one step earlier or later: on this
    analytic scene about 3% of rays move by more than 0.5 u and about 1% of
    encodings by more than 1e-3, while 99.9% stay within one voxel (16 u).
    The kernel itself is exact against the oracle on the f16-rounded grid
    (test_f16_store_matches_the_oracle_on_the_rounded_grid); this test pins
    the size of the storage effect so that a change to it is noticed."""
    w, sc = _scene("ramp_field_f16_bf16")
    ps = w.poses(sc, 256)
    _say(f"case f16 bricks vs f32 oracle envs={len(ps)}")
    lid = _lidar(dev, w, sc, grid_dtype=torch.float16)
    got = _gpu_render(lid, ps, dev).cpu().numpy()
    want, _ = _oracle(w, sc, ps, store="f32")
    d_enc = np.abs(got - want)
    d_u = np.abs(_depth(got, w.near_range, w.range_units) - _depth(want, w.near_range,
                                                                  w.range_units))
    _say(f"f16-vs-f32: enc<=1e-3 {float((d_enc <= ENC_TOL).mean()):.6f}, "
         f"depth<=0.5u {float((d_u <= DEPTH_TOL_U).mean()):.6f}, "
         f"depth<=16u {float((d_u <= 16.0).mean()):.6f}")
    assert (d_enc <= ENC_TOL).mean() >= 0.98
    assert (d_u <= 16.0).mean() >= 0.998


def test_march_events_time_the_march_alone(dev):
    """sdfr_grid_set_march_events: the library records the caller's two HIP
    events around each render's march kernel (bench.py's roofline figure)."""
    import ctypes
    w, sc = _scene("ramp_field")
    ps = w.poses(sc, 256)
    _say("case march events")
    lid = _lidar(dev, w, sc)
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                        ctypes.c_void_p]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    ev = [ctypes.c_void_p() for _ in range(2)]
    for e in ev:
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
    try:
        want = _gpu_render(lid, ps, dev)
        with pytest.raises(Exception):
            lid.set_march_events(ev[0].value, None)
        lid.set_march_events(ev[0].value, ev[1].value)
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        got = _gpu_render(lid, ps, dev)
        t1.record()
        torch.cuda.synchronize()
        ms = ctypes.c_float()
        assert hip.hipEventElapsedTime(ctypes.byref(ms), ev[0], ev[1]) == 0
        assert 0.0 < ms.value <= t0.elapsed_time(t1)
        assert torch.equal(got, want)
        lid.set_march_events(None, None)
        assert torch.equal(_gpu_render(lid, ps, dev), want)
    finally:
        torch.cuda.synchronize()
        for e in ev:
            hip.hipEventDestroy(e)


def test_two_lidars_on_two_streams_at_once(dev):
    """Handles share no state: two lidars (each with its own bucket counts,
    counters and workspace) rendering sorted batches on two streams at the
    same time give the images each gives alone."""
    w, sc = _scene("small_ramps")
    ps = w.poses(sc)
    _say("case two streams")
    lids = [_lidar(dev, w, sc), _lidar(dev, w, sc, schedule="persistent")]
    for lid in lids:
        lid.set_tile_order("lookahead", min_tiles=0)
    args = [torch.as_tensor(v, device=dev) for v in (ps.origin, ps.yaw, ps.pitch, ps.ducked)]
    shifted = [args[0], args[1] + 90.0, args[2], args[3]]
    want = [lids[0].render(*args).clone(), lids[1].render(*shifted).clone()]
    streams = [torch.cuda.Stream(device=dev) for _ in lids]
    outs = [torch.empty_like(want[0]) for _ in lids]
    torch.cuda.synchronize()
    for _ in range(8):
        for lid, st, a, o in zip(lids, streams, (args, shifted), outs):
            with torch.cuda.stream(st):
                o.fill_(-1.0)
                lid.render(*a, out=o)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], want[0]) and torch.equal(outs[1], want[1])


@pytest.mark.parametrize("name", ["winding_track", "sparse_grazing", "ramp_field_f16_bf16"])
def test_bench_configurations_are_bit_exact_at_full_size(dev, name):
    """Each bench.py workload at its full size and default schedule (tile
    order, rays per lane, occupancy cap, slot packing): every encoding equals
    the oracle's bit for bit (on the f16-rounded grid for the fp16 bricks,
    then rounded to bf16 as the bf16 output is)."""
    w, sc = _scene(name)
    ps = w.poses(sc)
    f16 = w.store == "f16"
    _say(f"case full-size {name} envs={len(ps)}")
    lid = _lidar(dev, w, sc, grid_dtype=torch.float16 if f16 else torch.float32)
    odt = torch.bfloat16 if w.out_dtype == "bf16" else torch.float32
    out = torch.empty(len(ps), 1, w.height, w.width, dtype=odt, device=dev)
    _gpu_render(lid, ps, dev, out=out)
    want, _ = _oracle(w, sc, ps, store=w.store)
    want_t = torch.as_tensor(want).reshape(out.shape).to(odt)
    got = out.cpu()
    exact = float((got == want_t).float().mean())
    _say(f"{name}: {got.numel()} rays, exact {exact:.6f}")
    assert torch.equal(got, want_t)


@pytest.mark.parametrize("variant", ["pinhole", "surf_mask"])
def test_variants_are_bit_exact_at_the_headline_size(dev, variant):
    """The two render variants at 2048 envs x 128x64 on ramp_field (sorted
    tiles, two rays per lane): every output equals the oracle's."""
    w, sc = _scene("ramp_field")
    ps = w.poses(sc)
    _say(f"case full-size variant {variant} envs={len(ps)}")
    kw, okw = {}, {}
    if variant == "pinhole":
        kw["pinhole"] = okw["pinhole"] = True
    else:
        snz = np.random.default_rng(11).integers(0, 128, sc.sdf.shape).astype(np.int8)
        kw["surf_nz"] = okw["surf_nz"] = snz
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, width=w.width, height=w.height,
                                    range_units=w.range_units, near_range=w.near_range,
                                    max_steps=w.max_steps, hit_eps=w.hit_eps,
                                    grid_dtype=torch.float32, device=dev, **kw)
    assert lid.effective_rays_per_lane(len(ps)) == 2
    got = _gpu_render(lid, ps, dev).cpu().numpy()
    want, _ = _oracle(w, sc, ps, **okw)
    assert got.shape == want.shape
    assert np.array_equal(got, want)


def test_a_batch_of_16384_envs_equals_its_halves(dev):
    """Batch independence beyond the bench sizes: 16384 envs x 128x64
    (268 M rays, 262144 sorted units, 1 GiB of output) render exactly as
    their two halves do apart."""
    w, sc = _scene("ramp_field")
    ps = w.poses(sc, 16384)
    _say("case 16384 envs")
    lid = _lidar(dev, w, sc)
    args = [torch.as_tensor(v, device=dev) for v in (ps.origin, ps.yaw, ps.pitch, ps.ducked)]
    full = lid.render(*args)
    h = 8192
    lo = lid.render(*[a[:h] for a in args])
    assert torch.equal(full[:h], lo)
    del lo
    hi = lid.render(*[a[h:] for a in args])
    assert torch.equal(full[h:], hi)
