"""The on-device SDF bake (sdfr_edt) against the reference's bake, i.e.
scipy.ndimage.distance_transform_edt on the solid-padded occupancy
(python/surfgym/vision.py:428-438; oracle/edt.py), bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import edt
from surfgym import synth, vision

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(6))
def test_random_occupancy_matches_scipy(dev, seed):
    rng = np.random.default_rng(100 + seed)
    shp = tuple(int(v) for v in rng.integers(1, 70, 3))
    occ = (rng.random(shp) < rng.uniform(0.0, 0.2)).astype(np.uint8)
    cell = (16.0, 32.0, 8.0)[seed % 3]
    print(f"case edt random shape={shp} cell={cell}", flush=True)
    ref = edt.bake(occ, cell)
    got = vision.sdf_from_occupancy(occ, cell, device=dev, dtype=torch.float32).cpu().numpy()
    assert np.array_equal(got, ref.astype(np.float32))
    got16 = vision.sdf_from_occupancy(occ, cell, device=dev, dtype=torch.float16).cpu().numpy()
    assert np.array_equal(got16, ref.astype(np.float16))


def test_empty_and_full_grids(dev):
    print("case edt empty/full", flush=True)
    for occ in (np.zeros((5, 7, 9), np.uint8), np.ones((5, 7, 9), np.uint8),
                np.zeros((1, 1, 1), np.uint8), np.zeros((40, 1, 3), np.uint8)):
        ref = edt.bake(occ, 16.0)
        got = vision.sdf_from_occupancy(occ, 16.0, device=dev).cpu().numpy()
        assert np.array_equal(got, ref.astype(np.float32)), occ.shape


@pytest.mark.parametrize("shape", [(64, 512, 512), (256, 32, 512)])
def test_both_pass_algorithms_match_scipy(dev, shape):
    """Each of the y and z passes walks the parabola envelope when it has
    many lines and searches a window per output when it has few (the switch
    is at 512 lines per CU: 131,072 on 256 CUs). (64, 512, 512): y by window
    (32,768 lines), z by envelope (262,144); (256, 32, 512): y by envelope
    (131,072), z by window (16,384). Both equal scipy bit for bit."""
    rng = np.random.default_rng(sum(shape))
    occ = (rng.random(shape) < 0.002).astype(np.uint8)
    occ[:, :, : shape[2] // 8] |= (rng.random((shape[0], shape[1], 1)) < 0.3).astype(np.uint8)
    print(f"case edt both algorithms {shape}", flush=True)
    ref = edt.bake(occ, 16.0).astype(np.float32)
    got = vision.sdf_from_occupancy(occ, 16.0, device=dev, dtype=torch.float32).cpu().numpy()
    assert np.array_equal(got, ref)


def test_scene_occupancy_matches_scipy_and_renders(dev):
    """The ramp_field scene's solids (256x256x128, 8.4 M voxels): baked on the
    GPU, equal to scipy's bake, and renderable as is."""
    w = synth.WORKLOADS["ramp_field"]
    sc = w.scene()
    occ = (sc.sdf == 0).astype(np.uint8)
    print(f"case edt ramp_field {occ.shape}", flush=True)
    got = vision.sdf_from_occupancy(occ, sc.cell, device=dev)
    ref = edt.stored(edt.bake(occ, sc.cell))
    assert got.dtype == torch.float32
    assert np.array_equal(got.cpu().numpy(), ref)
    lid = vision.GpuLidar.from_grid(got.cpu().numpy(), sc.mins, sc.cell, grid_dtype=torch.float32,
                                    device=dev)
    ps = w.poses(sc, 4)
    img = lid.render(torch.as_tensor(ps.origin, device=dev), torch.as_tensor(ps.yaw, device=dev),
                     torch.as_tensor(ps.pitch, device=dev), torch.as_tensor(ps.ducked, device=dev))
    assert torch.isfinite(img).all() and img.min() >= 0


def test_build_sdf_bakes_a_map_on_the_gpu_and_caches_it(dev, tmp_path, monkeypatch):
    """build_sdf on a map without a cache (vision.py:409-439): the slab
    occupancy, sampled through the map core, baked on the GPU; the npz it
    writes equals the reference's scipy bake of that occupancy bit for bit,
    and a second call loads it without baking."""
    import sys
    from test_drop_in import _Core, _zones_module
    bsp = tmp_path / "surf_g.bsp"
    bsp.write_bytes(b"BSP" * 50)
    core = _Core(bsp, [((0, 0, 0), (512, 384, 40)), ((100, 50, 40), (300, 90, 140)),
                       ((0, 0, 200), (512, 384, 203))], ((0, 0, 0), (512, 384, 256)))
    monkeypatch.setitem(sys.modules, "surfgym.zones", _zones_module(
        [{"classname": "func_wall", "model": "*1"}], [None, ((400.0, 0.0, 0.0),
                                                             (401.0, 300.0, 120.0))]))
    print("case build_sdf GPU bake", flush=True)
    sdf, mins, cell = vision.build_sdf(core, 16.0, device=dev)
    occ, omins = vision.slab_occupancy(core, 16.0)
    want = edt.stored(edt.bake(occ, 16.0))
    assert sdf.dtype == want.dtype and np.array_equal(sdf, want)
    z = np.load(tmp_path / "surf_g.sdf_16.npz", allow_pickle=False)
    assert np.array_equal(z["sdf"], want) and np.array_equal(z["mins"], omins.astype(np.float32))
    assert float(z["cell"]) == 16.0

    def no_bake(*a, **k):
        raise AssertionError("a current cache must not be baked again")

    monkeypatch.setattr(vision, "sdf_from_occupancy", no_bake)
    again, _, _ = vision.build_sdf(core, 16.0, device=dev)
    assert np.array_equal(again, want)
