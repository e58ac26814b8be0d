"""The GPU renderer against the committed fixture
tests/golden/small_ramps_golden.npz (inputs and oracle outputs), bit for bit:
depth, load census, the surf-mask channels, the pinhole camera and an f16
grid."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from surfgym import vision

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))

import make_golden  # noqa: E402

pytestmark = pytest.mark.gpu


def test_gpu_matches_the_golden_fixture(dev):
    print("case golden fixture", flush=True)
    g = np.load(HERE / "golden" / "small_ramps_golden.npz", allow_pickle=False)
    w, sc, ps, snz = make_golden.inputs()
    assert make_golden.grid_sha(sc.sdf) == str(g["grid_sha"])
    poses = [torch.as_tensor(g[k], device=dev) for k in ("origin", "yaw", "pitch", "ducked")]
    kw = dict(range_units=float(g["range_units"]), near_range=float(g["near_range"]),
              hit_eps=float(g["hit_eps"]), max_steps=int(g["max_steps"]), device=dev)
    lid = vision.GpuLidar.from_grid(sc.sdf, g["mins"], float(g["cell"]), grid_dtype=torch.float32,
                                    **kw)
    taps = torch.empty(3, 64, 128, dtype=torch.int32, device=dev)
    assert np.array_equal(lid.render(*poses, taps=taps).cpu().numpy(), g["enc"])
    assert np.array_equal(taps.cpu().numpy(), g["loads"])
    lid_m = vision.GpuLidar.from_grid(sc.sdf, g["mins"], float(g["cell"]), surf_nz=g["surf_nz"],
                                      grid_dtype=torch.float32, **kw)
    assert np.array_equal(lid_m.render(*poses).cpu().numpy(), g["surf"])
    lid_p = vision.GpuLidar.from_grid(sc.sdf, g["mins"], float(g["cell"]), pinhole=True,
                                      grid_dtype=torch.float32, **kw)
    assert np.array_equal(lid_p.render(*poses).cpu().numpy(), g["pinhole"])
    lid_h = vision.GpuLidar.from_grid(sc.sdf, g["mins"], float(g["cell"]), grid_dtype=torch.float16,
                                      **kw)
    assert np.array_equal(lid_h.render(*poses, taps=taps).cpu().numpy(), g["f16"])
    assert np.array_equal(taps.cpu().numpy(), g["f16_loads"])
    # the same at two rays per lane (these 3 envs render at one by default;
    # fp16 bricks then also pack slots)
    for lid_x in (lid, lid_m, lid_p, lid_h):
        lid_x.set_schedule("tiles", rays_per_lane=2)
    assert np.array_equal(lid.render(*poses, taps=taps).cpu().numpy(), g["enc"])
    assert np.array_equal(taps.cpu().numpy(), g["loads"])
    assert np.array_equal(lid_m.render(*poses).cpu().numpy(), g["surf"])
    assert np.array_equal(lid_p.render(*poses).cpu().numpy(), g["pinhole"])
    assert np.array_equal(lid_h.render(*poses, taps=taps).cpu().numpy(), g["f16"])
    assert np.array_equal(taps.cpu().numpy(), g["f16_loads"])
