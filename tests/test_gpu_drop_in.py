"""The trainer's own render sequence, end to end on the GPU, through the
install hook.

A stand-in of the reference's ``surfgym`` package (the layout of
tests/test_drop_in.py) and a map core of boxes sit in tmp_path. A script
that imports the way python/train_fast.py does (:58-76) runs under
``surfgym_mi355x.py``, constructs the lidar exactly as the trainer does
(train_fast.py:1461-1465: the map core, default grid dtype, no SDF cache yet,
so build_sdf bakes one on the GPU and writes it), fills a pinned (N,6) pose
block, copies it to the device and renders strided columns of it into the
image slice of an observation row (train_fast.py:1744-1760). The image slice
must equal the oracle's render of the cached grid as the default store holds
it (fp16) bit for bit.
"""
from __future__ import annotations

import json
import subprocess
import sys
import textwrap
from pathlib import Path

import numpy as np
import pytest

import oracle
from test_drop_in import _write_stand_in

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "rl_cs1.6_surf_amd"
TESTS = ROOT / "tests"

N, W, H = 48, 128, 64
RANGE, NEAR, CELL = 3000.0, 2000.0, 16.0
BOXES = [((0, 0, 0), (1024, 1024, 32)), ((200, 300, 32), (420, 380, 260)),
         ((600, 100, 32), (700, 900, 140)), ((300, 700, 200), (900, 760, 230))]
BOUNDS = ((0, 0, 0), (1024, 1024, 512))


def _poses():
    rng = np.random.default_rng(41)
    o = np.stack([rng.uniform(50, 974, N), rng.uniform(50, 974, N),
                  rng.uniform(300, 420, N)], 1).astype(np.float32)
    yaw = rng.uniform(0, 360, N).astype(np.float32)
    pitch = rng.uniform(-70, 30, N).astype(np.float32)
    duck = (rng.random(N) < 0.5).astype(np.float32)
    return o, yaw, pitch, duck


_SCRIPT = """
    import json
    import sys
    from pathlib import Path
    ROOT = Path(__file__).resolve().parent.parent
    sys.path.insert(0, str(ROOT / "python"))
    import numpy as np
    import torch
    from surfgym import SurfCore, default_config
    from surfgym.goalfield import build_goal_field
    from surfgym.vision import GpuLidar, pick_cell
    sys.path.insert(1, {tests!r})
    from test_drop_in import _Core

    core = _Core({bsp!r}, {boxes!r}, {bounds!r})
    device = torch.device("cuda")
    lidar = GpuLidar(core, {W}, {H},
                     range_units={rng}, near_range={near},
                     cell=(None or pick_cell(core)),
                     device=device, surf_mask=False,
                     pinhole=False)
    poses = np.load({poses!r})
    n = poses.shape[0]
    vis_pin = torch.empty((n, 6), dtype=torch.float32, pin_memory=True)
    vis_np = vis_pin.numpy()
    vis_gpu = torch.empty((n, 6), dtype=torch.float32, device=device)
    static_obs = torch.zeros((n, 15 + {W} * {H} * lidar.channels), device=device)
    vis_np[:, 0:3] = poses[:, 0:3]
    vis_np[:, 3] = poses[:, 3]
    vis_np[:, 4] = poses[:, 4]
    vis_np[:, 5] = poses[:, 5]
    vis_gpu.copy_(vis_pin, non_blocking=True)
    img = lidar.render(vis_gpu[:, 0:3], vis_gpu[:, 3],
                       vis_gpu[:, 4], vis_gpu[:, 5])
    static_obs[:, 15:].copy_(img.reshape(n, -1))
    np.save({out!r}, static_obs.cpu().numpy())
    print(json.dumps({{"GpuLidar": sys.modules[GpuLidar.__module__].__file__,
                      "cell": lidar.cell, "grid_dtype": str(lidar.grid_dtype),
                      "channels": lidar.channels}}))
"""


def test_the_trainers_render_sequence_through_the_hook(dev, tmp_path):
    _write_stand_in(tmp_path)
    bsp = tmp_path / "surf_e2e.bsp"
    bsp.write_bytes(b"BSP" * 64)
    o, yaw, pitch, duck = _poses()
    poses = tmp_path / "poses.npy"
    np.save(poses, np.concatenate([o, yaw[:, None], pitch[:, None], duck[:, None]], 1))
    out = tmp_path / "obs.npy"
    script = tmp_path / "python" / "train_gpu.py"
    script.write_text(textwrap.dedent(_SCRIPT.format(
        tests=str(TESTS), bsp=str(bsp), boxes=BOXES, bounds=BOUNDS, W=W, H=H, rng=RANGE,
        near=NEAR, poses=str(poses), out=str(out))))
    print("case drop-in: the trainer's render sequence through the hook", flush=True)
    r = subprocess.run([sys.executable, str(PKG / "surfgym_mi355x.py"), str(script)],
                       capture_output=True, text=True, timeout=240, cwd=str(tmp_path))
    assert r.returncode == 0, r.stderr[-3000:]
    got = json.loads(r.stdout.strip().splitlines()[-1])
    assert Path(got["GpuLidar"]) == PKG / "surfgym" / "vision.py"
    assert got["cell"] == CELL and got["grid_dtype"] == "torch.float16" and got["channels"] == 1
    # the SDF the constructor baked and cached (build_sdf on a miss)
    z = np.load(tmp_path / "surf_e2e.sdf_16.npz", allow_pickle=False)
    sdf, mins = z["sdf"], z["mins"]
    want, _ = oracle.render(sdf, mins, CELL, o, yaw, pitch, duck, width=W, height=H,
                            range_units=RANGE, near_range=NEAR, store="f16")
    obs = np.load(out)
    assert obs.shape == (N, 15 + W * H)
    assert not obs[:, :15].any()
    assert np.array_equal(obs[:, 15:].reshape(N, H, W), want)
    # the baked map is closed (build_sdf pads a solid shell), so every ray
    # ends on a surface; the images are not degenerate
    assert np.unique(want).size > 5000 and want.std() > 0.05
