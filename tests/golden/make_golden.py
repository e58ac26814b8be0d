"""Writes tests/golden/small_ramps_golden.npz: seeded inputs and the
oracle's outputs for a small render, as a fixture that pins both the oracle
(tests/test_golden.py, CPU) and the GPU renderer (tests/test_gpu_golden.py).

Inputs: the small_ramps scene (64x64x32 @16 u, plane + 8 ramps, seed 1000)
identified by the SHA-256 of its f32 grid, 3 poses from seed 2000, and a
seeded int8 surf-mask grid. Outputs: depth encodings (3,64,128) f32, grid
loads per ray, both channels with the mask, the pinhole depths, and the same
render over the f16-rounded grid.

The reference ships no numeric golden vectors for this path (its GPU test
compares two Triton kernels, tests/python/test_lidar_march.py:142-147), so
these are the oracle's own outputs, checked by tests/test_oracle.py.

Run from the repo root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
for p in (str(ROOT), str(ROOT / "rl_cs1.6_surf_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle                      # noqa: E402
from surfgym import synth          # noqa: E402

OUT = Path(__file__).resolve().parent / "small_ramps_golden.npz"


def inputs():
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, 3)
    snz = np.random.default_rng(11).integers(0, 128, sc.sdf.shape).astype(np.int8)
    return w, sc, ps, snz


def grid_sha(sdf) -> str:
    return hashlib.sha256(np.ascontiguousarray(sdf, np.float32).tobytes()).hexdigest()


def outputs(w, sc, ps, snz):
    kw = dict(range_units=w.range_units, near_range=w.near_range, hit_eps=w.hit_eps,
              max_steps=w.max_steps)
    args = (sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked)
    enc, loads = oracle.render(*args, **kw)
    both, _ = oracle.render(*args, surf_nz=snz, **kw)
    pin, _ = oracle.render(*args, pinhole=True, **kw)
    f16, f16_loads = oracle.render(*args, store="f16", **kw)
    return dict(enc=enc, loads=loads, surf=both, pinhole=pin, f16=f16, f16_loads=f16_loads)


def main():
    w, sc, ps, snz = inputs()
    out = outputs(w, sc, ps, snz)
    np.savez_compressed(OUT, grid_sha=np.str_(grid_sha(sc.sdf)), mins=sc.mins, cell=np.float32(sc.cell),
                        origin=ps.origin, yaw=ps.yaw, pitch=ps.pitch, ducked=ps.ducked,
                        surf_nz=snz, range_units=np.float32(w.range_units),
                        near_range=np.float32(w.near_range), hit_eps=np.float32(w.hit_eps),
                        max_steps=np.int32(w.max_steps), **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
