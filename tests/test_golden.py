"""The committed fixture tests/golden/small_ramps_golden.npz against a fresh
oracle run: the synthetic scene must still hash to the same grid, and the
oracle must reproduce every stored output bit for bit."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))

import make_golden  # noqa: E402


def test_oracle_reproduces_the_golden_fixture():
    g = np.load(HERE / "golden" / "small_ramps_golden.npz", allow_pickle=False)
    w, sc, ps, snz = make_golden.inputs()
    assert make_golden.grid_sha(sc.sdf) == str(g["grid_sha"]), "the synthetic scene changed"
    assert np.array_equal(ps.origin, g["origin"]) and np.array_equal(ps.yaw, g["yaw"])
    assert np.array_equal(snz, g["surf_nz"])
    out = make_golden.outputs(w, sc, ps, snz)
    for k, v in out.items():
        assert np.array_equal(v, g[k]), k
