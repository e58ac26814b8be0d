"""Pins oracle/lockstep.py, the torch restatement of the reference's CPU
render (python/surfgym/vision.py:596-666) that bench.py times as the CPU
baseline.

It is checked against the per-ray C oracle (oracle/march.c, pinned by
tests/test_oracle.py): the two are written independently (lockstep over all
rays with torch's vector cos/sin/exp, against a per-ray loop with
correctly-rounded fp64 transcendentals), so an error in either one's step
rule, index order, eye height or encoding shows up as disagreement. They
may differ only where torch's vector sin/cos round the last bit differently.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import lockstep
from surfgym import synth


def _both(name, n, **over):
    w = synth.WORKLOADS[name]
    sc = w.scene()
    ps = w.poses(sc, n)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps)
    kw.update(over)
    a = lockstep.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked, **kw)
    b, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                         threads=8, **kw)
    return a, b


@pytest.mark.parametrize("name,n", [("small_ramps", 16), ("ramp_field", 24)])
def test_lockstep_agrees_with_the_per_ray_oracle(name, n):
    a, b = _both(name, n)
    assert a.shape == b.shape and a.dtype == np.float32
    exact = float((a == b).mean())
    close = float((np.abs(a - b) <= 1e-3).mean())
    assert exact >= 0.999, exact
    assert close == 1.0, close


def test_lockstep_early_exit_changes_nothing():
    """The every-8-steps host any() exit (vision.py:651-653) is exact: rays
    that end before the step cap (per the oracle's load count) render the
    same under a cap of 64 and of 4096, and the capped ones only go further."""
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, 4)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, hit_eps=w.hit_eps)
    a = lockstep.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                        max_steps=64, **kw)
    b = lockstep.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                        max_steps=4096, **kw)
    _, loads = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                             max_steps=64, threads=8, **kw)
    ended = loads < 64
    assert 0.5 < ended.mean() < 1.0
    assert np.array_equal(a[ended], b[ended])
    assert np.all(b[~ended] >= a[~ended])


def test_lockstep_chunking_is_exact():
    """Envs are processed in chunks; the chunk size must not matter."""
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, 7)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps)
    a = lockstep.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                        env_chunk=64, **kw)
    b = lockstep.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                        env_chunk=3, **kw)
    assert np.array_equal(a, b)


def test_a_planted_mistake_in_the_lockstep_is_caught():
    """The comparison above is sharp enough: swapping the eye heights (a
    plausible slip) in a copy of the inputs moves far more than 0.1% of rays."""
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, 8)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps)
    flipped = 1.0 - (np.asarray(ps.ducked) != 0)
    a = lockstep.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, flipped, **kw)
    b, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                         threads=8, **kw)
    assert float((a == b).mean()) < 0.99
