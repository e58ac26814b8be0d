"""Pins oracle/lockstep.py, the torch restatement of the reference's CPU
render (python/surfgym/vision.py:596-666) that bench.py times as the CPU
baseline.

It is checked against the per-ray C oracle (oracle/march.c, pinned by
tests/test_oracle.py): the two are written independently (lockstep over all
rays with torch's vector cos/sin/exp, against a per-ray loop with
correctly-rounded fp64 transcendentals), so an error in either one's step
rule, index order, eye height or encoding shows up as disagreement. They
may differ only where torch's vector sin/cos round the last bit differently;
oracle/agreement.py measures and classifies those differences at the north
star's tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import agreement, lockstep
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
    assert exact >= 0.999, exact


def _agreement(name, n, *, yaw_shift=0.0, corrupt=0):
    """The oracle's render against the lockstep render of the same poses
    (the reference's CPU arithmetic), classified by oracle.agreement. The
    planted mistakes go into the CPU side: ``yaw_shift`` degrees added to the
    lockstep's yaw, ``corrupt`` pixels of the oracle's image set to 0.4321."""
    w = synth.WORKLOADS[name]
    sc = w.scene()
    ps = w.poses(sc, n)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps)
    keep = {}
    ref = lockstep.render(sc.sdf, sc.mins, sc.cell, ps.origin,
                          np.asarray(ps.yaw, np.float32) + np.float32(yaw_shift), ps.pitch,
                          ps.ducked, keep=keep, **kw)
    img, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                           threads=8, **kw)
    if corrupt:
        flat = img.reshape(-1)
        flat[np.random.default_rng(7).choice(flat.size, corrupt, replace=False)] = 0.4321
    return agreement.compare(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                             img, ref, keep, list_max=None, **kw)


def test_agreement_with_the_reference_arithmetic_at_256_envs():
    """The accuracy bar against the reference's own CPU arithmetic
    (torch's cos/sin/exp, vision.py:596-657) on 256 ramp_field envs (2.1 M
    rays): >= 99.9% of rays within 0.5 u and 1e-3, and every ray outside
    that is classified — a grazing hit, or two hits of the same surface one
    step of the march apart — none left unexplained. The oracle's image
    stands for the renderer's (the GPU tests show them bit-identical); each
    outlier's re-trace reproduces both sides' depths exactly."""
    a = _agreement("ramp_field", 256)
    assert a["rays"] == 256 * 64 * 128
    assert a["within_tol"] >= 0.999, a
    assert a["exact"] >= 0.999, a
    assert a["renderer_differs"] == 0 and a["ref_retrace_differs"] == 0, a
    assert a["outliers"] == len(a["listed"])
    assert a["outliers"] == a["outliers_grazing"] + a["outliers_step_phase"]
    assert a["outliers_other"] == a["outliers_tie_other"] == 0, a
    for o in a["listed"]:
        assert o["stop"] == o["stop_ref"] == "hit", o
        if o["class"] == "step_phase":
            assert abs(o["depth"] - o["depth_ref"]) <= o["last_step_u"], o
        else:
            assert o["angle_deg"] > agreement.GRAZING_DEG, o
        # the two marches part at a sample within float rounding of a voxel face
        assert o["split_face_u"] is not None and o["split_face_u"] <= agreement.TIE_U, o


def test_agreement_flags_a_planted_direction_error():
    """A reference rendered 0.5 degree off in yaw (a planted mistake) fails
    the bar by far, and its outliers are not explained away: most part from
    the true march at samples far from any voxel face, or hit elsewhere
    (class "other")."""
    a = _agreement("small_ramps", 8, yaw_shift=0.5)
    assert a["within_tol"] < 0.99, a
    assert a["outliers_other"] > 0.5 * a["outliers"], a


def test_agreement_flags_an_image_that_is_not_the_oracles():
    """Pixels of the image planted at a wrong value are re-traced, found to
    differ from the oracle's march, and counted."""
    a = _agreement("small_ramps", 4, corrupt=50)
    assert a["renderer_differs"] == 50, a


def test_normal_angle_of_a_floor_and_a_wall():
    """The grazing angle is the angle between the ray and the grid's
    central-difference gradient: a ray meeting a floor (distance = height
    above it) at 80 degrees from the vertical reads 80, and a wall across x
    (distance = how far short of it) at 30 degrees from its normal reads 30."""
    cell = 16.0
    n = 32
    c = (np.arange(n) + 0.5) * cell
    floor = np.broadcast_to(np.maximum(c - 8 * cell, 0.0)[:, None, None], (n, n, n))
    wall = np.broadcast_to(np.maximum(20 * cell - c, 0.0)[None, None, :], (n, n, n))
    kw = dict(range_units=4000.0, hit_eps=1.0, min_step=4.8, max_steps=400)
    th = np.radians(80.0)
    d = np.array([np.sin(th), 0.0, -np.cos(th)], np.float32)
    tr = agreement.trace(np.ascontiguousarray(floor, np.float32), np.zeros(3), cell,
                         (40.0, 250.0, 200.0), d, **kw)
    assert tr["why"] == "hit"
    assert abs(agreement._normal_angle(np.asarray(floor, np.float32), tr, d) - 80.0) < 0.01
    th = np.radians(30.0)
    d = np.array([np.cos(th), np.sin(th), 0.0], np.float32)
    tr = agreement.trace(np.ascontiguousarray(wall, np.float32), np.zeros(3), cell,
                         (100.0, 40.0, 250.0), d, **kw)
    assert tr["why"] == "hit"
    assert abs(agreement._normal_angle(np.asarray(wall, np.float32), tr, d) - 30.0) < 0.01


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


def _nz_code_grid(sdf):
    """|n_z| * 127 of the grid's own central-difference gradient, int8: the
    kind of grid the surf-mask channel reads (its bake is the reference's)."""
    gz = np.gradient(sdf, axis=0)
    gy = np.gradient(sdf, axis=1)
    gx = np.gradient(sdf, axis=2)
    nrm = np.sqrt(gx * gx + gy * gy + gz * gz)
    return np.where(nrm > 0, np.rint(np.abs(gz) / np.maximum(nrm, 1e-9) * 127), 0).astype(np.int8)


def _variant(n, **extra):
    w = synth.WORKLOADS["ramp_field"]
    sc = w.scene()
    ps = w.poses(sc, n)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps)
    keep = {}
    ref = lockstep.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                          keep=keep, **kw, **extra)
    img, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                           threads=8, **kw, **extra)
    return agreement.compare(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                             img, ref, keep, list_max=None, **kw, **extra)


def test_pinhole_agreement_with_the_reference_arithmetic():
    """The pinhole camera through torch's CPU kernels (``_dirs_pinhole``,
    vision.py:609-624: cos/sin of the view, the tangent-plane sum, rsqrt)
    against the oracle's correctly rounded directions, 256 ramp_field envs:
    the same bar, every outlier explained."""
    a = _variant(256, pinhole=True)
    assert a["within_tol"] >= 0.999 and a["exact"] >= 0.999, a
    assert a["renderer_differs"] == 0 and a["ref_retrace_differs"] == 0, a
    assert a["outliers_other"] == 0 and a["outliers"] == len(a["listed"]), a


def test_surf_channel_agreement_with_the_reference_arithmetic():
    """The surf-mask channel (the |n_z| code of the voxel under the clamped
    depth over 127, vision.py:658-666) against the lockstep's: on 256
    ramp_field envs with a gradient-derived |n_z| grid every channel value
    whose depth agrees is equal, and the depth channel meets the bar. A
    reference that divided by 128 (a planted slip) differs on most rays with
    a nonzero code, none of them explained by a voxel-face tie."""
    w = synth.WORKLOADS["ramp_field"]
    snz = _nz_code_grid(w.scene().sdf)
    a = _variant(256, surf_nz=snz)
    assert a["within_tol"] >= 0.999, a
    assert a["renderer_differs"] == 0 and a["ref_retrace_differs"] == 0, a
    assert a["surf_other"] == 0 and a["outliers_other"] == 0, a
    assert a["surf_differs"] == a["surf_with_depth_outlier"] + a["surf_tie"], a
    # the planted slip: the lockstep's channel scaled by 127/128
    sc = w.scene()
    ps = w.poses(sc, 4)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps)
    keep = {}
    ref = lockstep.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                          keep=keep, surf_nz=snz, **kw)
    ref[..., 1] = (ref[..., 1] * np.float32(127.0) / np.float32(128.0)).astype(np.float32)
    img, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                           surf_nz=snz, threads=8, **kw)
    b = agreement.compare(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                          img, ref, keep, surf_nz=snz, **kw)
    nonzero = int((img[..., 1] != 0).sum())
    assert b["surf_differs"] > 0.9 * nonzero and b["surf_other"] > 0.9 * nonzero, b


def test_lockstep_variants_agree_with_the_per_ray_oracle():
    """The lockstep's pinhole and surf-mask renders against the oracle's on
    small_ramps: bit-identical on at least 99.9% of rays."""
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, 16)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps)
    for extra in (dict(pinhole=True), dict(surf_nz=_nz_code_grid(sc.sdf))):
        a = lockstep.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                            **kw, **extra)
        b, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                             threads=8, **kw, **extra)
        assert a.shape == b.shape
        assert float((a == b).mean()) >= 0.999, extra.keys()
