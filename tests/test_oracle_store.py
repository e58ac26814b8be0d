"""Pins the oracle's r16 brick store (oracle.r16_encode / r16_decode).

r16 is this renderer's 2-byte grid store (no reference counterpart): per
4x4x4 brick an fp32 base (the brick's smallest value), a power-of-two scale
2^e and 64 uint16 codes. The checks below come from outside the vectorised
code: a per-brick loop written with Python's own math (frexp, round-half-even
``round``), known answers at the exponent's boundaries, the error bound the
format promises, exact round trips for representable grids, and what the
format does to the march on a real scene.
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "rl_cs1.6_surf_amd"))


def _brute(grid):
    """Per-brick loop: the format stated once more, scalar by scalar."""
    g = np.asarray(grid, np.float32)
    nz, ny, nx = g.shape
    out = np.empty_like(g)
    exps = {}
    for bz in range(0, nz, 4):
        for by in range(0, ny, 4):
            for bx in range(0, nx, 4):
                vals = [float(g[z, y, x]) for z in range(bz, min(bz + 4, nz))
                        for y in range(by, min(by + 4, ny)) for x in range(bx, min(bx + 4, nx))]
                lo, hi = min(vals), max(vals)
                rng = hi - lo
                if rng > 0:
                    m, ex = math.frexp(rng)
                    e = ex - 1 - 15
                    if rng / 2.0 ** e > 65535:
                        e += 1
                    e = max(-100, min(100, e))
                else:
                    e = -100
                exps[(bz // 4, by // 4, bx // 4)] = e
                scale = np.float32(2.0 ** e)
                for z in range(bz, min(bz + 4, nz)):
                    for y in range(by, min(by + 4, ny)):
                        for x in range(bx, min(bx + 4, nx)):
                            q = round((float(g[z, y, x]) - lo) / 2.0 ** e)
                            q = min(max(q, 0), 65535)
                            out[z, y, x] = np.float32(np.float32(lo) + np.float32(q) * scale)
    return out, exps


@pytest.mark.parametrize("shape,seed,spread", [((5, 7, 9), 0, 80.0), ((4, 4, 4), 1, 1e-3),
                                               ((9, 3, 6), 2, 3000.0), ((1, 1, 1), 3, 5.0)])
def test_r16_equals_a_per_brick_loop(shape, seed, spread):
    rng = np.random.default_rng(seed)
    g = (rng.random(shape) * spread - 0.25 * spread).astype(np.float32)
    g[0, 0, 0] = g.flat[-1]                   # a repeated value
    want, exps = _brute(g)
    got = oracle.as_stored(g, "r16")
    assert got.dtype == np.float32 and got.shape == g.shape
    assert np.array_equal(got, want)
    _, _, e = oracle.r16_encode(g)
    for (bz, by, bx), ev in exps.items():
        assert e[bz, by, bx] == ev


@pytest.mark.parametrize("top,want_e", [(100.0, -9), (65535.0 * 2.0 ** -9, -9),
                                        (127.999, -8), (128.0, -8), (65535.0, 0),
                                        (65536.0, 1), (0.0, -100), (2.0 ** -90, -100)])
def test_r16_exponent_boundaries(top, want_e):
    """One brick holding 0 and `top`: the smallest e with top <= 65535*2^e
    (never below -100)."""
    g = np.zeros((4, 4, 4), np.float32)
    g[3, 3, 3] = np.float32(top)
    codes, base, e = oracle.r16_encode(g)
    assert base[0, 0, 0] == 0.0
    assert int(e[0, 0, 0]) == want_e
    assert 0 <= int(codes.max()) <= 65535


def test_r16_error_bound_and_exact_minimum():
    """|decoded - value| <= 2^(e-1) plus one fp32 rounding of the sum, and
    each brick's smallest value comes back exactly (code 0)."""
    rng = np.random.default_rng(7)
    g = (rng.random((13, 10, 11)) * 1500.0).astype(np.float32)
    codes, base, e = oracle.r16_encode(g)
    d = oracle.as_stored(g, "r16")
    ev = np.repeat(np.repeat(np.repeat(e, 4, 0), 4, 1), 4, 2)[:13, :10, :11]
    bound = np.ldexp(1.0, ev - 1) + np.spacing(np.abs(g)).astype(np.float64)
    assert np.all(np.abs(d.astype(np.float64) - g) <= bound)
    mins = np.repeat(np.repeat(np.repeat(base, 4, 0), 4, 1), 4, 2)[:13, :10, :11]
    at_min = g == mins
    assert at_min.sum() >= base.size and np.array_equal(d[at_min], g[at_min])


def test_r16_is_exact_on_representable_grids():
    """Integers spanning less than 65536 per brick (scale <= 1) and
    multiples of 2^-9 spanning less than 128 come back bit for bit."""
    rng = np.random.default_rng(3)
    a = rng.integers(0, 60000, (8, 8, 8)).astype(np.float32)
    assert np.array_equal(oracle.as_stored(a, "r16"), a)
    b = (rng.integers(0, 60000, (6, 9, 5)) * 2.0 ** -9 + 1000.0).astype(np.float32)
    assert np.array_equal(oracle.as_stored(b, "r16"), b)


def test_r16_inner_order_is_x_fastest():
    """A planted gradient along one axis at a time survives the brick
    transposes: each axis' values come back at that axis' positions."""
    for axis in range(3):
        shape = [6, 7, 5]
        ramp = np.arange(shape[axis], dtype=np.float32) * 3.0
        g = np.broadcast_to(np.expand_dims(ramp, [a for a in range(3) if a != axis]),
                            shape).astype(np.float32)
        assert np.array_equal(oracle.as_stored(g, "r16"), g), axis


def test_r16_on_a_distance_field_is_within_a_thousandth():
    """A distance field changes by at most 3*sqrt(3)*cell across a brick
    (83 u at 16 u cells), so e <= -9 and the error stays below 2^-10 u."""
    from surfgym import synth
    sc = synth.WORKLOADS["ramp_field"].scene()
    _, _, e = oracle.r16_encode(sc.sdf)
    assert int(e.max()) <= -9
    d = oracle.as_stored(sc.sdf, "r16")
    assert float(np.abs(d - sc.sdf).max()) <= 2.0 ** -10


def test_r16_meets_the_render_tolerance_where_f16_does_not():
    """Through the oracle's march on the ramp_field scene (64 envs): the r16
    grid leaves >= 99.9% of rays within 0.5 u and 1e-3 of the fp32 grid's
    encodings; the fp16 grid (the reference's device dtype) does not."""
    from surfgym import synth
    w = synth.WORKLOADS["ramp_field"]
    sc = w.scene()
    ps = w.poses(sc, 64)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps, threads=8)
    ref, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked, **kw)

    def depth(enc):
        enc = enc.astype(np.float64)
        tail = w.near_range - 2500.0 * np.log(np.clip(1.0 - (enc - 1.0) / 0.25, 1e-12, None))
        return np.where(enc <= 1.0, enc * w.near_range, np.minimum(tail, w.range_units))

    frac = {}
    for store in ("r16", "f16"):
        got, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                               store=store, **kw)
        ok = (np.abs(got - ref) <= 1e-3) & (np.abs(depth(got) - depth(ref)) <= 0.5)
        frac[store] = float(ok.mean())
    assert frac["r16"] >= 0.999, frac
    assert frac["f16"] < 0.99, frac
