"""Lockstep torch restatement of the reference's CPU render — TEST
INFRASTRUCTURE ONLY (the CPU baseline bench.py times, and a cross-check of
oracle/march.c).

It has the shape of the reference's CPU fallback, ``_render_torch``
(python/surfgym/vision.py:626-666): every ray advances together, one grid
gather per step for all rays, with dead rays adding 0, and a host-side
``any()`` test every 8 steps (vision.py:651-653). Directions come from
``_dirs_equiangular`` (vision.py:596-607). The operation order per step is
the reference's: ``((e + d*t) - mins) * inv_cell``, truncate, clamp, gather,
``alive &= (s > eps) & (t < range)``, ``t += max(0.9*s, min_step) * alive``.

Rays are processed flat, in chunks of envs (exact, since rays are
independent), so memory stays bounded at any batch size.
"""
from __future__ import annotations

import numpy as np
import torch


def _equiangular_tables(width, height, hfov_deg, vfov_deg):
    d2r = np.pi / 180.0
    yoff = (hfov_deg * (0.5 - (np.arange(width) + 0.5) / width)) * d2r
    poff = (vfov_deg * (0.5 - (np.arange(height) + 0.5) / height)) * d2r
    return (torch.as_tensor(yoff, dtype=torch.float32),
            torch.as_tensor(poff, dtype=torch.float32))


def _pinhole_tables(width, height, hfov_deg, vfov_deg):
    """Tangent-plane offsets of the pinhole camera (vision.py:515-529): the
    outermost pixels on the fov edge, a one-pixel axis on the centre ray."""
    d2r = np.pi / 180.0
    tu = float(np.tan(0.5 * hfov_deg * d2r))
    tv = float(np.tan(0.5 * vfov_deg * d2r))
    uo = tu * (2.0 * np.arange(width) / max(width - 1, 1) - 1.0)
    vo = tv * (1.0 - 2.0 * np.arange(height) / max(height - 1, 1))
    if width == 1:
        uo[:] = 0.0
    if height == 1:
        vo[:] = 0.0
    return (torch.as_tensor(uo, dtype=torch.float32),
            torch.as_tensor(vo, dtype=torch.float32))


@torch.no_grad()
def render(grid, mins, cell, origin, yaw_deg, pitch_deg, ducked, *, width=128, height=64,
           hfov_deg=120.0, vfov_deg=90.0, range_units=2000.0, near_range=None, hit_eps=None,
           min_step=None, max_steps=64, env_chunk=64, keep=None, pinhole=False, surf_nz=None):
    """(N,H,W) f32 encodings, computed on the CPU with torch in lockstep;
    (N,H,W,2) with ``surf_nz`` (the int8 |n_z|*127 grid): the encoding and
    |n_z| of the voxel re-derived at the clamped depth, as a float divided by
    127 (vision.py:658-666). ``pinhole`` casts the tangent-plane rays of
    ``_dirs_pinhole`` (vision.py:609-624) instead of the equiangular ones.

    ``keep``: a dict that receives the march's own per-ray values, ``t``
    (N,H,W) f32 depths (clamped to the range) and ``dirs`` (N,H,W,3) f32
    directions as torch computed them, so a comparison can re-trace any ray
    exactly as this render marched it."""
    g = torch.as_tensor(np.ascontiguousarray(grid, np.float32)).reshape(-1)
    nz, ny, nx = np.shape(grid)
    mins_t = torch.as_tensor(np.asarray(mins, np.float32).reshape(3))
    origin = torch.as_tensor(np.asarray(origin, np.float32).reshape(-1, 3))
    yaw = torch.as_tensor(np.asarray(yaw_deg, np.float32).reshape(-1))
    pitch = torch.as_tensor(np.asarray(pitch_deg, np.float32).reshape(-1))
    duck = torch.as_tensor(np.asarray(ducked, np.float64).reshape(-1) != 0)
    rng = float(range_units)
    near = float(near_range) if near_range else rng
    eps = 0.6 * cell if hit_eps is None else float(hit_eps)
    mstep = 0.3 * cell if min_step is None else float(min_step)
    inv_cell = 1.0 / float(cell)
    d2r = np.pi / 180.0
    yoff, poff = _equiangular_tables(width, height, hfov_deg, vfov_deg)
    uoff, voff = _pinhole_tables(width, height, hfov_deg, vfov_deg)
    snz = None
    if surf_nz is not None:
        snz = torch.as_tensor(np.ascontiguousarray(surf_nz, np.int8)).reshape(-1)
    n_all = origin.shape[0]
    out = torch.empty((n_all, height, width) + ((2,) if snz is not None else ()))
    if keep is not None:
        keep["t"] = np.empty((n_all, height, width), np.float32)
        keep["dirs"] = np.empty((n_all, height, width, 3), np.float32)
    for a in range(0, n_all, env_chunk):
        b = min(n_all, a + env_chunk)
        n = b - a
        if pinhole:
            # forward + u*right + v*up, then times its rsqrt (vision.py:614-624)
            yw = (yaw[a:b] * d2r).view(n, 1, 1)
            pt = (pitch[a:b] * d2r).view(n, 1, 1)
            cy, sy = torch.cos(yw), torch.sin(yw)
            cp, sp = torch.cos(pt), torch.sin(pt)
            u = uoff.view(1, 1, width)
            v = voff.view(1, height, 1)
            fx = cp * cy + u * sy - v * sp * cy
            fy = cp * sy - u * cy - v * sp * sy
            fz = sp + v * cp
            inv = torch.rsqrt(fx * fx + fy * fy + fz * fz)
            dx = (fx * inv).reshape(-1)
            dy = (fy * inv).reshape(-1)
            dz = (fz * inv).reshape(-1)
        else:
            # per-pixel angles (vision.py:603-607)
            p = (pitch[a:b] * d2r).view(n, 1, 1) + poff.view(1, height, 1)
            y = (yaw[a:b] * d2r).view(n, 1, 1) + yoff.view(1, 1, width)
            cp = torch.cos(p)
            dx = (cp * torch.cos(y)).reshape(-1)
            dy = (cp * torch.sin(y)).reshape(-1)
            dz = torch.sin(p).expand(n, height, width).reshape(-1)
        hw = height * width
        eye_z = origin[a:b, 2] + torch.where(duck[a:b], 12.0, 17.0)
        ex = origin[a:b, 0].repeat_interleave(hw)
        ey = origin[a:b, 1].repeat_interleave(hw)
        ez = eye_z.repeat_interleave(hw)
        t = torch.zeros(n * hw)
        alive = torch.ones(n * hw, dtype=torch.bool)
        for k in range(max_steps):
            ix = ((ex + dx * t - mins_t[0]) * inv_cell).long().clamp_(0, nx - 1)
            iy = ((ey + dy * t - mins_t[1]) * inv_cell).long().clamp_(0, ny - 1)
            iz = ((ez + dz * t - mins_t[2]) * inv_cell).long().clamp_(0, nz - 1)
            s = g[(iz * ny + iy) * nx + ix]
            alive &= (s > eps) & (t < rng)
            t += torch.clamp(s * 0.9, min=mstep) * alive
            if (k & 7) == 7 and not bool(alive.any()):
                break
        t = torch.clamp(t, max=rng)
        if keep is not None:
            keep["t"][a:b] = t.view(n, height, width).numpy()
            keep["dirs"][a:b] = torch.stack((dx, dy, dz), 1).view(n, height, width, 3).numpy()
        enc = (torch.clamp(t, max=near) / near
               + 0.25 * (1.0 - torch.exp(-torch.clamp(t - near, min=0.0) / 2500.0)))
        if snz is None:
            out[a:b] = enc.view(n, height, width)
        else:
            # the voxel under the clamped depth, by the march's own index formula
            ix = ((ex + dx * t - mins_t[0]) * inv_cell).long().clamp_(0, nx - 1)
            iy = ((ey + dy * t - mins_t[1]) * inv_cell).long().clamp_(0, ny - 1)
            iz = ((ez + dz * t - mins_t[2]) * inv_cell).long().clamp_(0, nz - 1)
            m = snz[(iz * ny + iy) * nx + ix].float() / 127.0
            out[a:b] = torch.stack((enc, m), -1).view(n, height, width, 2)
    return out.numpy()
