"""Agreement of a render with the reference's CPU arithmetic — TEST
INFRASTRUCTURE ONLY (tests/ and bench.py's CPU-baseline leg).

The reference's CPU render (``_dirs_equiangular`` + ``_render_torch``,
python/surfgym/vision.py:596-607, :626-666) takes cos/sin/exp from torch's
CPU kernels; ``oracle/lockstep.py`` restates it with those same torch calls.
The renderer (and ``oracle/march.c``, which it equals bit for bit) takes
them correctly rounded. The two can therefore differ in the last bit of a
ray direction, and a sample that lies within that much of a voxel face then
reads the neighbouring voxel. :func:`compare` measures the renderer's
accuracy bar on a whole image pair — a ray agrees when its depth is within
0.5 u of the reference's and its encoding within 1e-3 — and classifies
every ray that does not:

* ``grazing``: a march that stopped on a surface met it at more than
  ``GRAZING_DEG`` (75) degrees from the surface normal. The normal is the
  central-difference gradient of the stored grid at the voxel the march
  stopped in (one-sided at the grid border, where the clamped neighbour is
  the voxel itself), or, when that gradient is zero (a stop deep inside a
  solid), at the last voxel it sampled outside; the angle is between the
  ray and that normal, taken unsigned.
* ``step_phase``: both marches stopped on a surface, their depths differ
  by no more than the longer of their two last steps, and they parted at a
  sample within ``TIE_U`` (0.01 u) of a voxel face: up to that sample they
  read the same voxels, there the two directions' last-bit difference put
  the samples on either side of the face (``split_face_u``, the larger of
  the two samples' distances to it), and the rest of the step sequence is
  shifted. The march resolves a hit only to its last step (``max(0.9*s,
  min_step)``, vision.py:96-98), so the hit lands elsewhere within one step.
* ``tie_other``: not grazing, parted at such a face tie, but with another
  outcome (e.g. one march clipping the edge of a solid that the other
  passes).
* ``other``: anything else — two marches that part at a sample farther
  than ``TIE_U`` from any face are not explained by the directions' last
  bits; each is listed.

Depths: the reference's from the lockstep render itself (``keep``); the
renderer's by re-tracing the ray with the oracle's march and directions,
whose encoding must equal the renderer's bit for bit (rays where it does
not are counted as ``renderer_differs``). Rays whose two encodings are equal
are not re-traced: equal fp32 encodings bound the depth difference by the
encoding's resolution (below 0.01 u for t <= 6144 at near 2000).
"""
from __future__ import annotations

import numpy as np

from . import _load, _ptr

GRAZING_DEG = 75.0
TIE_U = 0.01
DEPTH_TOL_U = 0.5
ENC_TOL = 1e-3
WHY = ("hit", "range", "exhausted")


def _dir(lib, width, height, hfov, vfov, yaw, pitch, r, c, pinhole=False):
    d = np.empty(3, np.float32)
    tan_h = float(np.tan(0.5 * hfov * (np.pi / 180.0)))
    tan_v = float(np.tan(0.5 * vfov * (np.pi / 180.0)))
    lib.oracle_ray_dir(1 if pinhole else 0, int(r), int(c), int(width), int(height), float(hfov),
                       float(vfov), tan_h, tan_v, float(yaw), float(pitch), _ptr(d))
    return d


def _stop_voxel(eye, d, t, mins, cell, shape):
    """The voxel under depth t along d (the surf channel's index, vision.py:
    658-665) in fp32, and each axis's voxel coordinate."""
    f = np.float32
    inv = f(1.0 / float(cell))
    nz, ny, nx = shape
    idx, pos = [], []
    for a, n in ((0, nx), (1, ny), (2, nz)):
        q = f(f(f(eye[a]) + f(f(d[a]) * f(t))) - f(mins[a])) * inv
        pos.append(float(q))
        idx.append(0 if not q > 0 else min(int(q), n - 1))
    return tuple(idx), pos


def trace(grid, mins, cell, eye, d, *, range_units, hit_eps, min_step, max_steps):
    """One ray through the oracle's march, sample by sample (oracle/march.c
    ``oracle_march_trace``): dict of t_k, vox (k,3), pos (k,3) voxel
    coordinates, s_k, the final t (unclamped) and the stop reason."""
    lib = _load()
    g = np.ascontiguousarray(grid, np.float32)
    nz, ny, nx = g.shape
    m = np.ascontiguousarray(mins, np.float32).reshape(3)
    cap = int(max_steps)
    t_k = np.empty(cap, np.float32)
    vox = np.empty((cap, 3), np.int32)
    pos = np.empty((cap, 3), np.float32)
    s_k = np.empty(cap, np.float32)
    tf = np.empty(1, np.float32)
    why = np.empty(1, np.int32)
    k = lib.oracle_march_trace(_ptr(g), nx, ny, nz, _ptr(m), float(np.float32(1.0 / float(cell))),
                               float(eye[0]), float(eye[1]), float(eye[2]),
                               float(d[0]), float(d[1]), float(d[2]), float(range_units),
                               float(hit_eps), float(min_step), cap, cap, _ptr(t_k), _ptr(vox),
                               _ptr(pos), _ptr(s_k), _ptr(tf), _ptr(why))
    return {"t_k": t_k[:k], "vox": vox[:k], "pos": pos[:k], "s_k": s_k[:k],
            "t": float(tf[0]), "why": WHY[int(why[0])]}


def _normal_angle(grid, tr, d):
    """Angle (degrees) between the ray and the grid's central-difference
    gradient at the stop voxel (or the last voxel sampled outside a solid
    when the gradient there is zero); None when both are zero."""
    nz, ny, nx = grid.shape
    for ix, iy, iz in (tr["vox"][-1], tr["vox"][-2] if len(tr["vox"]) > 1 else tr["vox"][-1]):
        gx = float(grid[iz, iy, min(ix + 1, nx - 1)]) - float(grid[iz, iy, max(ix - 1, 0)])
        gy = float(grid[iz, min(iy + 1, ny - 1), ix]) - float(grid[iz, max(iy - 1, 0), ix])
        gz = float(grid[min(iz + 1, nz - 1), iy, ix]) - float(grid[max(iz - 1, 0), iy, ix])
        gv = np.array([gx, gy, gz])
        nrm = float(np.linalg.norm(gv))
        if nrm > 0.0:
            dv = np.asarray(d, np.float64)
            c = abs(float(dv @ gv)) / (nrm * float(np.linalg.norm(dv)))
            return float(np.degrees(np.arccos(min(1.0, c))))
    return None


def _last_step(tr):
    return float(tr["t_k"][-1] - tr["t_k"][-2]) if len(tr["t_k"]) > 1 else 0.0


def compare(grid, mins, cell, origin, yaw_deg, pitch_deg, ducked, image, ref_enc, ref_keep, *,
            width, height, range_units, near_range, hit_eps, max_steps, min_step=None,
            hfov_deg=120.0, vfov_deg=90.0, list_max=64, pinhole=False, surf_nz=None):
    """Agreement of ``image`` (the renderer's (N,H,W) f32 encodings, or
    (N,H,W,2) with the surf channel and ``surf_nz``) with ``ref_enc`` (the
    lockstep render's, same inputs and camera) whose per-ray depths and
    directions are in ``ref_keep`` (lockstep.render(..., keep=...)).

    With the surf channel, the rays whose depths agree but whose |n_z|
    differ are counted separately: ``surf_tie`` when the two directions put
    the depth's end point on either side of a voxel face within ``TIE_U``
    (the same voxel-face tie, at the end of the march), ``surf_other``
    otherwise.

    Returns a dict: rays, exact (fraction of bit-identical encodings),
    within_tol (fraction within 0.5 u and 1e-3), outliers (count) and their
    classes, the largest depth and encoding differences, and the first
    ``list_max`` outliers described (all of them when None)."""
    lib = _load()
    g = np.ascontiguousarray(grid, np.float32)
    img_all = np.asarray(image, np.float32)
    ref_all = np.asarray(ref_enc, np.float32)
    surf = img_all.ndim == 4
    if img_all.shape != ref_all.shape or img_all.ndim not in (3, 4) or surf != (surf_nz is not None):
        raise ValueError(f"image shapes differ or the surf grid is missing: {img_all.shape} vs "
                         f"{ref_all.shape}")
    img = img_all[..., 0] if surf else img_all
    ref = ref_all[..., 0] if surf else ref_all
    rng = float(range_units)
    near = float(near_range) if near_range else rng
    mstep = float(np.float32(0.3 * cell)) if min_step is None else float(min_step)
    eps = float(hit_eps)
    org = np.asarray(origin, np.float32).reshape(-1, 3)
    yaw = np.asarray(yaw_deg, np.float32).reshape(-1)
    pitch = np.asarray(pitch_deg, np.float32).reshape(-1)
    duck = np.asarray(ducked, np.float64).reshape(-1) != 0
    kw = dict(range_units=rng, hit_eps=eps, min_step=mstep, max_steps=max_steps)
    rays = int(img.size)
    differ = np.argwhere(img != ref)
    classes = {"grazing": 0, "step_phase": 0, "tie_other": 0, "other": 0}
    listed, max_dt, max_de = [], 0.0, 0.0
    n_out = renderer_differs = ref_retrace_differs = 0
    depth_out = set()
    for e, r, c in differ:
        eye = (org[e, 0], org[e, 1], np.float32(org[e, 2] + np.float32(12.0 if duck[e] else 17.0)))
        d_o = _dir(lib, width, height, hfov_deg, vfov_deg, yaw[e], pitch[e], r, c, pinhole)
        d_t = ref_keep["dirs"][e, r, c]
        to = trace(g, mins, cell, eye, d_o, **kw)
        tt = trace(g, mins, cell, eye, d_t, **kw)
        t_o = min(np.float32(to["t"]), np.float32(rng))
        t_t = min(np.float32(tt["t"]), np.float32(rng))
        if np.float32(lib.oracle_encode(float(t_o), near)) != img[e, r, c]:
            renderer_differs += 1
        if t_t != ref_keep["t"][e, r, c]:
            ref_retrace_differs += 1
        dt = abs(float(t_o) - float(t_t))
        de = abs(float(img[e, r, c]) - float(ref[e, r, c]))
        max_dt, max_de = max(max_dt, dt), max(max_de, de)
        if dt <= DEPTH_TOL_U and de <= ENC_TOL:
            continue
        n_out += 1
        depth_out.add((int(e), int(r), int(c)))
        angles = [a for a in (_normal_angle(g, to, d_o) if to["why"] == "hit" else None,
                              _normal_angle(g, tt, d_t) if tt["why"] == "hit" else None)
                  if a is not None]
        last = max(_last_step(to), _last_step(tt))
        k = 0
        nk = min(len(to["vox"]), len(tt["vox"]))
        while k < nk and np.array_equal(to["vox"][k], tt["vox"][k]):
            k += 1
        split = None
        if k < nk:
            ax = int(np.argmax(to["vox"][k] != tt["vox"][k]))
            split = round(max(abs(f - round(f)) for f in (float(to["pos"][k, ax]),
                                                          float(tt["pos"][k, ax])))
                          * float(cell), 6)
        tie = split is not None and split <= TIE_U
        if angles and max(angles) > GRAZING_DEG:
            cls = "grazing"
        elif tie and to["why"] == tt["why"] == "hit" and dt <= last:
            cls = "step_phase"
        elif tie:
            cls = "tie_other"
        else:
            cls = "other"
        classes[cls] += 1
        if list_max is None or len(listed) < list_max:
            listed.append({"env": int(e), "row": int(r), "col": int(c), "class": cls,
                           "depth": round(float(t_o), 3), "depth_ref": round(float(t_t), 3),
                           "stop": to["why"], "stop_ref": tt["why"],
                           "angle_deg": round(max(angles), 1) if angles else None,
                           "last_step_u": round(last, 3), "split_step": k,
                           "split_face_u": split})
    extra = {}
    if surf:
        snz = np.ascontiguousarray(surf_nz, np.int8)
        sdiff = np.argwhere(img_all[..., 1] != ref_all[..., 1])
        tie = other = with_depth = 0
        for e, r, c in sdiff:
            if (int(e), int(r), int(c)) in depth_out:
                with_depth += 1
                continue
            eye = (org[e, 0], org[e, 1],
                   np.float32(org[e, 2] + np.float32(12.0 if duck[e] else 17.0)))
            d_o = _dir(lib, width, height, hfov_deg, vfov_deg, yaw[e], pitch[e], r, c, pinhole)
            d_t = ref_keep["dirs"][e, r, c]
            t_o = min(np.float32(trace(g, mins, cell, eye, d_o, **kw)["t"]), np.float32(rng))
            t_t = ref_keep["t"][e, r, c]
            vo, po = _stop_voxel(eye, d_o, t_o, mins, cell, g.shape)
            vt, pt_ = _stop_voxel(eye, d_t, t_t, mins, cell, g.shape)
            if np.float32(snz[vo[2], vo[1], vo[0]]) / np.float32(127.0) != img_all[e, r, c, 1]:
                renderer_differs += 1
            axes = [a for a in range(3) if vo[a] != vt[a]]
            near_face = bool(axes) and all(
                max(abs(q - round(q)) for q in (po[a], pt_[a])) * float(cell) <= TIE_U
                for a in axes)
            if near_face:
                tie += 1
            else:
                other += 1
        extra = {"surf_differs": int(len(sdiff)), "surf_with_depth_outlier": with_depth,
                 "surf_tie": tie, "surf_other": other}
    return {"rays": rays, "exact": round(1.0 - len(differ) / rays, 7),
            "within_tol": round(1.0 - n_out / rays, 7), "outliers": n_out,
            "outliers_grazing": classes["grazing"], "outliers_step_phase": classes["step_phase"],
            "outliers_tie_other": classes["tie_other"], "outliers_other": classes["other"],
            "max_abs_depth_u": round(max_dt, 4), "max_abs_enc": round(max_de, 6),
            "renderer_differs": renderer_differs, "ref_retrace_differs": ref_retrace_differs,
            "tolerance": f"depth within {DEPTH_TOL_U} u and encoding within {ENC_TOL}",
            "grazing": f"angle to the stop voxel's grid gradient above {GRAZING_DEG:g} deg",
            **extra, "listed": listed}
