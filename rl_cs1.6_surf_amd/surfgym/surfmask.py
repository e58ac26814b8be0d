"""Surf-mask grid source: the per-voxel |n_z|*127 (int8) second channel.

The reference bakes it by rasterising the map's exported triangle mesh into
the vision grid (python/surfgym/surfmask.py:1-50, build_surfnz :193-236) and
caches it as ``maps/<map>.surfnz_<cell>.npz``. This module loads that cache,
with the same signature check (the .bsp, the mesh and the bake's content
tag), so an existing bake is reused as-is; the rasteriser itself is not part
of this renderer. ``GpuLidar.from_grid(..., surf_nz=grid)`` takes any int8
grid instead, and tests replace ``build_surfnz`` on this module as the
reference's do.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

from .vision import _SDF_BUILDER_VERSION

__all__ = ["build_surfnz"]

_SURFNZ_SEMANTICS = "n2"


def build_surfnz(core, cell: float = 16.0, cache_dir=None, mesh_path=None):
    """(nz_grid int8 [nz, ny, nx], mins float32 (3,)) from the reference's cache."""
    bsp = Path(core.bsp_path)
    mesh = Path(mesh_path) if mesh_path else \
        bsp.parent.parent / "viewer" / "assets" / f"{bsp.stem}.mesh.json"
    if not mesh.exists():
        raise FileNotFoundError(f"{mesh}: the surf-mask signature covers the exported mesh")
    st, mst = bsp.stat(), mesh.stat()
    sig = (f"v{_SDF_BUILDER_VERSION}_{st.st_size}_{st.st_mtime_ns}"
           f"_m{mst.st_size}_{mst.st_mtime_ns}_{_SURFNZ_SEMANTICS}")
    cache = Path(cache_dir) if cache_dir else bsp.parent
    f = cache / f"{bsp.stem}.surfnz_{cell:g}.npz"
    if f.exists():
        z = np.load(f, allow_pickle=False)
        if "sig" in z and str(z["sig"]) == sig:
            return z["nz"], z["mins"].astype(np.float32)
    raise FileNotFoundError(
        f"no current surf-mask bake at {f} (signature {sig}); bake it once with the "
        "reference's surfmask.build_surfnz, or pass surf_nz to GpuLidar.from_grid")
