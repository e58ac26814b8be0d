"""surfgym (MI355X render path): the reference's ``surfgym.vision`` lidar,
re-implemented as hand-written HIP kernels behind a C ABI (include/sdfr.h).

Only the depth-render path lives here: ``from surfgym.vision import
GpuLidar, pick_cell`` (python/train_fast.py:75) resolves to this package
when ``rl_cs1.6_surf_amd/`` is on ``sys.path`` ahead of the reference's
``python/``.
"""
from __future__ import annotations

__all__ = ["vision", "synth"]
