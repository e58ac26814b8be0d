"""surfgym (MI355X render path): the reference's ``surfgym.vision`` lidar,
re-implemented as hand-written HIP kernels behind a C ABI (include/sdfr.h).

Only the depth-render path (and the goal field beside it) lives here. The
reference's trainer reaches it through ``surfgym_mi355x.install()``, which
puts this package's ``vision`` and ``goalfield`` modules under the
reference's own ``surfgym`` package before ``from surfgym.vision import
GpuLidar, pick_cell`` (python/train_fast.py:75) runs; the rest of that
package (the C core binding, zones, rewards) stays the reference's.
"""
from __future__ import annotations

__all__ = ["vision", "synth"]
