"""Installs the MI355X render path into the reference's ``surfgym`` package.

The reference's trainer puts its own ``python/`` directory first on
``sys.path`` and imports ``surfgym`` from there (python/train_fast.py:58-76):
``surfgym`` (the C core's binding), then ``surfgym.goalfield``, whose first
line imports ``surfgym.vision`` (goalfield.py:40), then ``surfgym.vision``
itself. By line 75 the reference's vision module is long bound, so putting
this package on the path changes nothing. :func:`install` instead registers
an import hook, before any of those imports, that serves

* ``surfgym.vision``    -> this package's vision.py (GpuLidar over libsdfr.so,
  the grid contract, the GPU SDF bake);
* ``surfgym.goalfield`` -> this package's goalfield.py (GPU goal-field bake
  and sampler, EuclidField), unless ``goalfield=False``;
* ``surfgym._sdfr``     -> the ctypes binding both of them use;

as members of the reference's own package, so everything else (the core,
rewards, zones, surfmask, ...) stays the reference's and imports these names
from them unchanged. Usage, with ``rl_cs1.6_surf_amd/`` on ``sys.path``::

    import surfgym_mi355x
    surfgym_mi355x.install()
    # ... the trainer's own imports, unchanged

or run the trainer itself unchanged::

    python rl_cs1.6_surf_amd/surfgym_mi355x.py python/train_fast.py [args ...]
"""
from __future__ import annotations

import importlib.abc
import importlib.util
import runpy
import sys
from pathlib import Path

IMPL = Path(__file__).resolve().parent / "surfgym"
PACKAGE = "surfgym"
_SERVED = ("vision", "goalfield", "_sdfr")

__all__ = ["install", "uninstall", "installed"]


def _is_ours(module) -> bool:
    f = getattr(module, "__file__", None)
    return f is not None and Path(f).resolve().parent == IMPL


class _Finder(importlib.abc.MetaPathFinder):
    """Serves the replaced modules of a ``surfgym`` package that is not this
    one; every other name goes to the normal finders."""

    def __init__(self, leaves):
        self.leaves = frozenset(leaves)

    def find_spec(self, fullname, path=None, target=None):
        pkg, _, leaf = fullname.rpartition(".")
        if pkg != PACKAGE or leaf not in self.leaves:
            return None
        parent = sys.modules.get(PACKAGE)
        if parent is None or _is_ours(parent):
            return None   # this package itself: its own files are found normally
        return importlib.util.spec_from_file_location(fullname, IMPL / f"{leaf}.py")


def installed():
    """The active hook, or None."""
    for f in sys.meta_path:
        if isinstance(f, _Finder):
            return f
    return None


def install(goalfield: bool = True):
    """Make later imports of ``surfgym.vision`` (and ``surfgym.goalfield``)
    load this package's modules. Raises if the reference's version of one of
    them is already imported: the hook has to run before the first import."""
    leaves = ["vision", "_sdfr"] + (["goalfield"] if goalfield else [])
    for leaf in leaves:
        m = sys.modules.get(f"{PACKAGE}.{leaf}")
        if m is not None and not _is_ours(m):
            raise RuntimeError(
                f"{PACKAGE}.{leaf} was imported from {getattr(m, '__file__', '?')} before "
                "surfgym_mi355x.install(); call install() before the first surfgym import")
    uninstall()
    finder = _Finder(leaves)
    sys.meta_path.insert(0, finder)
    return finder


def uninstall() -> None:
    """Remove the hook (modules already imported stay as they are)."""
    sys.meta_path[:] = [f for f in sys.meta_path if not isinstance(f, _Finder)]


def _main(argv) -> int:
    if not argv:
        print("usage: python surfgym_mi355x.py SCRIPT [args ...]", file=sys.stderr)
        return 2
    install()
    sys.argv = list(argv)
    # as `python SCRIPT` would: the script's directory first on the path, in
    # place of this file's (whose surfgym/ must not shadow the reference's)
    sys.path[0] = str(Path(argv[0]).resolve().parent)
    runpy.run_path(argv[0], run_name="__main__")
    return 0


if __name__ == "__main__":
    sys.exit(_main(sys.argv[1:]))
