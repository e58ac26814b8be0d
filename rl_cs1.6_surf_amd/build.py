"""Builds the native parts of the renderer in-tree.

* ``lib/libsdfr.so``  — csrc/sdfr.hip (the render), csrc/edt.hip (the
  distance-transform bake) and csrc/goal.hip (the goal-field bake and
  sampler), the HIP kernels and the C ABI of include/sdfr.h, compiled for
  gfx950 only.
* ``lib/libsurfsynth.so`` — csrc/synth.c, the host-side synthetic scene
  evaluator (gcc, OpenMP).

Usage: ``python rl_cs1.6_surf_amd/build.py`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
LIB = PKG / "lib"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# -ffp-contract=off: the march and the encoding are fp32 in the reference's
# operation order, one rounding per operation. packed-fp32-ops is switched
# off so the compiler never forms v_pk_{add,mul,fma}_f32.
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
             "-ffp-contract=off", "-fvisibility=hidden",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[0]} ... {cmd[-1]}")


def build_sdfr(verbose: bool = False) -> Path:
    LIB.mkdir(exist_ok=True)
    out = LIB / "libsdfr.so"
    tmp = out.with_name(out.name + ".tmp")
    _run([HIPCC, *HIP_FLAGS, "-I", str(REPO / "include"), str(PKG / "csrc" / "sdfr.hip"),
          str(PKG / "csrc" / "edt.hip"), str(PKG / "csrc" / "goal.hip"), "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    return out


def build_synth(verbose: bool = False) -> Path:
    LIB.mkdir(exist_ok=True)
    out = LIB / "libsurfsynth.so"
    tmp = out.with_name(out.name + ".tmp")
    _run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-fvisibility=hidden",
          str(PKG / "csrc" / "synth.c"), "-o", str(tmp), "-lm"], verbose)
    os.replace(tmp, out)
    return out


def build_all(verbose: bool = False):
    return [build_sdfr(verbose), build_synth(verbose)]


if __name__ == "__main__":
    for p in build_all(verbose=True):
        print("built", p)
