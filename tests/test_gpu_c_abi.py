"""The C ABI from plain C (tests/c_abi/render_check.c): a program that
includes only include/sdfr.h and the HIP runtime API creates a grid from host
memory, renders through sdfr_render and sdfr_render_noalloc, checks a refused
call, and compares every value with the C oracle. Built with gcc here (the
host code needs no hipcc), run as a child process."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def test_plain_c_caller_matches_the_oracle(tmp_path):
    import oracle
    if not oracle.LIB_PATH.exists():
        oracle.build()
    lib = ROOT / "rl_cs1.6_surf_amd" / "lib"
    exe = tmp_path / "render_check"
    subprocess.run(["gcc", "-O2", "-std=c11", "-D__HIP_PLATFORM_AMD__",
                    "-I", str(ROOT / "include"), "-I", "/opt/rocm/include",
                    str(ROOT / "tests" / "c_abi" / "render_check.c"), "-o", str(exe),
                    "-L", str(lib), "-lsdfr", "-L", str(oracle.HERE), "-l:liboracle_march.so",
                    "-L", "/opt/rocm/lib", "-lamdhip64", "-lm",
                    f"-Wl,-rpath,{lib}:{oracle.HERE}:/opt/rocm/lib"], check=True)
    print("case c-abi plain C caller", flush=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout + r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 differ from the oracle (noalloc: 0)" in r.stdout
