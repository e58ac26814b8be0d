"""bench.py's contract pieces that need no GPU: the option surface, the
one-GPU refusal and the profiled-traffic lookup the roofline line carries."""
from __future__ import annotations

import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr) or "single MI355X" in (r.stdout + r.stderr)


def test_every_traffic_line_in_profiles_parses_and_is_found():
    lines = []
    for f in sorted((ROOT / "profiles").glob("*.md")):
        for line in f.read_text().splitlines():
            if line.strip().startswith("traffic_bytes_per_launch["):
                m = re.match(r"traffic_bytes_per_launch\[(.+?)\] = (\d+)$", line.strip())
                assert m, (f.name, line)
                lines.append((m.group(1), int(m.group(2))))
    keys = [k for k, _ in lines]
    assert len(keys) == len(set(keys)), "a configuration is profiled twice"
    for k, v in lines:
        assert bench.profiled_traffic(k) == v
    # the default workload's key, as bench.py builds it
    assert bench.profiled_traffic("ramp_field tiles rpl=2 brick4 f32 order=lookahead")
    assert bench.profiled_traffic("no such workload") is None


@pytest.mark.parametrize("key", ["ramp_field tiles rpl=2 brick4 f32 order=lookahead",
                                 "winding_track tiles rpl=1 brick4 f32 order=lookahead",
                                 "sparse_grazing tiles rpl=2 brick4 f32 order=lookahead",
                                 "ramp_field_f16_bf16 tiles rpl=2 brick4 f16 order=lookahead"])
def test_bench_workloads_have_profiled_traffic(key):
    assert bench.profiled_traffic(key) > 0
