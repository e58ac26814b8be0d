"""bench.py's contract pieces that need no GPU: the option surface, the
one-GPU refusal and the profiled-traffic lookup the roofline line carries."""
from __future__ import annotations

import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr) or "single MI355X" in (r.stdout + r.stderr)


def test_every_profile_record_parses_and_names_its_kernels():
    """Each traffic_bytes_per_launch / limiter line under profiles/ parses,
    is found by the lookup bench.py uses, and sits in a file that records
    the hash of the kernels' source it was measured on."""
    traffic, limiter = bench.profile_records()
    assert traffic and limiter
    seen = []
    for f in sorted((ROOT / "profiles").glob("*.md")):
        text = f.read_text()
        keys = re.findall(r"^traffic_bytes_per_launch\[(.+?)\] = \d+$", text, re.M)
        keys += re.findall(r"^limiter\[(.+?)\] = \{", text, re.M)
        if keys:
            assert re.search(r"^sdfr_hip_sha256 = [0-9a-f]{64}$", text, re.M), f.name
        seen += keys
    for k, rec in traffic.items():
        assert rec["bytes"] > 0 and rec["profile"].startswith("profiles/"), k
    for k, rec in limiter.items():
        assert 0.0 < rec["busy"] <= 1.0 and rec["unit"], k
    assert bench.profiled("no such workload", traffic, "bytes") == (None, None)


def test_profiles_were_measured_on_the_current_kernels():
    """A change to csrc/sdfr.hip makes every profiled figure stale: re-profile
    (the commands are in each summary) and record the new hash."""
    traffic, limiter = bench.profile_records()
    now = bench.sdfr_source_sha256()
    stale = sorted({rec["profile"] for rec in list(traffic.values()) + list(limiter.values())
                    if rec["sdfr_hip_sha256"] != now})
    assert not stale, f"profiled on other kernels than csrc/sdfr.hip now holds: {stale}"


@pytest.mark.parametrize("key", ["ramp_field tiles rpl=2 brick4 f32 order=lookahead",
                                 "winding_track tiles rpl=1 brick4 f32 order=lookahead",
                                 "sparse_grazing tiles rpl=2 brick4 f32 order=lookahead",
                                 "ramp_field_r16_bf16 tiles rpl=2 brick4 r16 order=lookahead",
                                 "ramp_field_f16_bf16 tiles rpl=2 brick4 f16 order=lookahead"])
def test_bench_workloads_have_profiled_traffic(key):
    traffic, _ = bench.profile_records()
    value, src = bench.profiled(key, traffic, "bytes")
    assert src is not None and src["current"], key
    assert value > 0


@pytest.mark.parametrize("name", ["ramp_field", "winding_track", "sparse_grazing",
                                  "ramp_field_r16_bf16", "ramp_field_f16_bf16", "small_ramps"])
def test_bench_workloads_have_a_measured_limiter(name):
    _, limiter = bench.profile_records()
    value, src = bench.profiled(name, limiter)
    assert src is not None and src["current"], name
    assert value["unit"] and 0.0 < value["busy"] <= 1.0


def test_other_configurations_cover_the_metric_workloads():
    names = {n for n, _, _ in bench.OTHER_CONFIGS}
    assert names == {"small_ramps", "winding_track", "sparse_grazing", "ramp_field_r16_bf16",
                     "ramp_field_f16_bf16"}
    graph = {n: g for n, g, _ in bench.OTHER_CONFIGS}
    shape = {n: s for n, _, s in bench.OTHER_CONFIGS}
    for fused in ("ramp_field_r16_bf16", "ramp_field_f16_bf16"):
        assert graph[fused] is True
        assert shape[fused](8192) == (8192, 1, 64, 128)


def test_config_summary_carries_the_profiled_traffic_rate():
    r = {"envs": 2048, "rays": 16777216, "grid": "g", "out": "f32", "out_shape": [2048, 64, 128],
         "graph": False, "ms_per_step": 2.0, "march_kernel_ms_avg": 1.5, "loads": 335544320,
         "alg_bytes": 1_500_000_000, "rpl": 1}
    s = bench.config_summary(r, 15_000_000_000, {"profile": "p", "current": True},
                             {"unit": "L2-miss traffic", "busy": 0.9})
    assert s["traffic_bytes_per_launch"] == 15_000_000_000
    assert s["traffic_gbs"] == 10000.0          # 15 GB over 1.5 ms
    assert s["alg_frac_of_hbm_peak"] == 0.125   # 1 TB/s of 8
    assert s["limiter"] == "L2-miss traffic" and s["g_rays_per_s"] == round(16777216 / 2e-3 / 1e9, 4)
    stale = bench.config_summary(r)
    assert stale["traffic_bytes_per_launch"] is None and stale["traffic_gbs"] is None
    assert stale["limiter"] is None


def test_range_encoding_is_the_kernels_encoding_of_the_range():
    import oracle
    for rng, near in ((6144.0, 2000.0), (1536.0, 1536.0), (23529.728600219765, 2000.0), (900.0, 400.0)):
        assert bench.range_encoding(rng, near) == oracle.encode(float(np.float32(rng)), near)


def test_step_census_statistics_on_a_known_tally():
    import torch
    from types import SimpleNamespace
    w = SimpleNamespace(height=4, width=16, max_steps=10, range_units=100.0, near_range=100.0)
    taps = torch.arange(1, 65, dtype=torch.int32).clamp(max=10).view(1, 4, 16)
    out = torch.zeros(1, 4, 16)
    out[0, 0, :3] = 1.0   # the range's encoding when near == range
    c = bench.step_census(taps, out, w)
    assert c["max"] == 10 and c["median"] == 10 and c["p90"] == 10
    assert c["exhaust_frac"] == round(55 / 64, 5)
    assert c["reach_range_frac"] == round(3 / 64, 5)
    assert c["loads_mean"] == round((45 + 550) / 64, 3)
    # one 16x4 tile whose slowest ray takes 10 steps
    assert c["lane_efficiency_per_tile"] == round(595 / 640, 4)


def test_cpu_baseline_reports_its_agreement_with_the_render():
    """The CPU leg times the lockstep render and, given the GPU image of the
    same envs, reports the agreement record the JSON line carries. Here the
    oracle's image stands in for the GPU's (equal bit for bit on the GPU):
    on small_ramps the two arithmetics agree on every ray; a planted wrong
    pixel is caught as an image that is not the oracle's march."""
    import oracle
    from surfgym import synth
    w = synth.WORKLOADS["small_ramps"]
    sc = w.scene()
    ps = w.poses(sc, 16)
    img, _ = oracle.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                           width=w.width, height=w.height, range_units=w.range_units,
                           near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps)
    r = bench.cpu_baseline(w, sc, 16, repeats=1, image=img)
    a = r["agreement"]
    assert r["kind"] == "port" and r["cores"] >= 1 and r["value"] > 0
    for key in ("rays", "exact", "within_tol", "outliers", "outliers_grazing",
                "outliers_step_phase", "outliers_tie_other", "outliers_other",
                "renderer_differs", "not_step_phase"):
        assert key in a, key
    assert a["rays"] == 16 * 64 * 128 and a["exact"] == 1.0 and a["outliers"] == 0
    bad = img.copy()
    bad[3, 10, 20] = 0.123
    a = bench.cpu_baseline(w, sc, 16, repeats=1, image=bad)["agreement"]
    assert a["renderer_differs"] == 1 and a["outliers"] == 1
    assert bench.cpu_baseline(w, sc, 16, repeats=1)["agreement"] is None
