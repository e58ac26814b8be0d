"""Depth-render benchmark: G rays/s and ms per batch of the MI355X renderer.

One step = one render of the whole batch (N envs x 128x64 rays) from poses
already resident in HBM into a preallocated output, on the current stream.
Default workload: ``ramp_field`` — 2048 envs x 128x64 = 16,777,216 rays over
a 256x256x128 fp32 grid at 16 u (64 ramps + 16 boxes), max 96 steps,
hit_eps 1 u, range 6144 u, near 2000 u.

Prints ONE JSON line. ``roofline`` prices the march kernel against HBM:
algorithmic bytes per launch = sum over rays of (grid loads x voxel bytes)
+ rays x output bytes + envs x 24 B of pose input; the per-ray load counts
come from the kernel's census mode (run once, outside the timed region), and
the launch duration from HIP events around the timed launches on the stream
the kernel runs on. ``cpu_baseline`` times the lockstep torch restatement of
the reference's CPU render on this host's cores, on a bounded sample of the
same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "rl_cs1.6_surf_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
METRIC = "G rays/s and ms/batch at 2048 envs×128×64; % of HBM/cache BW roofline"


def _log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_baseline(w, sc, envs, repeats=5, image=None):
    """Lockstep torch render (the reference's CPU path shape) on host cores.

    With ``image`` (the GPU render of the same ``envs`` poses, (N,H,W) f32)
    it also reports ``agreement``: one more lockstep render, untimed, that
    keeps its per-ray depths and directions, compared ray by ray with the
    GPU image at the accuracy bar (0.5 u in depth, 1e-3 in the
    encoding), every ray outside it re-traced and classified
    (oracle/agreement.py)."""
    import torch
    from oracle import agreement, lockstep
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    ps = w.poses(sc, envs)
    kw = dict(width=w.width, height=w.height, range_units=w.range_units,
              near_range=w.near_range, hit_eps=w.hit_eps, max_steps=w.max_steps)
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        lockstep.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked, **kw)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    agree = None
    if image is not None:
        keep = {}
        ref = lockstep.render(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch, ps.ducked,
                              keep=keep, **kw)
        agree = agreement.compare(sc.sdf, sc.mins, sc.cell, ps.origin, ps.yaw, ps.pitch,
                                  ps.ducked, image, ref, keep, list_max=None, **kw)
        del keep, ref
        listed = agree.pop("listed")
        steps = [o for o in listed if o["class"] == "step_phase"]
        agree["step_phase_max_depth_over_last_step"] = (
            round(max(abs(o["depth"] - o["depth_ref"]) / o["last_step_u"] for o in steps), 4)
            if steps else None)
        agree["not_step_phase"] = [o for o in listed if o["class"] != "step_phase"][:16]
        _log(f"[bench] agreement with the torch lockstep: {agree['exact']:.5%} bit-identical, "
             f"{agree['within_tol']:.5%} within tolerance, {agree['outliers']} outliers "
             f"({agree['outliers_grazing']} grazing, {agree['outliers_step_phase']} one step "
             f"apart, {agree['outliers_tie_other']} other after a face tie, "
             f"{agree['outliers_other']} unexplained)")
    rays = envs * w.width * w.height
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(rays / t / 1e9, 6), "unit": "G rays/s", "cores": cores,
            "kind": "port",
            "sample": f"{envs} of {w.n_envs} envs of {w.name} ({rays} rays), torch lockstep, "
                      f"median of {repeats}: {t * 1e3:.1f} ms; cpu: {model}",
            "agreement": agree}


class HipEvents:
    """Timing events made up front with the HIP runtime torch has loaded
    (hipEventCreate), each recorded once in the timed loop. torch's events
    are created lazily at their first record, inside the loop, and that
    occasionally stalled the host for ~25 ms mid-run; re-recording events
    created beforehand slowed some renders instead."""

    def __init__(self, n):
        import ctypes
        self._c = ctypes
        lib = ctypes.CDLL("libamdhip64.so.7")       # the instance torch already loaded
        vp = ctypes.c_void_p
        lib.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        lib.hipEventRecord.argtypes = [vp, vp]
        lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        lib.hipEventDestroy.argtypes = [vp]
        self._lib = lib
        self.ev = []
        for _ in range(n):
            h = vp()
            self._check(lib.hipEventCreate(ctypes.byref(h)), "hipEventCreate")
            self.ev.append(h)

    @staticmethod
    def _check(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed ({rc})")

    def record(self, i, stream):
        self._check(self._lib.hipEventRecord(self.ev[i], stream), "hipEventRecord")

    def ms(self, i, j):
        out = self._c.c_float()
        self._check(self._lib.hipEventElapsedTime(self._c.byref(out), self.ev[i], self.ev[j]),
                    "hipEventElapsedTime")
        return out.value

    def close(self):
        for h in self.ev:
            self._lib.hipEventDestroy(h)
        self.ev = []


SDFR_SOURCE = ROOT / "rl_cs1.6_surf_amd" / "csrc" / "sdfr.hip"


def sdfr_source_sha256():
    """Hash of the render kernels' source: the profiles under profiles/
    record it, so a figure measured on another version of the kernels is
    recognised as stale."""
    import hashlib
    return hashlib.sha256(SDFR_SOURCE.read_bytes()).hexdigest()


def profile_records():
    """Per-workload records of the rocprofv3 summaries under profiles/: the
    lines ``traffic_bytes_per_launch[<key>] = <bytes>`` and
    ``limiter[<workload>] = <json>``, each with the file it came from and
    the file's ``sdfr_hip_sha256 = <hex>`` (the kernels it was measured on)."""
    import re
    traffic, limiter = {}, {}
    for f in sorted((ROOT / "profiles").glob("*.md")):
        text = f.read_text()
        m = re.search(r"^sdfr_hip_sha256 = ([0-9a-f]{64})\s*$", text, re.M)
        src = {"profile": f"profiles/{f.name}", "sdfr_hip_sha256": m.group(1) if m else None}
        for line in text.splitlines():
            line = line.strip()
            t = re.match(r"traffic_bytes_per_launch\[(.+?)\] = (\d+)$", line)
            if t:
                traffic[t.group(1)] = dict(src, bytes=int(t.group(2)))
            lm = re.match(r"limiter\[(.+?)\] = (\{.*\})$", line)
            if lm:
                limiter[lm.group(1)] = dict(src, **json.loads(lm.group(2)))
    return traffic, limiter


def profiled(key, table, field=None):
    """The record for `key`, marked current or stale against the kernels'
    source as it is now (a stale figure is reported as None)."""
    rec = table.get(key)
    if rec is None:
        return None, None
    current = rec.get("sdfr_hip_sha256") == sdfr_source_sha256()
    src = {"profile": rec["profile"], "sdfr_hip_sha256": rec.get("sdfr_hip_sha256"),
           "current": current}
    value = (rec[field] if field else {k: v for k, v in rec.items()
                                      if k not in ("profile", "sdfr_hip_sha256")})
    return (value if current else None), src


def copy_bandwidth(dev, n_bytes=2_000_000_000, iters=10):
    """Device copy bandwidth, 2 x bytes / time (read + write), median of
    `iters` copies of an n_bytes buffer: the reference's health check method
    (tools/gpu_health.py:76-78). Also the plain copy kernel whose HBM
    counters calibrate the march kernel's FETCH_SIZE / WRITE_SIZE."""
    import torch
    a = torch.empty(n_bytes // 2, dtype=torch.bfloat16, device=dev)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    ms = []
    for _ in range(iters):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        b.copy_(a)
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
    del a, b
    torch.cuda.empty_cache()
    return 2 * n_bytes / (statistics.median(ms) * 1e-3) / 1e9


def bench_bake(args, w, dev):
    """SDF bake: the workload's solid occupancy through sdf_from_occupancy
    (HIP events, median of the timed runs) and through the reference's scipy
    call on this host (one run)."""
    import numpy as np
    import torch
    from surfgym import vision
    sc = w.scene()
    occ = (sc.sdf == 0).astype(np.uint8)
    occ_dev = torch.as_tensor(occ, device=dev)
    for _ in range(max(1, args.warmup)):
        vision.sdf_from_occupancy(occ_dev, sc.cell, device=dev)
    torch.cuda.synchronize()
    ms = []
    for _ in range(args.steps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        vision.sdf_from_occupancy(occ_dev, sc.cell, device=dev)
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
    gpu_ms = statistics.median(ms)
    res = {"metric": "SDF bake ms (exact EDT of the occupancy)", "value": round(gpu_ms, 4),
           "unit": "ms", "higher_is_better": False, "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "data": "synthetic",
           "config": {"workload": w.name, "grid": f"{sc.nx}x{sc.ny}x{sc.nz}",
                      "voxels": int(occ.size), "cell": sc.cell},
           "cpu_baseline": None}
    if not args.no_cpu:
        from oracle import edt
        t0 = time.perf_counter()
        edt.stored(edt.bake(occ, sc.cell))
        cpu_s = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": round(cpu_s * 1e3, 1), "unit": "ms", "cores": 1,
                               "kind": "reference",
                               "sample": "scipy.ndimage.distance_transform_edt on the padded "
                                         "occupancy, the reference's own bake call, one run"}
    print(json.dumps(res), flush=True)


def _reference_goal_loop_seconds(occ_dev, cell, lo, hi):
    """Speed comparator for the goal-field bake: the reference's bake order
    (goalfield.py:232-270) as torch ops on this GPU. Each sweep lowers every
    free voxel to the smallest of its 26 neighbours plus cell * |offset|
    (the neighbours read from a halo-padded copy made at the sweep's start)
    and holds solids at +inf; the loop ends when the count of reached voxels
    and their float64 sum repeat at a check every 64 sweeps, or after 8000
    sweeps. Returns (sweeps, seconds). Not a parity reference."""
    import itertools
    import torch
    blocked = occ_dev != 0
    shape = tuple(blocked.shape)
    field = torch.full(shape, math.inf, device=occ_dev.device)
    box = tuple(slice(lo[a], hi[a] + 1) for a in (2, 1, 0))
    field[box] = torch.where(blocked[box], math.inf, 0.0)
    halo = torch.full(tuple(n + 2 for n in shape), math.inf, device=occ_dev.device)
    moves = []
    for off in itertools.product((-1, 0, 1), repeat=3):
        if any(off):
            view = halo[tuple(slice(1 + o, 1 + o + n) for o, n in zip(off, shape))]
            moves.append((view, cell * math.sqrt(sum(o * o for o in off))))
    cand = torch.empty_like(field)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    sweeps, last = 0, None
    while sweeps < 8000:
        halo[1:-1, 1:-1, 1:-1].copy_(field)
        for view, cost in moves:
            torch.minimum(field, torch.add(view, cost, out=cand), out=field)
        field.masked_fill_(blocked, math.inf)
        sweeps += 1
        if sweeps % 64 == 0:
            reached = field[torch.isfinite(field)]
            probe = (reached.numel(), float(reached.sum(dtype=torch.float64)))
            if probe == last:
                break
            last = probe
    torch.cuda.synchronize()
    return sweeps, time.perf_counter() - t0


def bench_goal(args, dev):
    """Goal-field bake and sampler (goalfield.py:159-298, :68-94): the GPU
    bake of the workload's occupancy (wall time per bake; the bake reads its
    wavefront queue length on the host every few sweeps), the reference's
    torch sweep loop on this same GPU, the oracle's Dijkstra on one host
    core, and the sampler at the trainer's 2048 positions and at 1 M."""
    import numpy as np
    import torch
    from surfgym import goalfield, synth
    name = args.workload if args.workload in ("ramp_field", "winding_track", "maze",
                                               "small_ramps") else "ramp_field"
    w = synth.goal_workload(name)
    nz, ny, nx = w.occ.shape
    occ_dev = torch.as_tensor(w.occ, device=dev)
    lo, hi = goalfield.seed_voxel_box(w.zone, w.mins, w.cell, (nx, ny, nz))
    _log(f"[bench] goal {name}: {nx}x{ny}x{nz} @{w.cell:g}u, seed box {lo.tolist()}..{hi.tolist()}")
    field = None
    for _ in range(max(1, args.warmup)):
        field = goalfield.goal_field_from_occupancy(occ_dev, w.mins, w.zone, w.cell, device=dev)
    torch.cuda.synchronize()
    ms = []
    for _ in range(args.steps):
        t0 = time.perf_counter()
        field = goalfield.goal_field_from_occupancy(occ_dev, w.mins, w.zone, w.cell, device=dev)
        torch.cuda.synchronize()
        ms.append((time.perf_counter() - t0) * 1e3)
    info = field.bake_info
    tiles = ((nx + 7) // 8) * ((ny + 7) // 8) * ((nz + 7) // 8)
    _log(f"[bench] bake median {statistics.median(ms):.3f} ms, {info['sweeps']} sweeps, "
         f"{info['tile_visits']} tile visits ({info['tile_visits'] / tiles:.2f} per tile)")
    # sampler: the trainer's per-tick batch and a throughput batch
    rng = np.random.default_rng(5)
    hi_u = w.mins + np.array([nx, ny, nz]) * w.cell
    samp = {}
    for n in (2048, 1 << 20):
        pos = torch.as_tensor(rng.uniform(w.mins, hi_u, (n, 3)), device=dev)
        for _ in range(5):
            field.sample(pos)
        stream = torch.cuda.current_stream(dev)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        reps = 200
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            field.sample(pos)
        e1.record(stream)
        torch.cuda.synchronize()
        samp[n] = e0.elapsed_time(e1) / reps * 1e3     # us per call
    res = {"metric": "goal-field bake ms (geodesic distance over free voxels)",
           "value": round(statistics.median(ms), 3), "unit": "ms", "higher_is_better": False,
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "dtype": "f32",
           "data": "synthetic",
           "config": {"workload": name, "grid": f"{nx}x{ny}x{nz}", "voxels": int(w.occ.size),
                      "cell": w.cell, "solid_frac": round(float(w.occ.mean()), 4),
                      "seed_voxels": info["n_seed"], "reach_max": round(info["reach_max"], 3),
                      "sweeps": info["sweeps"], "tile_visits": info["tile_visits"],
                      "visits_per_tile": round(info["tile_visits"] / tiles, 3)},
           "sample": {"us_per_call_2048": round(samp[2048], 3),
                      "us_per_call_1M": round(samp[1 << 20], 3),
                      "G_positions_per_s_1M": round((1 << 20) / (samp[1 << 20] * 1e-6) / 1e9, 3)},
           "reference_torch_gpu": None, "cpu_baseline": None}
    if not args.no_ref and w.occ.size <= 64 * 1024 * 1024:
        _log("[bench] the reference's torch sweep loop on this GPU ...")
        _reference_goal_loop_seconds(occ_dev, w.cell, lo, hi)     # first-call costs
        sweeps, sec = _reference_goal_loop_seconds(occ_dev, w.cell, lo, hi)
        res["reference_torch_gpu"] = {"value": round(sec * 1e3, 1), "unit": "ms", "sweeps": sweeps,
                                      "sample": "goalfield.py:232-270 loop as torch ops on "
                                                "this GPU, one run after a warm-up run"}
    if not args.no_cpu and w.occ.size <= 64 * 1024 * 1024:
        from oracle import goal as ogoal
        t0 = time.perf_counter()
        ogoal.distance(w.occ, w.cell, lo, hi)
        cpu_s = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": round(cpu_s * 1e3, 1), "unit": "ms", "cores": 1,
                               "kind": "port",
                               "sample": "oracle Dijkstra (fp32, binary heap) over the whole "
                                         "grid, one run"}
    print(json.dumps(res), flush=True)


def alg_bytes_per_load(store):
    """Grid bytes per sample: the stored size of a voxel, 4 B fp32, 2 B fp16,
    and for r16 bricks the 2 B code plus its share of the brick's 8 B header
    (base, scale) over 64 voxels."""
    return {"f32": 4.0, "f16": 2.0, "r16": 2.0 + 8.0 / 64.0}[store]


def range_encoding(rng, near):
    """The depth encoding of a ray that reached the range: the kernel's
    fp32 sequence for t = range (t/near at or below near; above it
    near/near + 0.25 * (1 - exp(-(t - near) / 2500)), the exponential
    taken in fp64 and rounded once)."""
    f = np.float32
    t, nr = f(rng), f(near)
    if not t > nr:
        return float(t / nr)
    xe = f(-(t - nr)) / f(2500.0)
    ed = f(math.exp(float(xe)))
    return float(nr / nr + f(0.25) * (f(1.0) - ed))


def step_census(taps, out, w):
    """The per-ray step statistics of the reference's step census
    (tools/bench_lidar.py:188-215): grid loads per ray (mean, median, p90,
    p99, max), the fraction of rays that exhaust the step budget and of rays
    that reach the range (their encoding is the range's), the loop trips
    that do work without an early exit (mean / max_steps); and, for this
    kernel's early exit per tile of 16x4 rays, the fraction of a tile's lane
    trips that do work (lane efficiency)."""
    import torch
    n = taps.shape[0]
    flat = taps.reshape(-1)
    srt = torch.sort(flat).values
    q = [int(srt[min(srt.numel() - 1, int(f * srt.numel()))].item()) for f in (0.5, 0.9, 0.99)]
    mean = float(flat.double().mean().item())
    enc = out.reshape(n, w.height, w.width).float()
    rng_enc = torch.tensor(range_encoding(w.range_units, w.near_range), dtype=torch.float32)
    if out.dtype == torch.bfloat16:
        rng_enc = rng_enc.to(torch.bfloat16).float()
    reach = float((enc == rng_enc.to(enc.device)).double().mean().item())
    eff = None
    if w.height % 4 == 0 and w.width % 16 == 0:
        tile_max = taps.view(n, w.height // 4, 4, w.width // 16, 16).amax(dim=(2, 4))
        eff = round(float(flat.double().sum().item()) / (64.0 * float(tile_max.double().sum().item())), 4)
    return {"loads_mean": round(mean, 3), "median": q[0], "p90": q[1], "p99": q[2],
            "max": int(srt[-1].item()),
            "exhaust_frac": round(float((flat >= w.max_steps).double().mean().item()), 5),
            "reach_range_frac": round(reach, 5),
            "work_frac_without_early_exit": round(mean / w.max_steps, 4),
            "lane_efficiency_per_tile": eff}


def measure_render(w, args, dev, *, graph, steps, warmup, out_shape=None, sc=None):
    """One workload: scene and poses, a lidar with the library defaults (or
    the command line's overrides), a census render (untimed) for the
    algorithmic bytes, then `warmup` untimed and `steps` timed renders back
    to back between two HIP events (eager, or replays of a captured graph),
    and a second pass of `steps` renders with events around each render and
    around each march kernel. Returns the figures as a dict."""
    import torch
    from surfgym import vision
    t0 = time.perf_counter()
    if sc is None:
        sc = w.scene()
    ps = w.poses(sc)
    _log(f"[bench] {w.name}: grid {sc.nz}x{sc.ny}x{sc.nx} baked, {len(ps)} poses "
         f"({time.perf_counter() - t0:.1f} s)")
    gdt = {"f32": torch.float32, "f16": torch.float16, "r16": "r16"}[w.store]
    odt = torch.bfloat16 if w.out_dtype == "bf16" else torch.float32
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, width=w.width, height=w.height,
                                    range_units=w.range_units, near_range=w.near_range,
                                    max_steps=w.max_steps, hit_eps=w.hit_eps, grid_dtype=gdt,
                                    layout=args.layout, schedule=args.schedule,
                                    refill_lanes=args.refill, rays_per_lane=args.rpl,
                                    tile_order=args.tile_order, device=dev)
    origin = torch.as_tensor(ps.origin, device=dev)
    yaw = torch.as_tensor(ps.yaw, device=dev)
    pitch = torch.as_tensor(ps.pitch, device=dev)
    duck = torch.as_tensor(ps.ducked, device=dev)
    n = len(ps)
    out = torch.empty(out_shape(n) if out_shape else (n, w.height, w.width), dtype=odt,
                      device=dev)

    # census (untimed): grid loads per ray -> algorithmic bytes
    taps = torch.empty(n, w.height, w.width, dtype=torch.int32, device=dev)
    lid.render(origin, yaw, pitch, duck, out=out, taps=taps)
    torch.cuda.synchronize()
    loads = int(taps.sum(dtype=torch.int64).item())
    max_taps = int(taps.max().item())
    census = step_census(taps, out, w)
    del taps
    rays = n * w.width * w.height
    out_b = 2 if w.out_dtype == "bf16" else 4
    alg_bytes = int(loads * alg_bytes_per_load(w.store)) + rays * out_b + n * 24
    _log(f"[bench] census: {loads} loads, mean {loads / rays:.2f}/ray, max {max_taps}; "
         f"median {census['median']}, p90 {census['p90']}, p99 {census['p99']}, "
         f"{census['exhaust_frac']:.2%} exhaust the budget, {census['reach_range_frac']:.2%} reach "
         f"the range, lane efficiency {census['lane_efficiency_per_tile']}")

    step = lambda: lid.render(origin, yaw, pitch, duck, out=out)   # noqa: E731
    g = None
    if graph:
        # the rollout step's render as a captured graph (capture on a side
        # stream after an eager warm-up render, then replay on the current one)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            lid.render(origin, yaw, pitch, duck, out=out)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            lid.render(origin, yaw, pitch, duck, out=out)
        step = g.replay
    stream = torch.cuda.current_stream(dev)
    for _ in range(warmup):
        step()
    # events 0 and 1 bracket the timed region: K renders back to back, with
    # nothing else on the stream (event markers between renders would add
    # their own gaps). A second pass of K renders, outside the timed
    # region, records 2 + 4k / 3 + 4k around render k and has the library
    # record 4 + 4k / 5 + 4k around its march kernel; graph replays, whose
    # launches were captured before, take those from K eager renders of the
    # same batch.
    ev = HipEvents(2 + 4 * steps)
    sp = stream.cuda_stream
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    ev.record(0, sp)
    for _ in range(steps):
        step()
    ev.record(1, sp)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    for k in range(steps):
        ev.record(2 + 4 * k, sp)
        step()
        ev.record(3 + 4 * k, sp)
    for k in range(steps):
        lid.set_march_events(ev.ev[4 + 4 * k].value, ev.ev[5 + 4 * k].value)
        lid.render(origin, yaw, pitch, duck, out=out)
    torch.cuda.synchronize()
    lid.set_march_events(None, None)
    total_ms = ev.ms(0, 1)
    launch_ms = [ev.ms(2 + 4 * k, 3 + 4 * k) for k in range(steps)]
    march_ms = [ev.ms(4 + 4 * k, 5 + 4 * k) for k in range(steps)]
    ev.close()
    ms_per_step = total_ms / steps
    kernel_ms = sum(march_ms) / len(march_ms)
    _log(f"[bench] {w.name}: {steps} steps: {ms_per_step:.4f} ms/step (events), wall {wall:.3f} s, "
         f"launch median {statistics.median(launch_ms):.4f} ms; march kernel avg "
         f"{kernel_ms * 1e3:.1f} us, median {statistics.median(march_ms) * 1e3:.1f} us")
    res = {"workload": w.name, "envs": n, "rays": rays, "sc": sc, "lid": lid,
           "grid": f"{sc.nx}x{sc.ny}x{sc.nz} {w.store} @{sc.cell:g}u", "store": w.store,
           "out": w.out_dtype, "out_shape": list(out.shape), "graph": bool(graph),
           "ms_per_step": ms_per_step, "launch_ms_median": statistics.median(launch_ms),
           "march_kernel_ms_avg": kernel_ms, "loads": loads, "alg_bytes": alg_bytes,
           "census": census, "rpl": lid.effective_rays_per_lane(n), "image": out}
    return res


# The reference's lidar phase per 128-decision PPO iteration after its early-exit
# kernel (docs/perf-results.md:86, :415): RTX 5090, surf_src_cannonball (fp16
# grid at 32 u), the live fleet's poses. Context, not a same-scene figure.
REFERENCE_LIDAR_PHASE_MS = 190.4


def lidar_phase(w, args, dev, sc, decisions=128):
    """The trainer's per-decision lidar work for one PPO iteration of
    `decisions` decisions (train_fast.py:1744-1765, the `lidar` phase of
    docs/perf-results.md): each decision copies the (N, 6) pinned pose block
    to the device, then renders from its column views, either straight into
    the image columns of the (N, 15 + H*W) observation row (`out=`) or, as
    the reference does, into a new tensor that is then copied into those
    columns. HIP events bracket each decision's render (+ copy), as the
    trainer's phase timer does, and the whole iteration (+ pose copies)."""
    import torch
    from surfgym import vision
    ps = w.poses(sc)
    n = len(ps)
    gdt = {"f32": torch.float32, "f16": torch.float16, "r16": "r16"}[w.store]
    lid = vision.GpuLidar.from_grid(sc.sdf, sc.mins, sc.cell, width=w.width, height=w.height,
                                    range_units=w.range_units, near_range=w.near_range,
                                    max_steps=w.max_steps, hit_eps=w.hit_eps, grid_dtype=gdt,
                                    layout=args.layout, schedule=args.schedule,
                                    refill_lanes=args.refill, rays_per_lane=args.rpl,
                                    tile_order=args.tile_order, device=dev)
    pin = torch.empty(n, 6, dtype=torch.float32, pin_memory=True)
    pin[:, 0:3] = torch.as_tensor(ps.origin)
    pin[:, 3] = torch.as_tensor(ps.yaw)
    pin[:, 4] = torch.as_tensor(ps.pitch)
    pin[:, 5] = torch.as_tensor(np.asarray(ps.ducked, np.float32))
    vis = torch.empty(n, 6, device=dev)
    scalars = 15
    obs = torch.zeros(n, scalars + w.width * w.height, device=dev)

    def fused():
        lid.render(vis[:, 0:3], vis[:, 3], vis[:, 4], vis[:, 5], out=obs[:, scalars:])

    def reference():
        img = lid.render(vis[:, 0:3], vis[:, 3], vis[:, 4], vis[:, 5])
        obs[:, scalars:].copy_(img.reshape(n, -1))

    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    out = {"workload": w.name, "envs": n, "decisions": decisions,
           "obs_row": f"({n}, {scalars}+{w.height}*{w.width}) f32"}
    images = {}
    for name, body in (("fused", fused), ("reference_sequence", reference)):
        obs.zero_()
        for _ in range(5):
            vis.copy_(pin, non_blocking=True)
            body()
        ev = HipEvents(2 + 2 * decisions)
        torch.cuda.synchronize()
        ev.record(0, sp)
        for k in range(decisions):
            vis.copy_(pin, non_blocking=True)
            ev.record(2 + 2 * k, sp)
            body()
            ev.record(3 + 2 * k, sp)
        ev.record(1, sp)
        torch.cuda.synchronize()
        phase = sum(ev.ms(2 + 2 * k, 3 + 2 * k) for k in range(decisions))
        out[f"{name}_phase_ms"] = round(phase, 3)
        out[f"{name}_iteration_ms"] = round(ev.ms(0, 1), 3)
        ev.close()
        images[name] = obs[:, scalars:].clone()
    out["identical"] = bool(torch.equal(images["fused"], images["reference_sequence"]))
    out["phase_saved_ms"] = round(out["reference_sequence_phase_ms"] - out["fused_phase_ms"], 3)
    out["reference_published_phase_ms"] = REFERENCE_LIDAR_PHASE_MS
    out["reference_published_context"] = ("RTX 5090, surf_src_cannonball fp16 grid at 32 u, the "
                                          "live fleet's poses (docs/perf-results.md:86, :415)")
    _log(f"[bench] lidar phase, {decisions} decisions of {n} envs: fused "
         f"{out['fused_phase_ms']:.2f} ms, render + copy {out['reference_sequence_phase_ms']:.2f} "
         f"ms (the reference's: {REFERENCE_LIDAR_PHASE_MS} ms on its scene and card)")
    del lid
    return out


def config_summary(r, traffic=None, traffic_src=None, limiter=None):
    """A workload's figures for the `configs` object of the JSON line; with
    its profile's L2-miss traffic per launch (None when the profile is
    stale), the rate that traffic streams at over the march kernel's
    average duration, and the unit the profile names as the limit."""
    achieved = r["alg_bytes"] / (r["march_kernel_ms_avg"] * 1e-3) / 1e9
    rate = traffic / (r["march_kernel_ms_avg"] * 1e-3) / 1e9 if traffic else None
    return {"envs": r["envs"], "rays": r["rays"], "grid": r["grid"], "out": r["out"],
            "out_shape": r["out_shape"], "graph": r["graph"],
            "ms_per_batch": round(r["ms_per_step"], 5),
            "g_rays_per_s": round(r["rays"] / (r["ms_per_step"] * 1e-3) / 1e9, 4),
            "march_kernel_ms_avg": round(r["march_kernel_ms_avg"], 5),
            "grid_loads_per_ray": round(r["loads"] / r["rays"], 4),
            "alg_bytes_per_launch": r["alg_bytes"],
            "alg_frac_of_hbm_peak": round(achieved / HBM_PEAK_GBS, 5),
            "census": r.get("census"),
            "traffic_bytes_per_launch": traffic,
            "traffic_gbs": round(rate, 1) if rate else None,
            "traffic_source": traffic_src,
            "limiter": limiter.get("unit") if limiter else None,
            "rays_per_lane": r["rpl"]}


def bench_steps_sweep(args, w, dev, shape):
    """Render time against the step budget (tools/bench_lidar.py:149-156):
    the workload timed at each budget of --steps-sweep, with its census."""
    import dataclasses
    import torch
    sc = w.scene()
    rows = []
    for cap in [int(v) for v in args.steps_sweep.split(",")]:
        r = measure_render(dataclasses.replace(w, max_steps=cap), args, dev, graph=args.graph,
                           steps=args.steps, warmup=args.warmup, out_shape=shape, sc=sc)
        r.pop("lid")
        r.pop("sc")
        r.pop("image")
        rows.append({"max_steps": cap, "ms_per_batch": round(r["ms_per_step"], 5),
                     "march_kernel_ms_avg": round(r["march_kernel_ms_avg"], 5),
                     "g_rays_per_s": round(r["rays"] / (r["ms_per_step"] * 1e-3) / 1e9, 4),
                     "census": r["census"]})
        torch.cuda.empty_cache()
    print(json.dumps({"workload": w.name, "steps_sweep": rows}), flush=True)


# The other workloads of the metric, timed in the same run (GPU legs only):
# (workload, captured graph, output shape)
OTHER_CONFIGS = (("small_ramps", False, None),
                 ("winding_track", False, None),
                 ("sparse_grazing", False, None),
                 ("ramp_field_r16_bf16", True, lambda n: (n, 1, 64, 128)),
                 ("ramp_field_f16_bf16", True, lambda n: (n, 1, 64, 128)))


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="ramp_field")
    ap.add_argument("--layout", default="brick4", choices=["brick4", "linear"])
    ap.add_argument("--schedule", default="tiles", choices=["persistent", "tiles"])
    ap.add_argument("--refill", type=int, default=16, help="free lanes that trigger a refill")
    ap.add_argument("--rpl", type=int, default=None,
                    help="rays per lane, 1 or 2 (default: the library's choice per render: "
                         "1 above 192 MiB and below 65536 tiles, else 2)")
    ap.add_argument("--tile-order", default="lookahead", choices=["lookahead", "launch"],
                    help="order the tiles schedule takes tiles in (library default: lookahead)")
    ap.add_argument("--cpu-envs", type=int, default=2048,
                    help="envs of the workload the CPU baseline renders (default: all of ramp_field)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-copy", action="store_true", help="skip the copy-bandwidth probe")
    ap.add_argument("--no-configs", action="store_true",
                    help="time the one workload only (not the other configurations)")
    ap.add_argument("--config-steps", type=int, default=20,
                    help="timed renders per other configuration")
    ap.add_argument("--bake", action="store_true",
                    help="time the SDF bake (GPU distance transform of the workload's "
                         "occupancy) against the reference's scipy bake instead")
    ap.add_argument("--goal", action="store_true",
                    help="time the goal-field bake and sampler (workloads ramp_field, "
                         "winding_track, maze, small_ramps)")
    ap.add_argument("--no-ref", action="store_true",
                    help="--goal: skip the reference's torch sweep loop")
    ap.add_argument("--graph", action="store_true",
                    help="capture one render in a hipGraph and time graph replays")
    ap.add_argument("--steps-sweep", default=None,
                    help="comma-separated step budgets: time the workload at each (the reference's "
                         "render-ms-vs-MAX_STEPS sweep) and print one JSON line of them instead")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        sys.exit("bench.py measures one GPU: the render is per-env data parallel with no "
                 "exchange, and this build runs on a single MI355X (use --gpus 1)")

    import torch
    from surfgym import synth

    dev = torch.device("cuda:0")
    if args.goal:
        return bench_goal(args, dev)
    w = synth.WORKLOADS[args.workload]
    if args.bake:
        return bench_bake(args, w, dev)
    shape = {n: s for n, _, s in OTHER_CONFIGS}.get(w.name)
    if args.steps_sweep:
        return bench_steps_sweep(args, w, dev, shape)
    r = measure_render(w, args, dev, graph=args.graph, steps=args.steps, warmup=args.warmup,
                       out_shape=shape)
    sc, lid, image = r.pop("sc"), r.pop("lid"), r.pop("image")
    # the last timed render's image, kept for the agreement with the CPU render
    image = (image.float().cpu().numpy()
             if not args.no_cpu and tuple(image.shape) == (r["envs"], w.height, w.width)
             else None)
    n, rays = r["envs"], r["rays"]
    ms_per_step, kernel_ms = r["ms_per_step"], r["march_kernel_ms_avg"]
    achieved = r["alg_bytes"] / (kernel_ms * 1e-3) / 1e9
    rpl = r["rpl"]
    traffic_tab, limiter_tab = profile_records()
    traffic, traffic_src = profiled(f"{w.name} {args.schedule} rpl={rpl} {args.layout} {w.store}"
                                    f" order={lid.tile_order}", traffic_tab, "bytes")
    limiter, limiter_src = profiled(w.name, limiter_tab)
    del lid
    torch.cuda.empty_cache()

    copy_gbs = None if args.no_copy else copy_bandwidth(dev)
    if copy_gbs:
        _log(f"[bench] device copy {copy_gbs:.0f} GB/s")
    res = {
        "metric": METRIC,
        "value": round(rays / (ms_per_step * 1e-3) / 1e9, 4),
        "unit": "G rays/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # the march's arithmetic is fp32 whatever the store: fp16 and r16
        # voxels are widened to fp32 as they are read
        "dtype": "f32",
        "grid_dtype": w.store,
        "out_dtype": w.out_dtype,
        "data": "synthetic",
        "config": {"workload": w.name, "envs": n, "image": f"{w.width}x{w.height}",
                   "rays": rays, "grid": r["grid"],
                   "layout": args.layout, "schedule": args.schedule, "refill_lanes": args.refill,
                   "rays_per_lane": rpl, "tile_order": args.tile_order,
                   "out": w.out_dtype, "max_steps": w.max_steps,
                   "hit_eps": w.hit_eps, "range": round(w.range_units, 3),
                   "near": round(w.near_range, 3),
                   "grid_loads_per_ray": round(r["loads"] / rays, 4),
                   "graph": bool(args.graph),
                   "launch_ms_median": round(r["launch_ms_median"], 5),
                   "march_kernel_ms_avg": round(kernel_ms, 5),
                   "census": r["census"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": traffic,
                     "traffic_gbs": (round(traffic / (kernel_ms * 1e-3) / 1e9, 1)
                                     if traffic else None),
                     "traffic_source": traffic_src,
                     "alg_bytes_per_launch": r["alg_bytes"],
                     "copy_gbs": round(copy_gbs, 1) if copy_gbs else None,
                     "frac_of_copy": round(achieved / copy_gbs, 5) if copy_gbs else None,
                     "limiter": limiter, "limiter_source": limiter_src},
        "configs": None,
        "cpu_baseline": None,
    }
    if not args.no_configs:
        configs = {}
        for name, graph, shape in OTHER_CONFIGS:
            if name == w.name:
                continue
            cw = synth.WORKLOADS[name]
            cr = measure_render(cw, args, dev, graph=graph, steps=args.config_steps,
                                warmup=min(args.warmup, 5), out_shape=shape)
            order = cr.pop("lid").tile_order
            cr.pop("sc")
            cr.pop("image")
            ct, ct_src = profiled(f"{name} {args.schedule} rpl={cr['rpl']} {args.layout} {cw.store}"
                                  f" order={order}", traffic_tab, "bytes")
            cl, _ = profiled(name, limiter_tab)
            configs[name] = config_summary(cr, ct, ct_src, cl)
            torch.cuda.empty_cache()
        configs["lidar_phase"] = lidar_phase(w, args, dev, sc)
        torch.cuda.empty_cache()
        res["configs"] = configs
    if not args.no_cpu:
        envs = min(args.cpu_envs, n)
        _log(f"[bench] cpu baseline on {envs} envs ...")
        res["cpu_baseline"] = cpu_baseline(w, sc, envs,
                                           image=image if envs == n else None)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
