"""sdfr_render_noalloc through the C ABI: the allocation-free variant of
sdfr_render (its workspace is the library's static device scratch) gives
the same images as sdfr_render with a caller workspace, call after call, on
the same GPU; renders whose workspace exceeds the scratch are refused before
any launch; and the call can be captured into a graph with allocations
forbidden (torch's global capture mode) and replayed."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from surfgym import _sdfr, synth

pytestmark = pytest.mark.gpu


class _Handle:
    """A grid handle made through the C ABI from a workload's scene."""

    def __init__(self, dev, name, schedule=None):
        self.lib = _sdfr.load()
        self.w = synth.WORKLOADS[name]
        self.sc = self.w.scene()
        self.src = torch.as_tensor(self.sc.sdf, device=dev).reshape(-1)
        desc = _sdfr.GridDesc(self.sc.nx, self.sc.ny, self.sc.nz,
                              (ctypes.c_float * 3)(*self.sc.mins.tolist()), self.sc.cell)
        err = ctypes.create_string_buffer(256)
        stream = torch.cuda.current_stream(dev).cuda_stream
        self.h = self.lib.sdfr_grid_create(ctypes.byref(desc), self.src.data_ptr(), _sdfr.F32, 1,
                                           _sdfr.F32, _sdfr.LAYOUT_BRICK4, stream, err, len(err))
        assert self.h, err.value
        if schedule is not None:
            assert self.lib.sdfr_grid_set_schedule(self.h, schedule, 16, 0) == 0
        w = self.w
        tan_h = float(np.tan(np.radians(60.0)))
        tan_v = float(np.tan(np.radians(45.0)))
        self.cam = _sdfr.Cam(w.width, w.height, 120.0, 90.0, tan_h, tan_v, w.range_units,
                             w.near_range, w.hit_eps, float(np.float32(0.3 * self.sc.cell)),
                             w.max_steps, _sdfr.CAM_EQUIANGULAR)

    def poses(self, dev, n):
        ps = self.w.poses(self.sc, n)
        keep = [torch.as_tensor(v, device=dev).contiguous()
                for v in (ps.origin, ps.yaw, ps.pitch, ps.ducked)]
        p = _sdfr.Poses(keep[0].data_ptr(), 3, keep[1].data_ptr(), 1, keep[2].data_ptr(), 1,
                        keep[3].data_ptr(), 1, _sdfr.F32, n)
        return p, keep

    def image(self, out):
        n = out.shape[0]
        return _sdfr.Image(out.data_ptr(), out[0].numel() if n > 1 else out.numel(),
                           _sdfr.F32, 1, None)

    def render(self, dev, poses, out):
        need = int(self.lib.sdfr_workspace_bytes(ctypes.byref(self.cam), poses.n_envs))
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        img = self.image(out)
        rc = self.lib.sdfr_render(self.h, ctypes.byref(self.cam), ctypes.byref(poses),
                                  ctypes.byref(img), ws.data_ptr(), need,
                                  torch.cuda.current_stream(dev).cuda_stream)
        assert rc == 0, _sdfr.last_error()
        torch.cuda.synchronize()
        return ws

    def render_noalloc(self, dev, poses, out):
        img = self.image(out)
        return self.lib.sdfr_render_noalloc(self.h, ctypes.byref(self.cam), ctypes.byref(poses),
                                            ctypes.byref(img),
                                            torch.cuda.current_stream(dev).cuda_stream)

    def close(self):
        torch.cuda.synchronize()
        self.lib.sdfr_grid_destroy(self.h)


@pytest.mark.parametrize("schedule", [None, _sdfr.SCHED_PERSISTENT])
def test_noalloc_equals_the_workspace_render_call_after_call(dev, schedule):
    """ramp_field at 2048 envs (sorted tiles, two rays per lane), then 300
    envs (launch order, one ray per lane) on the same scratch: each equals
    sdfr_render's image bit for bit."""
    h = _Handle(dev, "ramp_field", schedule)
    try:
        for n in (2048, 300):
            print(f"case noalloc schedule={schedule} n={n}", flush=True)
            poses, keep = h.poses(dev, n)
            want = torch.full((n, h.w.height, h.w.width), -1.0, device=dev)
            h.render(dev, poses, want)
            got = torch.full_like(want, -2.0)
            rc = h.render_noalloc(dev, poses, got)
            assert rc == 0, _sdfr.last_error()
            torch.cuda.synchronize()
            assert torch.equal(got, want), n
            del keep
    finally:
        h.close()


def test_noalloc_refuses_a_render_beyond_its_scratch(dev):
    h = _Handle(dev, "small_ramps")
    try:
        per_env = int(h.lib.sdfr_workspace_bytes(ctypes.byref(h.cam), 1))
        n_max = _sdfr.NOALLOC_SCRATCH_BYTES // per_env
        n = n_max + 64
        while int(h.lib.sdfr_workspace_bytes(ctypes.byref(h.cam), n)) <= \
                _sdfr.NOALLOC_SCRATCH_BYTES:
            n += 64
        print(f"case noalloc refusal n={n}", flush=True)
        poses, keep = h.poses(dev, n)
        out = torch.full((n, h.w.height, h.w.width), -3.0, device=dev)
        rc = h.render_noalloc(dev, poses, out)
        torch.cuda.synchronize()
        assert rc == -2
        assert "static scratch" in _sdfr.last_error()
        assert bool((out == -3.0).all()), "a refused render must launch nothing"
        # 8192 envs of 128x64, the largest render of the workloads, fits
        assert int(h.lib.sdfr_workspace_bytes(ctypes.byref(h.cam), 8192)) <= \
            _sdfr.NOALLOC_SCRATCH_BYTES
        # and the handle still renders correctly afterwards
        small, keep2 = h.poses(dev, 16)
        want = torch.empty(16, h.w.height, h.w.width, device=dev)
        h.render(dev, small, want)
        got = torch.empty_like(want)
        assert h.render_noalloc(dev, small, got) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    finally:
        h.close()


def test_noalloc_captures_with_allocations_forbidden(dev):
    """Captured in torch's global capture mode (an allocation during the
    capture would be an error), the graph replays the render correctly, with
    eager renders of other poses on the same scratch in between."""
    h = _Handle(dev, "small_ramps")
    try:
        poses, keep = h.poses(dev, 16)
        other, keep2 = h.poses(dev, 5)
        want = torch.empty(16, h.w.height, h.w.width, device=dev)
        h.render(dev, poses, want)
        out = torch.full_like(want, -1.0)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            assert h.render_noalloc(dev, poses, out) == 0
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize()
        print("case noalloc graph capture", flush=True)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, capture_error_mode="global"):
            rc = h.render_noalloc(dev, poses, out)
        assert rc == 0, _sdfr.last_error()
        scratch_out = torch.empty(5, h.w.height, h.w.width, device=dev)
        for i in range(3):
            out.fill_(-1.0)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, want), i
            assert h.render_noalloc(dev, other, scratch_out) == 0
            torch.cuda.synchronize()
    finally:
        h.close()


_FIRST_CALL_IN_CAPTURE = r"""
import sys
sys.path[:0] = sys.argv[1:4]
import torch
import test_zz_no_alloc as t
from surfgym import _sdfr
dev = torch.device("cuda:0")
h = t._Handle(dev, "small_ramps")
poses, keep = h.poses(dev, 16)
want = torch.empty(16, h.w.height, h.w.width, device=dev)
h.render(dev, poses, want)
out = torch.full_like(want, -1.0)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, capture_error_mode="global"):
    rc = h.render_noalloc(dev, poses, out)
assert rc == 0, _sdfr.last_error()
for i in range(3):
    out.fill_(-1.0)
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), i
h.close()
print("first call captured and replayed", flush=True)
"""


def test_the_first_noalloc_call_can_be_a_captured_one():
    """In a fresh process, whose first sdfr_render_noalloc call is made inside
    a global-mode graph capture: the scratch address was looked up when the
    grid was created, so the captured call makes no runtime call a capture
    forbids, and every replay equals sdfr_render's image."""
    import subprocess
    import sys
    from pathlib import Path
    here = Path(__file__).resolve().parent
    print("case noalloc first call inside a capture (child process)", flush=True)
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE, str(here),
                        str(here.parent), str(here.parent / "rl_cs1.6_surf_amd")],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "first call captured and replayed" in r.stdout
