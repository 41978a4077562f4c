#!/usr/bin/env python
"""Benchmark of the MI355X deformable-attention core (one GPU).

Metric (the benchmark definition's headline): fwd+bwd microseconds per call and achieved HBM GB/s
at the RF-DETR Nano group-DETR shape (config 2: batch 8, one 24x24 level, 16 heads x 16, 3900
queries, 2 points, f32). A "step" is one forward + one backward call over that batch, with
inputs already resident in HBM.

Timing: W warm-up steps and then further steps until at least WARM_MS milliseconds of them have
run (a fixed time-based warm-up, so that clocks and caches settle whatever W is), then K steps
launched from Python as a training loop calls the op (each call validates, plans and enqueues its
kernels; the host stays ahead of the GPU) between two events on the launch stream, synchronised on
both sides: `value`. Eager launches are the headline because that is how a training step calls the
op; the same steps replayed from a HIP graph (20 steps per graph) are reported beside it as
`graph_us_per_call` (within about a microsecond of the eager figure at the headline shape, either
side). The dominant call's average duration (the roofline's `avg_launch_us`) is measured the same
way, with events around K eager launches of that call alone, the launch pattern of the rocprofv3
kernel traces in profiles/. per_config times are graph replays (fwd_us, bwd_us, step_us) unless
marked eager.

Roofline: the dominant kernel's algorithmic HBM bytes (Workload.hbm_bytes) against 8 TB/s and its
algorithmic LDS bytes (Workload.lds_bytes) against the LDS read peak measured in the same run by
the library's probe (msda_probe_lds_read); `bound` is the resource whose time is larger. For the
backward, `roofline.lds_atomic` sets grad_value's f64 LDS additions (Workload.lds_atomic_adds)
against the ds_add_f64 rate of a second probe (msda_probe_lds_atomic). Configs
2 and 4 are also timed Infinity-Cache-cold ("cold" in per_config): the steps cycle through enough
copies of the buffers that one pass over them exceeds the 256 MiB cache.

CPU baseline: the repository's C restatement of the reference gather path (oracle/msda_ref.c,
OpenMP over slices) on the same inputs, on this host's cores (at most 16), rank 0 only.

``--gpus N`` with N > 1 exits: this build runs on one GPU (the op needs no collective; each GPU of
a data-parallel job runs it on its own batch shard).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "rf-detr-jax_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "deform-attn fwd+bwd μs/call + achieved HBM GB/s (% peak), Nano group-DETR shape"
HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E
LDS_PEAK_NOMINAL_GBPS = 256 * 128 * 2.4  # 256 CUs x 128 B/clk x 2.4 GHz, used only if the probe fails
MALL_BYTES = 256 << 20  # MI355X Infinity Cache
WARM_MS = 150.0  # time-based warm-up before the first timed step of a workload


def log(msg):
    sys.stderr.write(f"[bench] {msg}\n")
    sys.stderr.flush()


class Calls:
    """Pre-built C-ABI argument lists and output buffers for one workload (minimal host overhead)."""

    def __init__(self, w, dev):
        import torch

        from rfdetr_jax_amd import _native
        from rfdetr_jax_amd.workloads import workload_inputs

        self.w = w
        value, loc, attn, grad = workload_inputs(w, with_grad=True)
        bf16 = w.value_dtype == "bf16"
        self.v = torch.from_numpy(value).to(dev)
        if bf16:
            self.v = self.v.to(torch.bfloat16)
        self.loc = torch.from_numpy(loc).to(dev)
        self.attn = torch.from_numpy(attn).to(dev)
        self.grad = torch.from_numpy(grad).to(dev)
        self.out = torch.empty(w.batch, w.queries, w.heads * w.head_dim, device=dev)
        self.dv = torch.empty_like(self.v)
        self.dloc = torch.empty_like(self.loc)
        self.dattn = torch.empty_like(self.attn)
        self.host = (value, loc, attn, grad)
        flat = [x for hw in w.shapes for x in hw]
        self._shapes = (ctypes.c_int32 * len(flat))(*flat)
        starts, acc = [], 0
        for h, wd in w.shapes:
            starts.append(acc)
            acc += h * wd
        self._starts = (ctypes.c_int32 * len(starts))(*starts)
        vdt = _native.DTYPE_BF16 if bf16 else _native.DTYPE_F32
        shape_args = (w.batch, w.heads, w.head_dim, w.queries, w.levels, w.points, self._shapes, self._starts,
                      w.len_value)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        self.lib = _native.lib()
        ws_bytes = self.lib.msda_bwd_workspace_size(*shape_args)
        if ws_bytes < 0:
            _native.check(int(ws_bytes))
        self.ws = torch.empty((max(1, ws_bytes // 16), 4), dtype=torch.int32, device=dev)  # per-sample records
        self.fargs = (p(self.v), vdt, p(self.loc), p(self.attn), p(self.out), _native.DTYPE_F32) + shape_args
        self.bargs = (p(self.v), vdt, p(self.loc), p(self.attn), p(self.grad), _native.DTYPE_F32, p(self.dv),
                      p(self.dloc), p(self.dattn)) + shape_args + (p(self.ws), ctypes.c_int64(ws_bytes))
        self.check = _native.check

    def fwd(self, stream):
        rc = self.lib.msda_fwd(*self.fargs, stream)
        if rc:
            self.check(rc)

    def bwd(self, stream):
        rc = self.lib.msda_bwd(*self.bargs, stream)
        if rc:
            self.check(rc)


class FusedCalls:
    """Pre-built C-ABI calls of the fused-prologue op (msda_fused_fwd / msda_fused_bwd) on a
    workload's shape: box reference points, raw offsets and logits in, every gradient out."""

    def __init__(self, w, dev, ref_dim=4):
        import torch

        from rfdetr_jax_amd import _native
        from rfdetr_jax_amd.workloads import make_fused_inputs

        self.w = w
        value, ref, off, logits, grad = make_fused_inputs(w.cfg_id, w.batch, w.heads, w.head_dim, w.queries, w.shapes,
                                                          w.points, ref_dim, w.value_dtype)
        bf16 = w.value_dtype == "bf16"
        t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
        self.v = t(value).to(torch.bfloat16) if bf16 else t(value)
        self.ref, self.off, self.logits, self.grad = t(ref), t(off), t(logits), t(grad)
        self.out = torch.empty(w.batch, w.queries, w.heads * w.head_dim, device=dev)
        self.dv = torch.empty_like(self.v)
        self.dref, self.doff, self.dlog = torch.empty_like(self.ref), torch.empty_like(self.off), torch.empty_like(self.logits)
        flat = [x for hw in w.shapes for x in hw]
        self._shapes = (ctypes.c_int32 * len(flat))(*flat)
        starts, acc = [], 0
        for h, wd in w.shapes:
            starts.append(acc)
            acc += h * wd
        self._starts = (ctypes.c_int32 * len(starts))(*starts)
        vdt = _native.DTYPE_BF16 if bf16 else _native.DTYPE_F32
        shape_args = (w.batch, w.heads, w.head_dim, w.queries, w.levels, w.points, self._shapes, self._starts,
                      w.len_value)
        p = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
        self.lib = _native.lib()
        ws_bytes = self.lib.msda_fused_bwd_workspace_size(w.batch, w.heads, w.head_dim, w.queries, w.levels, w.points,
                                                          ref_dim, self._shapes, self._starts, w.len_value)
        if ws_bytes < 0:
            _native.check(int(ws_bytes))
        self.ws = torch.empty((max(1, ws_bytes // 16), 4), dtype=torch.int32, device=dev)
        self.fargs = (p(self.v), vdt, p(self.ref), ref_dim, p(self.off), p(self.logits), p(self.out),
                      _native.DTYPE_F32) + shape_args
        self.bargs = (p(self.v), vdt, p(self.ref), ref_dim, p(self.off), p(self.logits), p(self.grad), _native.DTYPE_F32,
                      p(self.dv), p(self.doff), p(self.dlog), p(self.dref)) + shape_args + (p(self.ws), ctypes.c_int64(ws_bytes))
        self.check = _native.check
        # the same step with the prologue in torch around the core op (what the fused op replaces)
        self.core = Calls(w, dev)
        self.core_loc = torch.empty_like(self.off)
        self.core_attn = torch.empty_like(self.logits)

    def fwd(self, stream):
        rc = self.lib.msda_fused_fwd(*self.fargs, stream)
        if rc:
            self.check(rc)

    def bwd(self, stream):
        rc = self.lib.msda_fused_bwd(*self.bargs, stream)
        if rc:
            self.check(rc)

    def unfused_step(self, stream):
        """ops.py:395-404 in torch, msda_fwd, msda_bwd, then the prologue's VJP in torch."""
        import torch

        c, P = self.core, float(self.w.points)
        wh = self.ref[:, :, None, :, None, 2:]
        t = self.off / P
        torch.add(self.ref[:, :, None, :, None, :2], t * wh * 0.5, out=c.loc)
        c.attn.copy_(torch.softmax(self.logits, dim=-1))
        c.fwd(stream)
        c.bwd(stream)
        half = c.dloc * 0.5
        torch.div(half * wh, P, out=self.doff)
        self.dref[..., :2] = c.dloc.sum(dim=(2, 4))
        self.dref[..., 2:] = (half * t).sum(dim=(2, 4))
        self.dlog.copy_(torch.ops.aten._softmax_backward_data(c.dattn, c.attn, -1, torch.float32))


def _stream_handle():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def time_graph(fn, reps, iters_per_graph=20):
    """Average device time (us) of ``fn`` (which enqueues work on the current stream) by replaying
    a HIP graph holding ``iters_per_graph`` copies of it ``ceil(reps / iters_per_graph)`` times."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(_stream_handle())  # warm inside the capture stream's context
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        h = _stream_handle()
        for _ in range(iters_per_graph):
            fn(h)
    replays = max(1, -(-reps // iters_per_graph))
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / (replays * iters_per_graph), replays * iters_per_graph


def time_eager(fn, reps):
    import torch

    h = _stream_handle()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn(h)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / reps


def warm_up(step, warmup, min_ms=WARM_MS):
    """`warmup` steps, then more until at least `min_ms` of wall time has passed (synchronised)."""
    import torch

    h = _stream_handle()
    for _ in range(warmup):
        step(h)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < min_ms:
        for _ in range(10):
            step(h)
        torch.cuda.synchronize()


def measure(w, dev, steps, warmup):
    calls = Calls(w, dev)

    def step(hs):
        calls.fwd(hs)
        if w.backward:
            calls.bwd(hs)

    warm_up(step, warmup)

    res = {}
    res["step_us_graph"], res["graph_steps"] = time_graph(step, steps)
    res["step_us_eager"] = time_eager(step, steps)
    res["fwd_us"] = time_graph(calls.fwd, steps)[0]
    res["fwd_us_eager"] = time_eager(calls.fwd, steps)
    if w.backward:
        res["bwd_us"] = time_graph(calls.bwd, steps)[0]
        res["bwd_us_eager"] = time_eager(calls.bwd, steps)
    b = w.hbm_bytes()
    res["hbm_bytes"] = b
    res["fwd_gbps"] = b["fwd"] / res["fwd_us"] / 1e3
    if w.backward:
        res["bwd_gbps"] = b["bwd"] / res["bwd_us"] / 1e3
    res["step_gbps"] = b["total"] / res["step_us_graph"] / 1e3
    res["step_gbps_eager"] = b["total"] / res["step_us_eager"] / 1e3
    return res, calls


def measure_fused(w, dev, steps, warmup):
    """The fused-prologue op on a workload's shape, beside the same step with the prologue in torch."""
    fc = FusedCalls(w, dev)
    h = _stream_handle()
    for _ in range(warmup):
        fc.fwd(h)
        fc.bwd(h)
        fc.unfused_step(h)

    def step(hs):
        fc.fwd(hs)
        fc.bwd(hs)

    return {
        "fused_step_us": round(time_graph(step, steps)[0], 3),
        "fused_fwd_us": round(time_graph(fc.fwd, steps)[0], 3),
        "fused_bwd_us": round(time_graph(fc.bwd, steps)[0], 3),
        "unfused_step_us": round(time_graph(fc.unfused_step, steps)[0], 3),
        "reference_points": "boxes [B,Q,L,4]",
    }


def measure_point_sample(dev, steps, masks=400, size=112, ratio=16):
    """The segmentation loss's point sampling (criterion.py:482-488, segmentation.py:200-233) on
    one-channel size x size mask logits: point_sample on 3 x P uncertainty candidates, on the P
    chosen points with the gradient of the logits, and nearest sampling of the labels at the same
    points (P = size^2 / ratio). Beside it, the same three samplings with torch's F.grid_sample."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    from rfdetr_jax_amd import _native
    from rfdetr_jax_amd.grid_sample import grid_sample_backward, grid_sample_forward

    rng = np.random.default_rng(7)
    npts = size * size // ratio
    logits = torch.from_numpy(rng.standard_normal((masks, 1, size, size), dtype=np.float32)).to(dev)
    labels = torch.from_numpy((rng.uniform(0, 1, (masks, 1, size, size)) > 0.5).astype(np.float32)).to(dev)
    cand = torch.from_numpy(rng.uniform(0, 1, (masks, 3 * npts, 2)).astype(np.float32)).to(dev)
    pts = torch.from_numpy(rng.uniform(0, 1, (masks, npts, 2)).astype(np.float32)).to(dev)
    gout = torch.from_numpy(rng.standard_normal((masks, 1, npts), dtype=np.float32)).to(dev)
    unit, border = _native.GRID_UNIT_POINTS, _native.PADDING["border"]
    bil, near = _native.SAMPLE_BILINEAR, _native.SAMPLE_NEAREST

    def ours(_h):
        grid_sample_forward(logits, cand, unit, border, bil)
        grid_sample_forward(logits, pts, unit, border, bil)
        grid_sample_backward(logits, pts, gout, unit, border, bil, needs=(True, False))
        grid_sample_forward(labels, pts, unit, border, near)

    cgrid, pgrid = (2 * cand - 1)[:, :, None, :], (2 * pts - 1)[:, :, None, :]
    lg = logits.clone().requires_grad_(True)

    def torch_step(_h):
        with torch.no_grad():
            F.grid_sample(logits, cgrid, mode="bilinear", padding_mode="border", align_corners=False)
        out = F.grid_sample(lg, pgrid, mode="bilinear", padding_mode="border", align_corners=False)
        torch.autograd.grad(out, lg, gout[..., None])
        with torch.no_grad():
            F.grid_sample(labels, pgrid, mode="nearest", padding_mode="border", align_corners=False)

    for _ in range(3):
        ours(None)
        torch_step(None)
    torch.cuda.synchronize()
    return {
        "masks": masks, "mask_size": size, "points": npts, "candidates": 3 * npts,
        "step_us": round(time_graph(ours, steps)[0], 3),
        "torch_grid_sample_step_us": round(time_eager(torch_step, steps), 3),
        "step_us_eager": round(time_eager(ours, steps), 3),
    }


def measure_value_proj(dev, steps, batch=8, seq=576, d_model=256, heads=16):
    """MSDeformAttn's value path at the config-2 memory shape (8 x 24x24 positions, d_model 256, 16
    heads): the fused projection (msda_value_proj_fwd, then _bwd for all three gradients) beside
    torch's F.linear + masked_fill + view/permute/contiguous and its autograd backward."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    from rfdetr_jax_amd.value_proj import value_proj_backward, value_proj_forward

    rng = np.random.default_rng(9)
    x = torch.from_numpy(rng.standard_normal((batch, seq, d_model), dtype=np.float32)).to(dev)
    w = torch.from_numpy((rng.standard_normal((d_model, d_model)) / 16).astype(np.float32)).to(dev)
    b = torch.from_numpy(rng.standard_normal(d_model).astype(np.float32)).to(dev)
    mask = torch.from_numpy(rng.uniform(0, 1, (batch, seq)) < 0.05).to(dev)
    d = d_model // heads
    gv = torch.from_numpy(rng.standard_normal((batch * heads, seq, d), dtype=np.float32)).to(dev)

    def ours(_h):
        value_proj_forward(x, w, b, heads, mask)
        value_proj_backward(x, w, heads, gv, mask)

    xt, wt, bt = (t.clone().requires_grad_(True) for t in (x, w, b))

    def torch_step(_h):
        y = F.linear(xt, wt, bt).masked_fill(mask[..., None], 0.0)
        v = y.view(batch, seq, heads, d).permute(0, 2, 1, 3).reshape(batch * heads, seq, d)
        torch.autograd.grad(v, (xt, wt, bt), gv)

    for _ in range(3):
        ours(None)
        torch_step(None)
    torch.cuda.synchronize()
    return {
        "shape": {"batch": batch, "len_in": seq, "d_model": d_model, "heads": heads},
        "fwd_us": round(time_graph(lambda h: value_proj_forward(x, w, b, heads, mask), steps)[0], 3),
        "step_us": round(time_graph(ours, steps)[0], 3),
        "step_us_eager": round(time_eager(ours, steps), 3),
        "torch_step_us_eager": round(time_eager(torch_step, steps), 3),
    }


def measure_attention(dev, steps, batch=8, groups=13, per=300, heads=8, head_dim=32, dtype="f32"):
    """The decoder's grouped self-attention at the config-2 shape (8 images x 13 groups x 300
    queries, 8 heads x 32, f32): the attention alone (msda_attention_fwd, then _bwd for q, k and v)
    on the [B, G * P, C] rows in place, beside torch's F.scaled_dot_product_attention on the same
    tensors split into groups and heads (the reference's _split_groups + head transposes) with its
    autograd backward. Algorithmic FLOPs: forward 4 L^2 D per (slice, head) (two products), backward
    twice that (dV, dP, dQ, dK; the kernels' recomputation of the scores is not counted). Also the
    step with the backward's two kernels (MSDA_ATTN_FUSED=0) in place of the fused one."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    from rfdetr_jax_amd.attention import _Layout, attention_backward, attention_forward

    c = heads * head_dim
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    rng = np.random.default_rng(10)
    qk = torch.from_numpy(rng.standard_normal((batch, groups * per, 2 * c), dtype=np.float32)).to(dev, tdt)
    v = torch.from_numpy(rng.standard_normal((batch, groups * per, c), dtype=np.float32)).to(dev, tdt)
    g = torch.from_numpy(rng.standard_normal((batch, groups * per, c), dtype=np.float32)).to(dev, tdt)
    q, k = qk[..., :c], qk[..., c:]
    lay = _Layout(batch, groups, heads, per, head_dim)
    out, stats = attention_forward(q, k, v, lay, lay.strides_rows)

    def fwd(_h):
        attention_forward(q, k, v, lay, lay.strides_rows)

    def ours(_h):
        o, st = attention_forward(q, k, v, lay, lay.strides_rows)
        attention_backward(q, k, v, o, st, g, lay, lay.strides_rows)

    def split(x):  # [B, G P, C] -> [G B, H, P, D]
        return x.reshape(batch, groups, per, heads, head_dim).permute(1, 0, 3, 2, 4).reshape(groups * batch, heads, per, head_dim)

    tq, tk, tv = (split(x).detach().clone().requires_grad_(True) for x in (q, k, v))
    tg = split(g).contiguous()

    def torch_step(_h):
        o = F.scaled_dot_product_attention(tq, tk, tv)
        torch.autograd.grad(o, (tq, tk, tv), tg)

    for _ in range(3):
        ours(None)
        torch_step(None)
    torch.cuda.synchronize()
    flops_fwd = 4 * per * per * head_dim * batch * groups * heads
    fwd_us = time_graph(fwd, steps)[0]
    step_us = time_graph(ours, steps)[0]
    # the same step with the backward's two kernels (each forming S, P and dP) instead of the fused one
    from rfdetr_jax_amd import _native

    lib = _native.lib()
    _native.check(lib.msda_set_tuning(b"MSDA_ATTN_FUSED", b"0"))
    try:
        step_split_us = time_graph(ours, steps)[0]
    finally:
        lib.msda_set_tuning(b"MSDA_ATTN_FUSED", None)
    return {
        "shape": {"batch": batch, "groups": groups, "queries_per_group": per, "heads": heads, "head_dim": head_dim, "dtype": dtype},
        "fwd_us": round(fwd_us, 3),
        "step_us": round(step_us, 3),
        "step_us_two_kernel_backward": round(step_split_us, 3),
        "fwd_tflops": round(flops_fwd / fwd_us / 1e6, 1),
        "step_tflops": round(3 * flops_fwd / step_us / 1e6, 1),
        "torch_step_us_eager": round(time_eager(torch_step, steps), 3),
    }


def lds_peak(dev, blocks=5120, reps=256, trials=5):
    """Device LDS read bandwidth (GB/s), measured with the library's probe (msda_probe_lds_read:
    ds_read_b128, contiguous 1 KB per wave instruction) on the current stream: best of `trials`."""
    import torch

    from rfdetr_jax_amd import _native

    lib = _native.lib()
    out = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    ptr = ctypes.c_void_p(out.data_ptr())
    nbytes = lib.msda_probe_lds_read_bytes(blocks, reps)
    h = _stream_handle()
    _native.check(0 if lib.msda_probe_lds_read(ptr, blocks, reps, h) == 0 else _native.ERR_LAUNCH)
    torch.cuda.synchronize()
    best = None
    for _ in range(trials):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        lib.msda_probe_lds_read(ptr, blocks, reps, h)
        end.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(end) * 1000.0
        best = us if best is None else min(best, us)
    return {"gbps": round(nbytes / best / 1e3, 1), "bytes": nbytes, "us": round(best, 3), "blocks": blocks, "reps": reps,
            "probe": "msda_probe_lds_read (ds_read_b128, 1 KB per wave instruction)"}


def lds_atomic_peak(dev, blocks=5120, reps=64, trials=5, f32=False):
    """Device LDS atomic-add rate (lane additions per second), measured with the library's probe
    (msda_probe_lds_atomic: ds_add_f64, or with f32 msda_probe_lds_atomic_f32: ds_add_f32; each wave
    instruction on 64 consecutive elements) on the current stream: best of `trials`; the probe's
    sums are checked."""
    import torch

    from rfdetr_jax_amd import _native

    lib = _native.lib()
    probe = lib.msda_probe_lds_atomic_f32 if f32 else lib.msda_probe_lds_atomic
    out = torch.empty(blocks * 256, dtype=torch.float32 if f32 else torch.float64, device=dev)
    ptr = ctypes.c_void_p(out.data_ptr())
    ops = lib.msda_probe_lds_atomic_ops(blocks, reps)
    h = _stream_handle()
    _native.check(0 if probe(ptr, blocks, reps, h) == 0 else _native.ERR_LAUNCH)
    torch.cuda.synchronize()
    if not bool(torch.all(out == 16.0 * reps).item()):
        raise RuntimeError("LDS atomic probe: wrong sums")
    best = None
    for _ in range(trials):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        probe(ptr, blocks, reps, h)
        end.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(end) * 1000.0
        best = us if best is None else min(best, us)
    name = "msda_probe_lds_atomic_f32 (ds_add_f32" if f32 else "msda_probe_lds_atomic (ds_add_f64"
    return {"gops": round(ops / best / 1e3, 1), "ops": ops, "us": round(best, 3), "blocks": blocks, "reps": reps,
            "probe": f"{name}, 64 consecutive elements per wave instruction)"}


def measure_cold(w, dev, steps):
    """The step with its inputs and outputs not cache-resident: enough copies of the workload's
    buffers (at least three) that one pass over them exceeds the 256 MiB Infinity Cache; the steps
    cycle through the copies (HIP graph replays, and eager launches for step_us_eager), so each
    step finds its data evicted by the steps of the other copies."""
    per_set = w.hbm_bytes()["total"]
    sets = max(3, -(-(MALL_BYTES + (64 << 20)) // per_set))
    calls = [Calls(w, dev) for _ in range(sets)]

    def step(h):
        for c in calls:
            c.fwd(h)
            if w.backward:
                c.bwd(h)

    def only(k):
        def fn(h):
            for c in calls:
                getattr(c, k)(h)
        return fn

    reps = max(1, steps // sets)
    res = {"sets": sets, "bytes_per_set": per_set}
    us, n = time_graph(step, reps, iters_per_graph=max(1, min(20, reps)))
    res["step_us"] = round(us / sets, 3)
    res["step_us_eager"] = round(time_eager(step, reps) / sets, 3)
    res["fwd_us"] = round(time_graph(only("fwd"), reps, iters_per_graph=max(1, min(20, reps)))[0] / sets, 3)
    if w.backward:
        res["bwd_us"] = round(time_graph(only("bwd"), reps, iters_per_graph=max(1, min(20, reps)))[0] / sets, 3)
    res["step_hbm_frac"] = round(per_set / (res["step_us"] * 1e3) / HBM_PEAK_GBPS, 4)
    del calls
    return res


def cpu_baseline(calls, budget_s=3.0, max_reps=20):
    """fwd+bwd of the C oracle on the same inputs; median us/call."""
    from oracle import cref

    value, loc, attn, grad = calls.host
    w = calls.w
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    threads = max(1, min(16, cores))
    times = []
    t_end = time.perf_counter() + budget_s
    cref.forward(value, w.shapes, loc, attn, threads)  # warm-up
    while len(times) < max_reps and (not times or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        cref.forward(value, w.shapes, loc, attn, threads)
        if w.backward:
            cref.backward(value, w.shapes, loc, attn, grad, threads)
        times.append(time.perf_counter() - t0)
    return {
        "value": statistics.median(times) * 1e6,
        "unit": "us/call",
        "cores": threads,
        "kind": "port",
        "sample": (f"full {w.name} workload (B={w.batch}, Q={w.queries}, levels={list(w.shapes)}, "
                   f"{w.heads}x{w.head_dim}, P={w.points}) {'fwd+bwd' if w.backward else 'fwd'}, "
                   f"median of {len(times)} runs of oracle/msda_ref.c (f32, OpenMP, {threads} threads)"),
    }


def profile_run(w, dev, steps, warmup, copy_mb, fused=False):
    """Eager launches only (every dispatch visible to a counter profiler), plus a copy kernel."""
    import torch

    calls = FusedCalls(w, dev) if fused else Calls(w, dev)
    h = _stream_handle()
    for _ in range(warmup):
        calls.fwd(h)
        if w.backward:
            calls.bwd(h)
    torch.cuda.synchronize()
    fwd_us = time_eager(calls.fwd, steps)
    bwd_us = time_eager(calls.bwd, steps) if w.backward else None
    n = copy_mb * (1 << 20) // 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    copy_us = time_eager(lambda _h: dst.copy_(src), steps)
    print(json.dumps({"workload": w.name, "steps": steps, "fwd_us_eager": fwd_us, "bwd_us_eager": bwd_us,
                      "copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "copy_us": copy_us,
                      "hbm_bytes": w.hbm_bytes()}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2, help="workload id (default 2: the headline shape)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-per-config", action="store_true", help="skip timing the other four workloads")
    ap.add_argument("--profile", action="store_true",
                    help="for rocprofv3 runs: W + K eager steps of the workload, then K plain copies of a "
                         "--copy-mb buffer (counter calibration); prints one JSON line of timings")
    ap.add_argument("--copy-mb", type=int, default=256)
    ap.add_argument("--fused", action="store_true", help="with --profile: the fused-prologue op instead of the core")
    ap.add_argument("--profile-point-sample", action="store_true",
                    help="for rocprofv3 runs: K eager steps of the segmentation loss's point sampling, ours then torch's")
    ap.add_argument("--profile-value-proj", action="store_true",
                    help="for rocprofv3 runs: K eager steps of the value projection fwd+bwd, ours then torch's")
    ap.add_argument("--profile-attention", action="store_true",
                    help="for rocprofv3 runs: K steps of the decoder self-attention fwd+bwd, ours then torch's")
    ap.add_argument("--attention-dtype", choices=["f32", "bf16"], default="f32", help="with --profile-attention")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}): the deformable-attention op needs no "
              "collective, so each GPU of a data-parallel job runs it on its own batch shard.", file=sys.stderr)
        sys.exit(2)

    import torch

    from rfdetr_jax_amd.workloads import CONFIGS

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    w = CONFIGS[args.config]
    if args.profile:
        profile_run(w, dev, args.steps, args.warmup, args.copy_mb, args.fused)
        return
    if args.profile_point_sample:
        print(json.dumps(measure_point_sample(dev, args.steps)), flush=True)
        return
    if args.profile_value_proj:
        print(json.dumps(measure_value_proj(dev, args.steps)), flush=True)
        return
    if args.profile_attention:
        print(json.dumps(measure_attention(dev, args.steps, dtype=args.attention_dtype)), flush=True)
        return
    log(f"workload {w.name}: warmup {args.warmup}, steps {args.steps}")
    res, calls = measure(w, dev, args.steps, args.warmup)
    log(f"step {res['step_us_graph']:.2f} us (graph), {res['step_us_eager']:.2f} us (eager); fwd {res['fwd_us']:.2f} us"
        + (f", bwd {res['bwd_us']:.2f} us" if w.backward else ""))

    log("LDS peak (probe)")
    try:
        lds = lds_peak(dev)
    except Exception as e:  # the probe is a measurement aid; the roofline then uses the nominal peak
        log(f"LDS probe failed ({e}); nominal {LDS_PEAK_NOMINAL_GBPS:.0f} GB/s")
        lds = {"gbps": LDS_PEAK_NOMINAL_GBPS, "probe": "nominal (probe failed)"}
    lds_peak_gbps = lds["gbps"]
    log(f"LDS read peak {lds_peak_gbps:.0f} GB/s")
    atom = atom32 = None
    if w.backward:
        try:
            atom = lds_atomic_peak(dev)
            log(f"LDS f64 atomic-add peak {atom['gops']:.0f} G lane-adds/s")
            atom32 = lds_atomic_peak(dev, blocks=1024, reps=4, f32=True)
            log(f"LDS f32 atomic-add rate {atom32['gops']:.0f} G lane-adds/s")
        except Exception as e:  # a measurement aid: the entry is left out
            log(f"LDS atomic probe failed ({e})")

    kernels = {"fwd": (res["fwd_us_eager"], res["hbm_bytes"]["fwd"])}
    if w.backward:
        kernels["bwd"] = (res["bwd_us_eager"], res["hbm_bytes"]["bwd"])
    dom = max(kernels, key=lambda k: kernels[k][0])
    dom_us, dom_bytes = kernels[dom]
    dom_lds = w.lds_bytes()[dom]
    t_hbm = dom_bytes / HBM_PEAK_GBPS / 1e3  # us
    t_lds = dom_lds / lds_peak_gbps / 1e3
    bound = "hbm" if t_hbm >= t_lds else "lds"
    achieved = (dom_bytes if bound == "hbm" else dom_lds) / dom_us / 1e3
    peak = HBM_PEAK_GBPS if bound == "hbm" else lds_peak_gbps
    traffic = None
    lds_counters = None
    tfile = os.path.join(ROOT, "profiles", f"traffic_{w.name}.json")
    if os.path.exists(tfile):
        # calibrated FETCH_SIZE + WRITE_SIZE of the kernel, from the rocprofv3 counter passes that file records
        tinfo = json.load(open(tfile))
        traffic = tinfo.get("kernels", {}).get(dom, {}).get("hbm_bytes_per_launch")
        lds_counters = tinfo.get("lds", {}).get(dom)

    per_config = {}
    if not args.no_per_config:
        for cid, cw in sorted(CONFIGS.items()):
            if cid == args.config:
                r = res
            else:
                log(f"workload {cw.name}")
                r, _ = measure(cw, dev, max(50, args.steps // 4), 10)
            lb = cw.lds_bytes()
            entry = {"step_us": round(r["step_us_graph"], 3), "step_us_eager": round(r["step_us_eager"], 3),
                     "fwd_us": round(r["fwd_us"], 3),
                     "fwd_hbm_gbps": round(r["fwd_gbps"], 1), "hbm_bytes": r["hbm_bytes"]["total"],
                     "step_hbm_frac": round(r["step_gbps"] / HBM_PEAK_GBPS, 4),
                     "lds_bytes": lb["total"], "fwd_lds_gbps": round(lb["fwd"] / r["fwd_us"] / 1e3, 1),
                     "step_lds_frac": round(lb["total"] / r["step_us_graph"] / 1e3 / lds_peak_gbps, 4)}
            if cw.backward:
                entry.update({"bwd_us": round(r["bwd_us"], 3), "bwd_us_eager": round(r["bwd_us_eager"], 3),
                              "bwd_hbm_gbps": round(r["bwd_gbps"], 1),
                              "bwd_lds_gbps": round(lb["bwd"] / r["bwd_us"] / 1e3, 1)})
                if atom is not None:
                    entry["bwd_atomic_frac"] = round(cw.lds_atomic_adds() / atom["gops"] / 1e3 / r["bwd_us_eager"], 4)
            if cid in (2, 4):
                log(f"workload {cw.name}: Infinity-Cache-cold steps")
                entry["cold"] = measure_cold(cw, dev, max(60, args.steps // 2))
            per_config[cw.name] = entry
        if w.backward:
            log("fused prologue")
            per_config[f"fused_prologue_{w.name}"] = measure_fused(w, dev, max(50, args.steps // 2), 10)
        log("value projection")
        per_config["value_proj_b8_s576_c256_h16"] = measure_value_proj(dev, max(50, args.steps // 2))
        log("decoder self-attention")
        per_config["self_attention_b8_g13_p300_h8_d32_f32"] = measure_attention(dev, max(20, args.steps // 8))
        per_config["self_attention_b8_g13_p300_h8_d32_bf16"] = measure_attention(dev, max(20, args.steps // 8), dtype="bf16")
        log("point sample (segmentation loss)")
        per_config["point_sample_mask_loss_400x112x112"] = measure_point_sample(dev, max(50, args.steps // 2))

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(calls)
        log(f"cpu {cpu['value']:.0f} us/call on {cpu['cores']} threads")

    line = {
        "metric": METRIC,
        "value": round(res["step_us_eager"], 3),
        "unit": "us/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["step_us_eager"] / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w.value_dtype == "bf16" else "f32",
        "data": "synthetic (seeded N(0,1) value, U[0,1]^2 + N(0,0.05) locations, softmax weights, N(0,1) grad)",
        "config": {"workload": w.name, "batch": w.batch, "heads": w.heads, "head_dim": w.head_dim,
                   "queries": w.queries, "levels": [list(s) for s in w.shapes], "points": w.points,
                   "value_dtype": w.value_dtype, "mode": "fwd+bwd" if w.backward else "fwd"},
        "achieved_hbm_gbps": round(res["step_gbps_eager"], 1),
        "hbm_peak_frac": round(res["step_gbps_eager"] / HBM_PEAK_GBPS, 4),
        "graph_us_per_call": round(res["step_us_graph"], 3),
        "cold_us_per_call": per_config.get(w.name, {}).get("cold", {}).get("step_us_eager"),
        "roofline": {"bound": bound, "kernel": dom, "achieved": round(achieved, 1), "peak": peak,
                     "unit": "GB/s", "frac": round(achieved / peak, 4), "traffic": traffic,
                     "algorithmic_bytes": dom_bytes, "avg_launch_us": round(dom_us, 3),
                     "hbm": {"algorithmic_bytes": dom_bytes, "achieved": round(dom_bytes / dom_us / 1e3, 1),
                             "peak": HBM_PEAK_GBPS, "time_us": round(t_hbm, 3)},
                     "lds": {"algorithmic_bytes": dom_lds, "achieved": round(dom_lds / dom_us / 1e3, 1),
                             "peak": lds_peak_gbps, "peak_source": lds.get("probe"), "time_us": round(t_lds, 3),
                             "counters": lds_counters}},
        "cpu_baseline": cpu,
        "per_config": per_config,
    }
    if dom == "bwd" and atom is not None:
        # grad_value's f64 LDS additions against the probe's rate: the backward's LDS-atomic bound
        adds = w.lds_atomic_adds()
        line["roofline"]["lds_atomic"] = {"adds": adds, "achieved_gops": round(adds / dom_us / 1e3, 1), "peak_gops": atom["gops"],
                                          "peak_source": atom["probe"], "time_us": round(adds / atom["gops"] / 1e3, 3),
                                          "frac": round(adds / atom["gops"] / 1e3 / dom_us, 4)}
        if atom32 is not None:  # why the accumulator is f64: the same adds at the f32 instruction's rate
            line["roofline"]["lds_atomic"]["f32_gops"] = atom32["gops"]
            line["roofline"]["lds_atomic"]["f32_source"] = atom32["probe"]
            line["roofline"]["lds_atomic"]["f32_time_us"] = round(adds / atom32["gops"] / 1e3, 3)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
