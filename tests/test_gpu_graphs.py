"""Every entry-point family captured in a HIP graph on a side stream, on an MI355X.

Capture fails if a call launches onto another stream or synchronises the host, so a clean capture
shows that each call only enqueues on the stream it was given. Each graph is replayed three
times, with other eager work of the library and its synchronisation between replays, and every
replay is compared with the eager results: bit for bit where the kernels sum in a fixed order,
within one f32 ulp-scale bound for grad_value (its f64 LDS sums follow the atomics' order).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from rfdetr_jax_amd import ops as hip
from rfdetr_jax_amd.attention import grouped_attention
from rfdetr_jax_amd.grid_sample import bilinear_grid_sample
from rfdetr_jax_amd.value_proj import value_proj_backward, value_proj_forward
from rfdetr_jax_amd.workloads import make_fused_inputs, make_inputs

pytestmark = pytest.mark.gpu


def _note(msg):
    sys.stderr.write(f"[gpu] {msg}\n")
    sys.stderr.flush()


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")
    return t if dtype is None else t.to(dtype)


def _replays(fn, eager, other, exact):
    """Captures fn (returning a tuple of tensors) on a side stream, replays it three times with
    `other` run eagerly and synchronised between replays, and checks each replay against `eager`:
    torch.equal for the indices in `exact`, a 1e-6 relative bound otherwise."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up on the side stream (first-use caches, the allocator)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        outs = fn()
    for rep in range(3):
        other()
        torch.cuda.synchronize()
        for o in outs:
            if o is not None:
                o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        _note(f"replay {rep}")
        for i, (got, want) in enumerate(zip(outs, eager)):
            if want is None:
                continue
            if i in exact:
                assert torch.equal(got, want), f"output {i}, replay {rep}"
            else:
                scale = max(1.0, float(want.abs().max()))
                assert float((got.float() - want.float()).abs().max()) <= 1e-6 * scale, f"output {i}, replay {rep}"


def test_core_op_in_a_graph():
    shapes = ((24, 24), (12, 12))
    value, loc, attn, grad = make_inputs(3, 2, 8, 16, 900, shapes, 2)
    v, lc, a, g = (_t(x) for x in (value, loc, attn, grad))
    v2 = v.flip(1).contiguous()

    def fn():
        out = hip.ms_deform_attn_forward(v, shapes, lc, a)
        return (out, *hip.ms_deform_attn_backward(v, shapes, lc, a, g))

    eager = fn()
    torch.cuda.synchronize()
    _replays(fn, eager, lambda: hip.ms_deform_attn_backward(v2, shapes, lc, a, g), exact={0, 2, 3})


def test_sampler_and_fused_ops_in_a_graph():
    shapes = ((20, 20), (10, 10))
    value, ref, off, logits, grad = make_fused_inputs(4, 2, 4, 16, 300, shapes, 4, 4)
    v, r, o, lg, g = (_t(x) for x in (value, ref, off, logits, grad))
    value2, loc2, attn2, _ = make_inputs(5, 2, 4, 16, 300, shapes, 4, value_dtype="bf16")
    vb, lc2, a2 = _t(value2, torch.bfloat16), _t(loc2), _t(attn2)

    def fn():
        out = hip.ms_deform_attn_fused_forward(v, shapes, r, o, lg)
        grads = hip.ms_deform_attn_fused_backward(v, shapes, r, o, lg, g)
        outs = hip.ms_deform_attn_forward(vb, shapes, lc2, a2, sampler="gather")
        return (out, *grads, outs)

    eager = fn()
    torch.cuda.synchronize()
    _replays(fn, eager, lambda: hip.ms_deform_attn_forward(v, shapes, lc2, a2), exact={0, 2, 3, 4, 5})


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_attention_and_dropout_in_a_graph(bf16):
    rng = np.random.default_rng(6)
    b, gr, p, h, d = 2, 3, 120, 4, 32
    dt = torch.bfloat16 if bf16 else torch.float32
    q, k, v, go = (_t(rng.standard_normal((b, gr * p, h * d)).astype(np.float32), dt) for _ in range(4))
    from rfdetr_jax_amd.attention import _Layout, attention_backward, attention_forward

    lay = _Layout(b, gr, h, p, d)

    def fn():
        o, st = attention_forward(q, k, v, lay, lay.strides_rows)
        grads = attention_backward(q, k, v, o, st, go, lay, lay.strides_rows)
        od, std = attention_forward(q, k, v, lay, lay.strides_rows, drop=(0.1, 99))
        gd = attention_backward(q, k, v, od, std, go, lay, lay.strides_rows, drop=(0.1, 99))
        return (o, *grads, od, *gd)

    eager = fn()
    torch.cuda.synchronize()
    _replays(fn, eager, lambda: grouped_attention(k, q, v, h, gr), exact=set(range(8)))


def test_value_projection_and_grid_sample_in_a_graph():
    rng = np.random.default_rng(7)
    x = _t(rng.standard_normal((2, 300, 64)).astype(np.float32))
    w = _t((rng.standard_normal((64, 64)) / 8).astype(np.float32))
    bias = _t(rng.standard_normal(64).astype(np.float32))
    mask = _t(rng.uniform(0, 1, (2, 300)) < 0.2)
    gv = _t(rng.standard_normal((16, 300, 4)).astype(np.float32))
    maps = _t(rng.standard_normal((3, 2, 40, 56)).astype(np.float32))
    grid = _t(rng.uniform(-1.2, 1.2, (3, 120, 2)).astype(np.float32))
    gout = _t(rng.standard_normal((3, 2, 120)).astype(np.float32))
    from rfdetr_jax_amd import _native
    from rfdetr_jax_amd.grid_sample import grid_sample_backward, grid_sample_forward

    modes = (_native.GRID_COORDS, _native.PADDING["border"], _native.SAMPLE_BILINEAR)

    def fn():
        y = value_proj_forward(x, w, bias, 16, mask)
        gx, gw, gb = value_proj_backward(x, w, 16, gv, mask)
        s = grid_sample_forward(maps, grid, *modes)
        gi, gg = grid_sample_backward(maps, grid, gout, *modes)
        return (y, gx, gw, gb, s, gi, gg)

    eager = fn()
    torch.cuda.synchronize()
    other = lambda: bilinear_grid_sample(maps, grid.flip(-1).reshape(3, 120, 1, 2).contiguous(), "zeros")  # noqa: E731
    _replays(fn, eager, other, exact={0, 1, 2, 3, 4, 6})
