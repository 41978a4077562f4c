"""msda_bwd_noalloc (no workspace argument, no device allocation: the partial sums live in the
library's file-scope device array) against msda_bwd with a caller-allocated workspace, through the
C ABI: two calls in a row, the second with a smaller input, so that the second reuses the array
the first left filled. grad_sampling_locations and grad_attention_weights must be bit-identical
(their sums have a fixed order); grad_value within the f32 parity tolerance of the module (its
f64 LDS accumulation order may differ between runs)."""

from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest
import torch

from rfdetr_jax_amd import _native
from rfdetr_jax_amd import ops as hip
from rfdetr_jax_amd.workloads import make_inputs
from tests._util import assert_close

pytestmark = pytest.mark.gpu


def _note(msg):
    sys.stderr.write(f"[gpu] {msg}\n")
    sys.stderr.flush()


def _noalloc_backward(v, shapes, loc, attn, grad):
    lib = _native.lib()
    batch, len_query, n_heads, n_levels, n_points = loc.shape[:5]
    head_dim = v.shape[2]
    arr, starts = hip._shape_arrays(hip._as_shapes(shapes))
    dims = (batch, n_heads, head_dim, len_query, n_levels, n_points, arr, starts, v.shape[1])
    gv = torch.empty_like(v)
    gl = torch.empty(loc.shape, dtype=torch.float32, device=v.device)
    ga = torch.empty(attn.shape, dtype=torch.float32, device=v.device)
    ws = lib.msda_bwd_workspace_size(*dims)
    assert ws > 0, "the case must need partial sums, or the array is not exercised"
    with torch.cuda.device(v.device):
        rc = lib.msda_bwd_noalloc(
            hip._ptr(v), hip._VALUE_DTYPES[v.dtype], hip._ptr(loc), hip._ptr(attn), hip._ptr(grad),
            hip._VALUE_DTYPES[grad.dtype], hip._ptr(gv), hip._ptr(gl), hip._ptr(ga), *dims, hip._stream(v.device),
        )
    _native.check(rc)
    return gv, gl, ga


def _case(seed, batch, heads, queries, shapes, points):
    d = torch.device("cuda:0")
    value, loc, attn, grad = make_inputs(seed, batch, heads, 16, queries, shapes, points)
    return [torch.from_numpy(np.ascontiguousarray(x)).to(d) for x in (value, loc, attn, grad)]


def test_noalloc_first_call_captured_in_a_graph():
    """The process's first msda_bwd_noalloc call (this test runs first in this file) is made under
    graph capture: the scratch array's address was looked up when the library first used the
    device (the reference call below), so the captured call only launches. Every replay, with
    eager work and a synchronisation between replays, matches msda_bwd."""
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    shapes = ((24, 24),)
    v, lc, a, g = _case(21, 2, 8, 3900, shapes, 2)
    want = hip.ms_deform_attn_backward(v, shapes, lc, a, g)
    torch.cuda.synchronize()
    lib = _native.lib()
    arr, starts = hip._shape_arrays(hip._as_shapes(shapes))
    dims = (2, 8, 16, 3900, 1, 2, arr, starts, 576)
    assert lib.msda_bwd_workspace_size(*dims) > 0, "the case must need partial sums"
    gv, gl, ga = torch.empty_like(v), torch.empty_like(lc), torch.empty_like(a)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = lib.msda_bwd_noalloc(
                hip._ptr(v), hip._VALUE_DTYPES[v.dtype], hip._ptr(lc), hip._ptr(a), hip._ptr(g),
                hip._VALUE_DTYPES[g.dtype], hip._ptr(gv), hip._ptr(gl), hip._ptr(ga), *dims, hip._stream(v.device),
            )
    _native.check(rc)
    other = torch.zeros(1 << 20, device=v.device)
    for rep in range(3):
        gv.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        _note(f"noalloc graph replay {rep}")
        assert torch.equal(gl, want[1]), "grad_sampling_locations differs"
        assert torch.equal(ga, want[2]), "grad_attention_weights differs"
        assert_close(gv.cpu().numpy(), want[0].cpu().numpy(), 1e-5, "grad_value")
        other.add_(1.0)
        torch.cuda.synchronize()


def test_noalloc_matches_workspace_entry_point_twice():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    cases = [(11, 2, 8, 3900, ((24, 24),), 2), (12, 1, 4, 1500, ((24, 24), (12, 12)), 2)]
    for seed, batch, heads, queries, shapes, points in cases:
        _note(f"noalloc seed={seed} batch={batch} heads={heads} queries={queries} shapes={shapes}")
        v, lc, a, g = _case(seed, batch, heads, queries, shapes, points)
        want = hip.ms_deform_attn_backward(v, shapes, lc, a, g)
        got = _noalloc_backward(v, shapes, lc, a, g)
        torch.cuda.synchronize()
        assert torch.equal(got[1], want[1]), "grad_sampling_locations differs"
        assert torch.equal(got[2], want[2]), "grad_attention_weights differs"
        assert_close(got[0].cpu().numpy(), want[0].cpu().numpy(), 1e-5, "grad_value")


def test_noalloc_rejects_shapes_beyond_its_array(tune):
    """A plan whose partial sums exceed the 16 MiB array (the sorted gather with 64-query blocks)
    is refused before anything runs."""
    tune({"MSDA_BWD_GATHER": "1", "MSDA_BWD_GATHER_QB": "64"})
    lib = _native.lib()
    shapes = ((24, 24),)
    arr, starts = hip._shape_arrays(hip._as_shapes(shapes))
    dims = (4, 4, 16, 20000, 1, 2, arr, starts, 576)
    ws = lib.msda_bwd_workspace_size(*dims)
    assert ws > 16 << 20, ws
    null = ctypes.c_void_p(0)
    rc = lib.msda_bwd_noalloc(null, 0, null, null, null, 0, null, null, null, *dims, null)
    assert rc == _native.ERR_UNSUPPORTED
    assert b"scratch" in lib.msda_last_error()


@pytest.mark.parametrize("seed", range(8))
def test_noalloc_random_shapes_with_query_blocks(seed):
    """Random shapes whose levels fit the LDS whole and whose queries are split into blocks (so the
    partial sums go to the library's array): 1-2 levels of 4-24 rows and columns, 1-8 heads,
    head_dim 8-32, 1-4 points, 600-4000 queries, f32 or bf16, against msda_bwd with a workspace."""
    rng = np.random.default_rng(1200 + seed)
    levels = int(rng.integers(1, 3))
    shapes = tuple((int(rng.integers(4, 25)), int(rng.integers(4, 25))) for _ in range(levels))
    heads, dim = int(rng.choice([1, 2, 4, 8])), int(rng.choice([8, 16, 32]))
    points, queries = int(rng.integers(1, 5)), int(rng.integers(600, 4001))
    bf16 = bool(rng.integers(0, 2))
    _note(f"noalloc random seed={seed} shapes={shapes} heads={heads} dim={dim} points={points} queries={queries} bf16={bf16}")
    d = torch.device("cuda:0")
    value, loc, attn, grad = make_inputs(1300 + seed, 1, heads, dim, queries, shapes, points,
                                         value_dtype="bf16" if bf16 else "f32")
    v, lc, a, g = (torch.from_numpy(np.ascontiguousarray(x)).to(d) for x in (value, loc, attn, grad))
    if bf16:
        v = v.to(torch.bfloat16)
    want = hip.ms_deform_attn_backward(v, shapes, lc, a, g)
    got = _noalloc_backward(v, shapes, lc, a, g)
    torch.cuda.synchronize()
    assert torch.equal(got[1], want[1]), "grad_sampling_locations differs"
    assert torch.equal(got[2], want[2]), "grad_attention_weights differs"
    assert_close(got[0].float().cpu().numpy(), want[0].float().cpu().numpy(), 2e-2 if bf16 else 1e-5, "grad_value")
