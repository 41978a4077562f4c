"""Parity of the HIP kernels (called through the C ABI) with the CPU oracles, on an MI355X.

Tolerances (the benchmark definition's bar, in the reference's criterion form
``max|got - want| <= tol * max(1, max|want|)``, tests/test_ops.py:245-248):
* f32 value: forward 1e-5; gradients 1e-4 (grad_value is summed with LDS atomics, whose order
  is not fixed);
* bf16 value: 2e-2 for everything (the reference compares bf16 runs against f32 math on the
  bf16-rounded values, tests/test_ops.py:238, with tolerance 1e-2 on gradients).
The expected values are the float64 NumPy oracle at fixture / reduced sizes and the f32 C oracle
at the full benchmark sizes, plus size-independent identities (linearity in value and weights).
"""

from __future__ import annotations

import math
import os
import sys

import numpy as np
import pytest
import torch

from oracle import cref
from oracle import msda_ref as R
from rfdetr_jax_amd import ops as hip
from rfdetr_jax_amd.workloads import CONFIGS, make_inputs, workload_inputs
from tests._util import assert_close, golden_names, load_golden

pytestmark = pytest.mark.gpu


def _dev():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch.device("cuda:0")


def _note(msg):
    sys.stderr.write(f"[gpu] {msg}\n")
    sys.stderr.flush()


def _to_dev(value, loc, attn, grad=None, bf16=False):
    d = _dev()
    v = torch.from_numpy(np.ascontiguousarray(value)).to(d)
    if bf16:
        v = v.to(torch.bfloat16)
    out = [v, torch.from_numpy(np.ascontiguousarray(loc)).to(d), torch.from_numpy(np.ascontiguousarray(attn)).to(d)]
    out.append(None if grad is None else torch.from_numpy(np.ascontiguousarray(grad)).to(d))
    return out


def _np(t):
    return t.detach().float().cpu().numpy()


def _run(value, shapes, loc, attn, grad, bf16=False):
    v, lc, a, g = _to_dev(value, loc, attn, grad, bf16)
    out = hip.ms_deform_attn_forward(v, shapes, lc, a)
    grads = hip.ms_deform_attn_backward(v, shapes, lc, a, g) if g is not None else (None, None, None)
    torch.cuda.synchronize()
    return _np(out), [None if x is None else _np(x) for x in grads]


# --------------------------------------------------------------------------------------------
# golden fixtures (float64 oracle, cross-checked with torch grid_sample when generated)


@pytest.mark.parametrize("name", golden_names())
def test_golden_fixture(name):
    g = load_golden(name)
    bf16 = g["meta"].get("value_dtype") == "bf16"
    _note(f"golden {name} shapes={g['shapes']} value={g['value'].shape} bf16={bf16}")
    out, (gv, gl, ga) = _run(g["value"], g["shapes"], g["loc"], g["attn"], g["grad"], bf16)
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(out, g["out"], tf, f"{name} out")
    assert_close(gv, g["grad_value"], tg, f"{name} grad_value")
    assert_close(gl, g["grad_loc"], tg, f"{name} grad_loc")
    assert_close(ga, g["grad_attn"], tg, f"{name} grad_attn")
    if "expect" in g["meta"]:
        assert np.allclose(out.reshape(-1), g["meta"]["expect"], atol=1e-6)


# --------------------------------------------------------------------------------------------
# the five benchmark configurations


@pytest.mark.parametrize("cfg", sorted(CONFIGS))
def test_config_reduced_against_float64_oracle(cfg):
    """Each configuration's shape at batch 1 (queries capped at 600) against the float64 oracle."""
    w = CONFIGS[cfg].scaled(batch=1, queries=min(CONFIGS[cfg].queries, 600))
    bf16 = w.value_dtype == "bf16"
    _note(f"config {cfg} reduced B=1 Q={w.queries} shapes={w.shapes}")
    value, loc, attn, grad = make_inputs(100 + cfg, w.batch, w.heads, w.head_dim, w.queries, w.shapes, w.points,
                                         w.value_dtype, w.uniform_locations, True)
    out, (gv, gl, ga) = _run(value, w.shapes, loc, attn, grad, bf16)
    assert_close(out, R.ms_deform_attn_core_rows(value, w.shapes, loc, attn), 2e-2 if bf16 else 1e-5, "out")
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, w.shapes, loc, attn, grad)
    tg = 2e-2 if bf16 else 1e-4
    assert_close(gv, rv, tg, "grad_value")
    assert_close(gl, rl, tg, "grad_loc")
    assert_close(ga, ra, tg, "grad_attn")


@pytest.mark.parametrize("cfg", sorted(CONFIGS))
def test_config_full_size(cfg):
    """Full benchmark size against the f32 C oracle, plus <G,out> = <dV,V> = <dA,A>."""
    w = CONFIGS[cfg]
    bf16 = w.value_dtype == "bf16"
    _note(f"config {cfg} full size {w.name}")
    value, loc, attn, grad = workload_inputs(w, with_grad=True)
    out, (gv, gl, ga) = _run(value, w.shapes, loc, attn, grad, bf16)
    assert_close(out, cref.forward(value, w.shapes, loc, attn), 2e-2 if bf16 else 1e-5, "out")
    cv, cl, ca = cref.backward(value, w.shapes, loc, attn, grad)
    tg = 2e-2 if bf16 else 1e-4
    assert_close(gv, cv, tg, "grad_value")
    assert_close(gl, cl, tg, "grad_loc")
    assert_close(ga, ca, tg, "grad_attn")
    inner = float(np.sum(out.astype(np.float64) * grad))
    assert math.isclose(float(np.sum(gv.astype(np.float64) * value)), inner, rel_tol=1e-2 if bf16 else 1e-4)
    assert math.isclose(float(np.sum(ga.astype(np.float64) * attn)), inner, rel_tol=1e-4)


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_multi_scale_training_shape(bf16):
    """A four-level, 32-channel, 4-point shape of the larger RF-DETR variants (levels 80x80 down
    to 10x10, so the large levels are gathered through L2 and every query has 16 samples) against
    the C oracle, plus <G,out> = <dV,V> = <dA,A>."""
    shapes = ((80, 80), (40, 40), (20, 20), (10, 10))
    value, loc, attn, grad = make_inputs(123, 2, 8, 32, 300, shapes, 4)
    if bf16:
        value = R.bf16_round(value)
    _note(f"multi-scale training shape bf16={bf16}")
    out, (gv, gl, ga) = _run(value, shapes, loc, attn, grad, bf16)
    tol = 2e-2 if bf16 else 1e-5
    assert_close(out, cref.forward(value, shapes, loc, attn), tol, "out")
    cv, cl, ca = cref.backward(value, shapes, loc, attn, grad)
    tg = 2e-2 if bf16 else 1e-4
    assert_close(gv, cv, tg, "grad_value")
    assert_close(gl, cl, tg, "grad_loc")
    assert_close(ga, ca, tg, "grad_attn")
    inner = float(np.sum(out.astype(np.float64) * grad))
    assert math.isclose(float(np.sum(gv.astype(np.float64) * value)), inner, rel_tol=1e-2 if bf16 else 1e-4)
    assert math.isclose(float(np.sum(ga.astype(np.float64) * attn)), inner, rel_tol=1e-4)


# --------------------------------------------------------------------------------------------
# the differentiable entry points (autograd.Function over the C ABI)


def test_autograd_matches_oracle_vjp():
    g = load_golden("two_level_f32")
    v, lc, a, gr = _to_dev(g["value"], g["loc"], g["attn"], g["grad"])
    v.requires_grad_(True)
    lc.requires_grad_(True)
    a.requires_grad_(True)
    out = hip.ms_deform_attn_core_rows(v, g["shapes"], lc, a, "gather")
    assert out.dtype == torch.float32 and tuple(out.shape) == (2, 70, 16)
    (out * gr).sum().backward()
    assert_close(_np(v.grad), g["grad_value"], 1e-4, "grad_value")
    assert_close(_np(lc.grad), g["grad_loc"], 1e-4, "grad_loc")
    assert_close(_np(a.grad), g["grad_attn"], 1e-4, "grad_attn")


def test_ms_deform_attn_signature_and_core_layout():
    g = load_golden("two_level_f32")
    v, lc, a, _ = _to_dev(g["value"], g["loc"], g["attn"])
    starts = torch.tensor([0, 128], device=v.device)
    out = hip.ms_deform_attn(v, torch.tensor(g["shapes"]), starts, lc, a)
    assert_close(_np(out), g["out"], 1e-5, "ms_deform_attn")
    # ms_deform_attn_core takes [B, H, D, S] (a non-contiguous transpose of the rows layout)
    v_bhds = v.reshape(2, 2, 160, 8).permute(0, 1, 3, 2)
    out2 = hip.ms_deform_attn_core(v_bhds, g["shapes"], lc, a)
    assert_close(_np(out2), g["out"], 1e-5, "ms_deform_attn_core")


def test_only_requested_gradients_are_computed():
    g = load_golden("two_level_f32")
    v, lc, a, gr = _to_dev(g["value"], g["loc"], g["attn"], g["grad"])
    a.requires_grad_(True)
    out = hip.ms_deform_attn_core_rows(v, g["shapes"], lc, a)
    (out * gr).sum().backward()
    assert v.grad is None and lc.grad is None
    assert_close(_np(a.grad), g["grad_attn"], 1e-4, "grad_attn alone")


def test_bf16_weights_give_bf16_output():
    """result_type(bf16 value, bf16 weights) = bf16 (ops.py:260)."""
    g = load_golden("two_level_bf16")
    v, lc, a, _ = _to_dev(g["value"], g["loc"], g["attn"], bf16=True)
    out = hip.ms_deform_attn_core_rows(v, g["shapes"], lc, a.to(torch.bfloat16))
    assert out.dtype == torch.bfloat16
    want = R.ms_deform_attn_core_rows(g["value"], g["shapes"], g["loc"], R.bf16_round(g["attn"]))
    assert_close(_np(out), want, 2e-2, "bf16 out")


# --------------------------------------------------------------------------------------------
# alternative kernel paths and edge cases


def test_global_gather_path_and_many_bands(tune):
    """Forward without LDS staging (levels read through L2) and backward split into many bands."""
    g = load_golden("nano_small")
    tune({"MSDA_FWD_LDS_BUDGET": "0"})
    tune({"MSDA_BWD_GATHER": "0", "MSDA_BWD_FORCE_BANDS": "1", "MSDA_BWD_BANDS": "7"})
    out, (gv, gl, ga) = _run(g["value"], g["shapes"], g["loc"], g["attn"], g["grad"])
    assert_close(out, g["out"], 1e-5, "out")
    assert_close(gv, g["grad_value"], 1e-4, "grad_value")
    assert_close(gl, g["grad_loc"], 1e-4, "grad_loc")
    assert_close(ga, g["grad_attn"], 1e-4, "grad_attn")


_BAND = {"MSDA_BWD_GATHER": "0"}  # the atomic-accumulation band kernel (the default)
_GATHER = {"MSDA_BWD_GATHER": "1"}  # the sorted-gather kernel


@pytest.mark.parametrize("variant", [
    {**_GATHER},                                                # sorted gather, default blocks
    {**_GATHER, "MSDA_BWD_GATHER_QB": "64"},                    # many query blocks: partial sums
    {**_GATHER, "MSDA_BWD_GATHER_QB": "333"},                   # ragged last block
    {**_GATHER, "MSDA_BWD_GATHER_THREADS": "1024"},             # short runs: cells span many threads
    {**_GATHER, "MSDA_BWD_GATHER_STAGE": "0"},                  # value rows from global memory
    {**_GATHER, "MSDA_BWD_GATHER_STAGE": "1"},                  # value rows staged in LDS
    {**_GATHER, "MSDA_BWD_GATHER_WGS_PER_CU": "2"},
    {**_BAND},                                                  # band kernel: whole levels, query blocks
    {**_BAND, "MSDA_BWD_THREADS": "64"},                        # one-wave workgroups
    {**_BAND, "MSDA_BWD_FORCE_BANDS": "1"},                     # row bands, scanned and listed
    {**_BAND, "MSDA_BWD_FORCE_BANDS": "1", "MSDA_BWD_BANDS": "24"},  # one row per band: points straddle
    {**_BAND, "MSDA_BWD_FORCE_BANDS": "1", "MSDA_BWD_LIST": "64"},   # several list passes per band
    {**_BAND, "MSDA_BWD_FORCE_BANDS": "1", "MSDA_BWD_THREADS": "64"},
    {**_BAND, "MSDA_BWD_MAX_VEC": "16"},                        # one lane per query
    {**_BAND, "MSDA_BWD_MAX_VEC": "4"},                         # four lanes per query
    {**_BAND, "MSDA_BWD_MAX_VEC": "1"},                         # one channel per lane
], ids=lambda v: ",".join(f"{k}={x}" for k, x in v.items()) or "default")
@pytest.mark.parametrize("queries", [700, 5000])
def test_backward_launch_variants(tune, variant, queries):
    """The backward kernels' launch shapes against the float64 oracle. Sorted gather: query blocks
    from 64 queries to the LDS limit (partial sums added by a second kernel), 8 to 16 waves, value
    rows from global memory or LDS. Band kernel: whole levels with the queries split in blocks, row
    bands from one per level to one per image row with one or several list passes, workgroups of
    one to sixteen waves, and one to sixteen lanes per query."""
    tune(variant)
    shapes = ((24, 24), (12, 12))
    value, loc, attn, grad = make_inputs(77, 2, 4, 16, queries, shapes, 2)
    _note(f"variant={variant} queries={queries}")
    out, (gv, gl, ga) = _run(value, shapes, loc, attn, grad)
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    assert_close(gv, rv, 1e-4, "grad_value")
    assert_close(gl, rl, 1e-4, "grad_loc")
    assert_close(ga, ra, 1e-4, "grad_attn")


@pytest.mark.parametrize("pair", [0, 1])
def test_forward_paired_lanes(tune, pair):
    """One level, two points, 16 channels (two lanes of 8 per query-head): the forward with the
    two lanes splitting the samples' coordinate work (pair=1, the default) and without (pair=0)."""
    tune({"MSDA_FWD_PAIR": str(pair)})
    shapes = ((24, 24),)
    value, loc, attn, grad = make_inputs(91, 2, 8, 16, 1000, shapes, 2)
    _note(f"pair={pair}")
    out, _ = _run(value, shapes, loc, attn, grad)
    assert_close(out, R.ms_deform_attn_core_rows(value, shapes, loc, attn), 1e-5, "out")


@pytest.mark.parametrize("variant", [
    {"MSDA_FWD_GROUPED": "0"},
    {"MSDA_FWD_MAX_VEC": "16"},
    {**_BAND, "MSDA_BWD_MAX_VEC": "16"},
    {"MSDA_FWD_HEADS": "2"},
    {"MSDA_FWD_HEADS": "4"},
], ids=lambda v: ",".join(f"{k}={x}" for k, x in v.items()))
@pytest.mark.parametrize("shapes", [((24, 24),), ((24, 24), (12, 12))], ids=["one_level", "two_levels"])
def test_kernel_variants(tune, variant, shapes):
    """Other launch variants (one query at a time and 16-channel lanes in the forward, one lane per
    query in the backward, two- and four-head forward workgroups, which 700 queries do not get by
    default) against the float64 oracle."""
    for k, v in variant.items():
        tune({k: v})
    value, loc, attn, grad = make_inputs(5, 2, 8, 16, 700, shapes, 2)
    _note(f"variant={variant} shapes={shapes}")
    out, (gv, gl, ga) = _run(value, shapes, loc, attn, grad)
    assert_close(out, R.ms_deform_attn_core_rows(value, shapes, loc, attn), 1e-5, "out")
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    assert_close(gv, rv, 1e-4, "grad_value")
    assert_close(gl, rl, 1e-4, "grad_loc")
    assert_close(ga, ra, 1e-4, "grad_attn")


def test_level_larger_than_lds():
    """A 200x120 f32 level (1.5 MB per slice) plus a small one: global-gather forward, banded backward."""
    shapes = ((200, 120), (10, 12))
    value, loc, attn, grad = make_inputs(21, 1, 2, 16, 150, shapes, 3)
    out, (gv, gl, ga) = _run(value, shapes, loc, attn, grad)
    assert_close(out, R.ms_deform_attn_core_rows(value, shapes, loc, attn), 1e-5, "out")
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    assert_close(gv, rv, 1e-4, "grad_value")
    assert_close(gl, rl, 1e-4, "grad_loc")
    assert_close(ga, ra, 1e-4, "grad_attn")


def test_misaligned_value_uses_narrow_loads():
    """A value tensor offset by one element is not 16-byte aligned: the library narrows its loads."""
    g = load_golden("two_level_f32")
    d = _dev()
    base = torch.zeros(g["value"].size + 1, device=d)
    v = base[1:].view(g["value"].shape)
    v.copy_(torch.from_numpy(g["value"]).to(d))
    _, lc, a, gr = _to_dev(g["value"], g["loc"], g["attn"], g["grad"])
    out = hip.ms_deform_attn_forward(v, g["shapes"], lc, a)
    gv, gl, ga = hip.ms_deform_attn_backward(v, g["shapes"], lc, a, gr)
    assert_close(_np(out), g["out"], 1e-5, "out")
    assert_close(_np(gv), g["grad_value"], 1e-4, "grad_value")


def test_empty_queries_and_batch():
    d = _dev()
    shapes = ((4, 4),)
    v = torch.randn(2, 16, 16, device=d)
    lc = torch.zeros(1, 0, 2, 1, 2, 2, device=d)
    a = torch.zeros(1, 0, 2, 2, device=d)
    out = hip.ms_deform_attn_forward(v, shapes, lc, a)
    assert tuple(out.shape) == (1, 0, 32)
    gv, gl, ga = hip.ms_deform_attn_backward(v, shapes, lc, a, torch.zeros(1, 0, 32, device=d))
    torch.cuda.synchronize()
    assert torch.count_nonzero(gv).item() == 0 and gl.numel() == 0 and ga.numel() == 0
    v0 = torch.zeros(0, 16, 16, device=d)
    out0 = hip.ms_deform_attn_forward(v0, shapes, torch.zeros(0, 3, 2, 1, 2, 2, device=d), torch.zeros(0, 3, 2, 2, device=d))
    assert tuple(out0.shape) == (0, 3, 32)


def test_location_and_weight_gradients_are_deterministic():
    """grad_sampling_locations and grad_attention_weights are sums in a fixed order: bit-identical
    between runs. grad_value is summed in f64 in LDS (atomic order) and rounded once to f32, so two
    runs differ only where the f64 sums straddle an f32 rounding boundary: at most one f32 ulp, in
    a vanishing share of the elements."""
    w = CONFIGS[2].scaled(batch=2)
    value, loc, attn, grad = workload_inputs(w, with_grad=True)
    v, lc, a, g = _to_dev(value, loc, attn, grad)
    first = hip.ms_deform_attn_backward(v, w.shapes, lc, a, g)
    second = hip.ms_deform_attn_backward(v, w.shapes, lc, a, g)
    assert torch.equal(first[1], second[1]) and torch.equal(first[2], second[2])
    diff = (first[0] - second[0]).abs()
    assert bool((diff <= torch.finfo(torch.float32).eps * first[0].abs()).all()), "grad_value differs by more than one ulp"
    changed = int(torch.count_nonzero(diff).item())
    _note(f"grad_value elements that differ between two runs: {changed} of {diff.numel()}")
    assert changed <= diff.numel() // 10000


@pytest.mark.parametrize(
    "dtype,heads,dim,shape",
    [("bf16", 16, 16, (32, 40)), ("f32", 8, 32, (16, 20)), ("f32", 16, 16, (32, 40))],
    ids=["bf16_h16_d16_32x40", "f32_h8_d32_16x20", "f32_h16_d16_32x40"],
)
def test_backward_where_the_forward_head_group_fills_the_lds(tune, dtype, heads, dim, shape):
    """Shapes whose forward stages a group of heads into the whole 160 KB LDS (bf16: 4 heads x 32 x
    40 x 16 x 2 B = 163,840 B; the forward groups four heads by default from 1024 queries, forced
    here at 400): the backward plans its own LDS use and must run them too."""
    tune({"MSDA_FWD_HEADS": 4})
    bf16 = dtype == "bf16"
    shapes = (shape,)
    value, loc, attn, grad = make_inputs(91, 2, heads, dim, 400, shapes, 2)
    if bf16:
        value = R.bf16_round(value)
    _note(f"lds-filling shape {dtype} heads={heads} dim={dim} level={shape}")
    out, (gv, gl, ga) = _run(value, shapes, loc, attn, grad, bf16)
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(out, R.ms_deform_attn_core_rows(value, shapes, loc, attn), tf, "out")
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    assert_close(gv, rv, tg, "grad_value")
    assert_close(gl, rl, tg, "grad_loc")
    assert_close(ga, ra, tg, "grad_attn")


def _bwd_through_abi(v, shapes, lc, a, g, ws_bytes):
    """msda_bwd with a workspace of exactly ws_bytes (NULL when 0); returns the status."""
    from rfdetr_jax_amd import _native

    lib = _native.lib()
    batch, len_query, n_heads, n_levels, n_points = lc.shape[:5]
    arr, starts = hip._shape_arrays(hip._as_shapes(shapes))
    dims = (batch, n_heads, v.shape[2], len_query, n_levels, n_points, arr, starts, v.shape[1])
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=v.device)
    gv, gl, ga = torch.empty_like(v), torch.empty_like(lc), torch.empty_like(a)
    rc = lib.msda_bwd(
        hip._ptr(v), hip._VALUE_DTYPES[v.dtype], hip._ptr(lc), hip._ptr(a), hip._ptr(g), hip._VALUE_DTYPES[g.dtype],
        hip._ptr(gv), hip._ptr(gl), hip._ptr(ga), *dims, hip._ptr(ws) if ws_bytes > 0 else None, ws_bytes,
        hip._stream(v.device),
    )
    torch.cuda.synchronize()
    return rc, lib.msda_bwd_workspace_size(*dims), (gv, gl, ga)


@pytest.mark.parametrize(
    "name,batch,heads,dim,queries,shapes,points",
    [
        ("config2", 8, 16, 16, 3900, ((24, 24),), 2),
        ("four_levels_p4", 8, 8, 32, 3900, ((80, 80), (40, 40), (20, 20), (10, 10)), 4),
    ],
)
def test_workspace_size_is_the_contract(name, batch, heads, dim, queries, shapes, points):
    """The size msda_bwd_workspace_size returns is accepted by msda_bwd, one byte less is refused,
    and the size is a few f32 copies of grad_value (the query blocks' partial sums), independent
    of how the samples fall. The figures are printed for the record."""
    from rfdetr_jax_amd import _native

    value, loc, attn, grad = make_inputs(5, batch, heads, dim, queries, shapes, points)
    v, lc, a, g = _to_dev(value, loc, attn, grad)
    rc, ws, _ = _bwd_through_abi(v, shapes, lc, a, g, 0)
    dv_f32 = v.numel() * 4
    _note(f"{name}: workspace {ws} bytes = {ws / dv_f32:.2f} x the f32 grad_value ({dv_f32} bytes)")
    assert ws >= 0 and ws % 16 == 0 and ws <= 8 * dv_f32
    if ws > 0:
        assert rc == _native.ERR_INVALID_ARGUMENT
        rc_short, _, _ = _bwd_through_abi(v, shapes, lc, a, g, ws - 1)
        assert rc_short == _native.ERR_INVALID_ARGUMENT
    rc, _, (gv, gl, ga) = _bwd_through_abi(v, shapes, lc, a, g, ws)
    assert rc == 0
    want = hip.ms_deform_attn_backward(v, shapes, lc, a, g)
    assert torch.equal(gl, want[1]) and torch.equal(ga, want[2])
    assert_close(_np(gv), _np(want[0]), 1e-5, "grad_value")


def test_nan_location_propagates_like_the_reference():
    """A NaN position gives a NaN interpolation weight, so that query's output is NaN (ops.py:123-128)."""
    g = load_golden("nano_small")
    loc = g["loc"].copy()
    loc[0, 5, 1, 0, 0, 0] = np.nan
    out, _ = _run(g["value"], g["shapes"], loc, g["attn"], None)
    assert np.isnan(out[0, 5, 16:32]).all()
    finite = np.ones(out.shape, bool)
    finite[0, 5, 16:32] = False
    assert np.isfinite(out[finite]).all()


def test_non_default_stream():
    g = load_golden("nano_small")
    v, lc, a, gr = _to_dev(g["value"], g["loc"], g["attn"], g["grad"])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = hip.ms_deform_attn_forward(v, g["shapes"], lc, a)
        gv, _, _ = hip.ms_deform_attn_backward(v, g["shapes"], lc, a, gr)
    s.synchronize()
    assert_close(_np(out), g["out"], 1e-5, "out on side stream")
    assert_close(_np(gv), g["grad_value"], 1e-4, "grad_value on side stream")


@pytest.mark.parametrize("d", [2, 4, 8, 64])
def test_other_head_dims(d):
    shapes = ((9, 7), (5, 3))
    value, loc, attn, grad = make_inputs(40 + d, 2, 3, d, 33, shapes, 3)
    out, (gv, gl, ga) = _run(value, shapes, loc, attn, grad)
    assert_close(out, R.ms_deform_attn_core_rows(value, shapes, loc, attn), 1e-5, "out")
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    assert_close(gv, rv, 1e-4, "grad_value")
    assert_close(gl, rl, 1e-4, "grad_loc")
    assert_close(ga, ra, 1e-4, "grad_attn")


def test_library_loaded_from_tree():
    """The process loaded the in-tree library (not a copy elsewhere)."""
    from rfdetr_jax_amd.build import LIB_PATH

    maps = open(f"/proc/{os.getpid()}/maps").read()
    assert os.path.realpath(LIB_PATH) in maps or LIB_PATH in maps


def test_far_out_locations_contribute_nothing():
    """Locations whose pixel coordinates leave the int32 range (|loc| up to 1e10, also 2^31 / W
    exactly and just past it): every corner is masked, so those samples add nothing to the output
    or to grad_value, and their weight and location gradients are zero, as the float64 oracle has
    it. The other samples of the same queries are unaffected."""
    shapes = ((24, 24), (12, 12))
    value, loc, attn, grad = make_inputs(44, 2, 4, 16, 200, shapes, 3)
    far = np.array([1e10, -1e10, 3e9, -3e9, 2.0 ** 31 / 24, -(2.0 ** 31) / 24, 1e6, -1e6], np.float32)
    rng = np.random.default_rng(45)
    sel = rng.random(loc.shape[:-1]) < 0.3
    loc = loc.copy()
    loc[sel, 0] = rng.choice(far, int(sel.sum()))
    loc[sel, 1] = rng.choice(far, int(sel.sum()))
    _note("far-out locations")
    out, (gv, gl, ga) = _run(value, shapes, loc, attn, grad)
    assert_close(out, R.ms_deform_attn_core_rows(value, shapes, loc, attn), 1e-5, "out")
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    assert_close(gv, rv, 1e-4, "grad_value")
    assert_close(gl, rl, 1e-4, "grad_loc")
    assert_close(ga, ra, 1e-4, "grad_attn")
    ga5 = ga.reshape(loc.shape[:-1])
    assert not ga5[sel].any() and not gl[sel].any()
