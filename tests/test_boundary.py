"""The C ABI and the host-side mirror, without a GPU.

* The HIP library loads and exports every function the headers under include/ declare.
* Malformed calls return the documented error codes and messages; validation runs before any HIP
  call, so these run on any host (no kernel is launched).
* The Python mirror of ``ms_deform_attn_core_rows`` rejects unknown samplers and inconsistent
  shapes as the reference does (ops.py:235-238), and refuses CPU tensors (there is no CPU path).
"""

from __future__ import annotations

import ctypes
import glob
import os
import re

import pytest
import torch

from rfdetr_jax_amd import _native
from rfdetr_jax_amd import ops as hip_ops
from rfdetr_jax_amd.build import LIB_PATH

INCLUDE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")


def _declared_functions():
    """Every msda_* function the headers under include/ declare."""
    names = set()
    for header in sorted(glob.glob(os.path.join(INCLUDE, "*.h"))):
        text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
        names.update(re.findall(r"\b(msda_\w+)\s*\(", text))
    return sorted(names)


def test_library_is_built():
    assert os.path.exists(LIB_PATH), f"run __graft_entry__.build() first: {LIB_PATH} missing"


def test_library_exports_every_declared_function():
    declared = _declared_functions()
    assert {"msda_fwd", "msda_bwd", "msda_bwd_workspace_size", "msda_version", "msda_last_error"} <= set(declared)
    lib = ctypes.CDLL(LIB_PATH)
    for name in declared:
        assert hasattr(lib, name), f"{name} declared under include/ but not exported"
    assert set(declared) == set(_native.SIGNATURES), "ctypes signatures out of sync with include/*.h"


def test_version():
    assert _native.lib().msda_version().decode().startswith("msda-gfx950")


# --------------------------------------------------------------------------------------------
# argument validation through the raw C ABI (no GPU work happens on these paths)


def _shapes(pairs):
    flat = [v for hw in pairs for v in hw]
    return (ctypes.c_int32 * len(flat))(*flat)


def _starts(vals):
    return (ctypes.c_int32 * len(vals))(*vals)


def _fwd(sampler=None, **kw):
    """msda_fwd, or msda_fwd_sampler with the given sampler code."""
    args = dict(value=1 << 20, vdt=0, loc=1 << 20, attn=1 << 20, out=1 << 20, odt=0, batch=1, heads=2, dim=16,
                queries=4, levels=1, points=2, shapes=_shapes([(4, 4)]), starts=_starts([0]), len_value=16)
    args.update(kw)
    lib = _native.lib()
    head = (ctypes.c_void_p(args["value"]), args["vdt"], ctypes.c_void_p(args["loc"]), ctypes.c_void_p(args["attn"]),
            ctypes.c_void_p(args["out"]), args["odt"])
    dims = (args["batch"], args["heads"], args["dim"], args["queries"], args["levels"], args["points"], args["shapes"],
            args["starts"], args["len_value"], None)
    rc = lib.msda_fwd(*head, *dims) if sampler is None else lib.msda_fwd_sampler(*head, sampler, *dims)
    return rc, lib.msda_last_error().decode()


def _bwd(sampler=None, **kw):
    """msda_bwd, or msda_bwd_sampler with the given sampler code."""
    args = dict(value=1 << 20, vdt=0, loc=1 << 20, attn=1 << 20, gout=1 << 20, gdt=0, dv=1 << 20, dl=1 << 20,
                da=1 << 20, batch=1, heads=2, dim=16, queries=4, levels=1, points=2, shapes=_shapes([(4, 4)]),
                starts=_starts([0]), len_value=16, ws=1 << 20, ws_bytes=1 << 20)
    args.update(kw)
    lib = _native.lib()
    head = (ctypes.c_void_p(args["value"]), args["vdt"], ctypes.c_void_p(args["loc"]), ctypes.c_void_p(args["attn"]),
            ctypes.c_void_p(args["gout"]), args["gdt"], ctypes.c_void_p(args["dv"]), ctypes.c_void_p(args["dl"]),
            ctypes.c_void_p(args["da"]))
    dims = (args["batch"], args["heads"], args["dim"], args["queries"], args["levels"], args["points"], args["shapes"],
            args["starts"], args["len_value"], ctypes.c_void_p(args["ws"]), args["ws_bytes"], None)
    rc = lib.msda_bwd(*head, *dims) if sampler is None else lib.msda_bwd_sampler(*head, sampler, *dims)
    return rc, lib.msda_last_error().decode()


def _fwd_gather(**kw):
    return _fwd(sampler=1, **kw)


def _bwd_pallas(**kw):
    return _bwd(sampler=5, **kw)


@pytest.mark.parametrize("call", [_fwd, _bwd, _fwd_gather, _bwd_pallas])
@pytest.mark.parametrize(
    "kw, code, message",
    [
        (dict(starts=_starts([3])), _native.ERR_INVALID_ARGUMENT, "level_start_index"),
        (dict(len_value=17), _native.ERR_INVALID_ARGUMENT, "len_value"),
        (dict(levels=0), _native.ERR_INVALID_ARGUMENT, "n_levels"),
        (dict(levels=17), _native.ERR_INVALID_ARGUMENT, "n_levels"),
        (dict(shapes=_shapes([(0, 16)]), len_value=0), _native.ERR_INVALID_ARGUMENT, "positive"),
        (dict(heads=0), _native.ERR_INVALID_ARGUMENT, "n_heads"),
        (dict(points=0), _native.ERR_INVALID_ARGUMENT, "n_points"),
        (dict(batch=-1), _native.ERR_INVALID_ARGUMENT, "batch"),
        (dict(vdt=7), _native.ERR_UNSUPPORTED, "dtype"),
        (dict(dim=2048, shapes=_shapes([(4, 4)])), _native.ERR_UNSUPPORTED, "head_dim"),
        (dict(shapes=None), _native.ERR_INVALID_ARGUMENT, "spatial_shapes"),
    ],
)
def test_invalid_arguments_are_reported(call, kw, code, message):
    rc, msg = call(**kw)
    assert rc == code, msg
    assert message in msg


@pytest.mark.parametrize("call", [_fwd, _bwd])
@pytest.mark.parametrize("code", [-1, 6, 99])
def test_unknown_sampler_code_is_rejected(call, code):
    rc, msg = call(sampler=code)
    assert rc == _native.ERR_INVALID_ARGUMENT and "unknown sampler code" in msg


def test_two_levels_level_start_index_checked():
    pairs = [(4, 4), (2, 2)]
    rc, msg = _fwd(levels=2, shapes=_shapes(pairs), starts=_starts([0, 16]), len_value=20, value=0)
    assert rc == _native.ERR_INVALID_ARGUMENT and "NULL" in msg  # shapes fine, then the NULL value
    rc, msg = _fwd(levels=2, shapes=_shapes(pairs), starts=_starts([0, 15]), len_value=20)
    assert rc == _native.ERR_INVALID_ARGUMENT and "level_start_index[1]" in msg


def test_workspace_size_validates_first():
    """The size query validates its shape before touching the device; empty shapes need nothing.
    (Otherwise the size depends on the device's CU count and LDS size: the query blocks' partial
    grad_value sums; it is checked on the GPU.)"""
    lib = _native.lib()
    assert lib.msda_bwd_workspace_size(1, 2, 16, 4, 1, 2, _shapes([(4, 4)]), _starts([3]), 16) == _native.ERR_INVALID_ARGUMENT
    assert lib.msda_bwd_workspace_size(0, 2, 16, 4, 1, 2, _shapes([(4, 4)]), _starts([0]), 16) == 0
    assert lib.msda_bwd_workspace_size(1, 2, 16, 0, 1, 2, _shapes([(4, 4)]), _starts([0]), 16) == 0


def test_workspace_checked_only_when_the_plan_splits_queries():
    """A NULL workspace passes validation for a shape whose plan does not split queries (on a host
    without a GPU the call then stops at the device query)."""
    for ws in (0, (1 << 20) + 8):
        rc, msg = _bwd(ws=ws, ws_bytes=0)
        assert "workspace" not in msg
        assert rc in (_native.OK, _native.ERR_DEVICE), msg


def test_misaligned_locations_rejected():
    rc, msg = _fwd(loc=(1 << 20) + 4)
    assert rc == _native.ERR_INVALID_ARGUMENT and "aligned" in msg


def test_empty_calls_are_no_ops():
    """batch = 0 (both) and len_query = 0 (forward) succeed without touching the device."""
    assert _fwd(batch=0)[0] == _native.OK
    assert _fwd(queries=0)[0] == _native.OK
    assert _bwd(batch=0)[0] == _native.OK
    assert _bwd(dv=0, dl=0, da=0)[0] == _native.OK  # nothing requested


def test_error_message_is_per_call():
    _fwd(levels=0)
    assert _fwd(batch=0)[1] == ""


# --------------------------------------------------------------------------------------------
# host-side mirror of the reference interface


def _cpu_inputs(b=1, q=3, h=2, l=1, p=2, d=4, shapes=((4, 4),)):
    s = sum(x * y for x, y in shapes)
    return (torch.zeros(b * h, s, d), torch.zeros(b, q, h, l, p, 2), torch.zeros(b, q, h, l * p))


def test_unknown_sampler_is_rejected():
    value, loc, attn = _cpu_inputs()
    with pytest.raises(ValueError, match="unknown sampler"):
        hip_ops.ms_deform_attn_core_rows(value, ((4, 4),), loc, attn, "nearest")


def test_reference_sampler_names_are_accepted():
    assert set(hip_ops.SAMPLERS) >= {"gather", "gather-f32", "matmul", "auto", "pallas", "hip"}


def test_cpu_tensors_fail_loudly():
    value, loc, attn = _cpu_inputs()
    with pytest.raises(RuntimeError, match="no CPU path"):
        hip_ops.ms_deform_attn_core_rows(value, ((4, 4),), loc, attn, "gather")


def test_level_start_index_must_match():
    value, loc, attn = _cpu_inputs(l=2, shapes=((4, 4), (2, 2)))
    with pytest.raises(ValueError, match="level_start_index"):
        hip_ops.ms_deform_attn(value, ((4, 4), (2, 2)), torch.tensor([0, 15]), loc, attn)


@pytest.mark.parametrize(
    "bad",
    ["value_rows", "value_len", "levels", "weights"],
)
def test_inconsistent_shapes_are_rejected(bad):
    value, loc, attn = _cpu_inputs()
    shapes = ((4, 4),)
    if bad == "value_rows":
        value = torch.zeros(3, 16, 4)
    elif bad == "value_len":
        value = torch.zeros(2, 15, 4)
    elif bad == "levels":
        shapes = ((4, 4), (2, 2))
    else:
        attn = torch.zeros(1, 3, 2, 3)
    with pytest.raises(ValueError):
        hip_ops.ms_deform_attn_forward(value, shapes, loc, attn)


def test_unsupported_value_dtype():
    value, loc, attn = _cpu_inputs()
    with pytest.raises(TypeError, match="not supported"):
        hip_ops.ms_deform_attn_forward(value.double(), ((4, 4),), loc, attn)


# --------------------------------------------------------------------------------------------
# fused-prologue entry points (msda_fused_fwd / msda_fused_bwd)


def _ffwd(**kw):
    args = dict(value=1 << 20, vdt=0, ref=1 << 20, ref_dim=4, off=1 << 20, logits=1 << 20, out=1 << 20, odt=0, batch=1,
                heads=2, dim=16, queries=4, levels=1, points=2, shapes=_shapes([(4, 4)]), starts=_starts([0]), len_value=16)
    args.update(kw)
    lib = _native.lib()
    rc = lib.msda_fused_fwd(
        ctypes.c_void_p(args["value"]), args["vdt"], ctypes.c_void_p(args["ref"]), args["ref_dim"],
        ctypes.c_void_p(args["off"]), ctypes.c_void_p(args["logits"]), ctypes.c_void_p(args["out"]), args["odt"],
        args["batch"], args["heads"], args["dim"], args["queries"], args["levels"], args["points"], args["shapes"],
        args["starts"], args["len_value"], None,
    )
    return rc, lib.msda_last_error().decode()


def _fbwd(**kw):
    args = dict(value=1 << 20, vdt=0, ref=1 << 20, ref_dim=2, off=1 << 20, logits=1 << 20, gout=1 << 20, gdt=0,
                dv=1 << 20, doff=1 << 20, dlog=1 << 20, dref=1 << 20, batch=1, heads=2, dim=16, queries=4, levels=1,
                points=2, shapes=_shapes([(4, 4)]), starts=_starts([0]), len_value=16, ws=1 << 20, ws_bytes=1 << 20)
    args.update(kw)
    lib = _native.lib()
    rc = lib.msda_fused_bwd(
        ctypes.c_void_p(args["value"]), args["vdt"], ctypes.c_void_p(args["ref"]), args["ref_dim"],
        ctypes.c_void_p(args["off"]), ctypes.c_void_p(args["logits"]), ctypes.c_void_p(args["gout"]), args["gdt"],
        ctypes.c_void_p(args["dv"]), ctypes.c_void_p(args["doff"]), ctypes.c_void_p(args["dlog"]),
        ctypes.c_void_p(args["dref"]), args["batch"], args["heads"], args["dim"], args["queries"], args["levels"],
        args["points"], args["shapes"], args["starts"], args["len_value"], ctypes.c_void_p(args["ws"]), args["ws_bytes"],
        None,
    )
    return rc, lib.msda_last_error().decode()


@pytest.mark.parametrize("call", [_ffwd, _fbwd])
@pytest.mark.parametrize(
    "kw, code, message",
    [
        (dict(ref_dim=3), _native.ERR_INVALID_ARGUMENT, "ref_dim"),
        (dict(ref_dim=0), _native.ERR_INVALID_ARGUMENT, "ref_dim"),
        (dict(ref=0), _native.ERR_INVALID_ARGUMENT, "reference_points is NULL"),
        (dict(ref=(1 << 20) + 4), _native.ERR_INVALID_ARGUMENT, "reference_points must be"),
        (dict(starts=_starts([3])), _native.ERR_INVALID_ARGUMENT, "level_start_index"),
        (dict(vdt=7), _native.ERR_UNSUPPORTED, "dtype"),
        (dict(off=(1 << 20) + 4), _native.ERR_INVALID_ARGUMENT, "aligned"),
    ],
)
def test_fused_invalid_arguments_are_reported(call, kw, code, message):
    rc, msg = call(**kw)
    assert rc == code, msg
    assert message in msg


def test_fused_workspace_size_validates_first():
    lib = _native.lib()
    f = lib.msda_fused_bwd_workspace_size
    assert f(1, 2, 16, 4, 1, 2, 3, _shapes([(4, 4)]), _starts([0]), 16) == _native.ERR_INVALID_ARGUMENT
    assert "ref_dim" in lib.msda_last_error().decode()
    assert f(1, 2, 16, 4, 1, 2, 4, _shapes([(4, 4)]), _starts([3]), 16) == _native.ERR_INVALID_ARGUMENT
    assert f(0, 2, 16, 4, 1, 2, 4, _shapes([(4, 4)]), _starts([0]), 16) == 0
    assert f(1, 2, 16, 0, 1, 2, 2, _shapes([(4, 4)]), _starts([0]), 16) == 0


def test_fused_workspace_needed_for_any_gradient():
    """The prologue's locations and weights live in the workspace, whatever gradient is asked."""
    rc, msg = _fbwd(ws=0)
    assert rc == _native.ERR_INVALID_ARGUMENT and "workspace" in msg
    rc, msg = _fbwd(ws=0, dv=0, dref=0, dlog=0)  # grad_sampling_offsets alone
    assert rc == _native.ERR_INVALID_ARGUMENT and "workspace" in msg


def test_fused_empty_calls_are_no_ops():
    assert _ffwd(batch=0)[0] == _native.OK
    assert _ffwd(queries=0)[0] == _native.OK
    assert _fbwd(batch=0)[0] == _native.OK
    assert _fbwd(dv=0, doff=0, dlog=0, dref=0)[0] == _native.OK


def _cpu_fused_inputs(ref_dim=4, b=1, q=3, h=2, l=1, p=2, d=4, shapes=((4, 4),)):
    value, off, logits = _cpu_inputs(b, q, h, l, p, d, shapes)
    return value, torch.zeros(b, q, l, ref_dim), off, logits


def test_fused_mirror_rejects_bad_reference_points():
    value, ref, off, logits = _cpu_fused_inputs()
    with pytest.raises(ValueError, match="2 or 4"):
        hip_ops.ms_deform_attn_fused_forward(value, ((4, 4),), torch.zeros(1, 3, 1, 3), off, logits)
    with pytest.raises(ValueError, match="reference_points"):
        hip_ops.ms_deform_attn_fused_forward(value, ((4, 4),), torch.zeros(1, 2, 1, 4), off, logits)


def test_fused_cpu_tensors_fail_loudly():
    value, ref, off, logits = _cpu_fused_inputs()
    with pytest.raises(RuntimeError, match="no CPU path"):
        hip_ops.ms_deform_attn_fused(value, ((4, 4),), ref, off, logits)


# --------------------------------------------------------------------------------------------
# grid sampling (msda_grid_sample_fwd / msda_grid_sample_bwd) and its mirror


def _gs_fwd(**kw):
    args = dict(inp=1 << 20, dt=0, grid=1 << 20, kind=0, out=1 << 20, n=2, c=1, h=8, w=8, p=16, pad=0, mode=0)
    args.update(kw)
    lib = _native.lib()
    rc = lib.msda_grid_sample_fwd(ctypes.c_void_p(args["inp"]), args["dt"], ctypes.c_void_p(args["grid"]), args["kind"],
                                  ctypes.c_void_p(args["out"]), args["n"], args["c"], args["h"], args["w"], args["p"],
                                  args["pad"], args["mode"], None)
    return rc, lib.msda_last_error().decode()


def _gs_bwd(**kw):
    args = dict(inp=1 << 20, dt=0, grid=1 << 20, kind=1, gout=1 << 20, gin=1 << 20, ggrid=1 << 20, n=2, c=1, h=8, w=8, p=16,
                pad=1, mode=0)
    args.update(kw)
    lib = _native.lib()
    rc = lib.msda_grid_sample_bwd(ctypes.c_void_p(args["inp"]), args["dt"], ctypes.c_void_p(args["grid"]), args["kind"],
                                  ctypes.c_void_p(args["gout"]), ctypes.c_void_p(args["gin"]), ctypes.c_void_p(args["ggrid"]),
                                  args["n"], args["c"], args["h"], args["w"], args["p"], args["pad"], args["mode"], None)
    return rc, lib.msda_last_error().decode()


@pytest.mark.parametrize("call", [_gs_fwd, _gs_bwd])
@pytest.mark.parametrize(
    "kw, code, message",
    [
        (dict(dt=5), _native.ERR_UNSUPPORTED, "dtype"),
        (dict(pad=2), _native.ERR_INVALID_ARGUMENT, "padding_mode"),
        (dict(kind=3), _native.ERR_INVALID_ARGUMENT, "grid_kind"),
        (dict(mode=2), _native.ERR_INVALID_ARGUMENT, "sample mode"),
        (dict(mode=1, pad=0), _native.ERR_UNSUPPORTED, "border padding only"),
        (dict(c=0), _native.ERR_INVALID_ARGUMENT, "channels"),
        (dict(n=-1), _native.ERR_INVALID_ARGUMENT, "n ("),
        (dict(grid=0), _native.ERR_INVALID_ARGUMENT, "NULL"),
        (dict(grid=(1 << 20) + 4), _native.ERR_INVALID_ARGUMENT, "aligned"),
    ],
)
def test_grid_sample_invalid_arguments_are_reported(call, kw, code, message):
    rc, msg = call(**kw)
    assert rc == code, msg
    assert message in msg


def test_grid_sample_empty_calls_are_no_ops():
    assert _gs_fwd(n=0)[0] == _native.OK
    assert _gs_fwd(p=0)[0] == _native.OK
    assert _gs_bwd(n=0)[0] == _native.OK
    assert _gs_bwd(gin=0, ggrid=0)[0] == _native.OK


def test_grid_sample_mirror_errors():
    from rfdetr_jax_amd import grid_sample as gs

    inputs, grid = torch.zeros(1, 1, 2, 2), torch.zeros(1, 1, 1, 2)
    with pytest.raises(ValueError, match="padding_mode"):
        gs.bilinear_grid_sample(inputs, grid, "reflection")
    with pytest.raises(ValueError, match="bilinear and nearest"):
        gs.point_sample(inputs, torch.zeros(1, 1, 2), mode="bicubic")
    with pytest.raises(RuntimeError, match="no CPU path"):
        gs.point_sample(inputs, torch.zeros(1, 1, 2))
    with pytest.raises(TypeError, match="not supported"):
        gs.bilinear_grid_sample(inputs.double(), grid)


# --------------------------------------------------------------------------------------------
# value projection (msda_value_proj_fwd / msda_value_proj_bwd)


def _vp_fwd(**kw):
    args = dict(x=1 << 20, dt=0, w=1 << 20, b=1 << 20, m=0, v=1 << 20, batch=2, s=16, k=32, h=2, d=16)
    args.update(kw)
    lib = _native.lib()
    rc = lib.msda_value_proj_fwd(ctypes.c_void_p(args["x"]), args["dt"], ctypes.c_void_p(args["w"]), ctypes.c_void_p(args["b"]),
                                 ctypes.c_void_p(args["m"]), ctypes.c_void_p(args["v"]), args["batch"], args["s"], args["k"],
                                 args["h"], args["d"], None)
    return rc, lib.msda_last_error().decode()


def _vp_bwd(**kw):
    args = dict(x=1 << 20, dt=0, w=1 << 20, m=0, gv=1 << 20, gx=1 << 20, gw=1 << 20, gb=1 << 20, batch=2, s=16, k=32, h=2, d=16,
                ws=1 << 20, ws_bytes=1 << 24)
    args.update(kw)
    lib = _native.lib()
    rc = lib.msda_value_proj_bwd(ctypes.c_void_p(args["x"]), args["dt"], ctypes.c_void_p(args["w"]), ctypes.c_void_p(args["m"]),
                                 ctypes.c_void_p(args["gv"]), ctypes.c_void_p(args["gx"]), ctypes.c_void_p(args["gw"]),
                                 ctypes.c_void_p(args["gb"]), args["batch"], args["s"], args["k"], args["h"], args["d"],
                                 ctypes.c_void_p(args["ws"]), args["ws_bytes"], None)
    return rc, lib.msda_last_error().decode()


@pytest.mark.parametrize("call", [_vp_fwd, _vp_bwd])
@pytest.mark.parametrize(
    "kw, code, message",
    [
        (dict(dt=9), _native.ERR_UNSUPPORTED, "dtype"),
        (dict(batch=-1), _native.ERR_INVALID_ARGUMENT, "batch"),
        (dict(k=0), _native.ERR_INVALID_ARGUMENT, "in_features"),
        (dict(h=0), _native.ERR_INVALID_ARGUMENT, "n_heads"),
        (dict(w=0), _native.ERR_INVALID_ARGUMENT, "NULL"),
        (dict(w=(1 << 20) + 2), _native.ERR_INVALID_ARGUMENT, "aligned"),
    ],
)
def test_value_proj_invalid_arguments_are_reported(call, kw, code, message):
    rc, msg = call(**kw)
    assert rc == code, msg
    assert message in msg


def test_value_proj_workspace():
    lib = _native.lib()
    size = lib.msda_value_proj_bwd_workspace_size(2, 16, 32, 2, 16)
    assert size == 1 * 32 * 33 * 4  # one split of the 32 rows; [splits][N][K + 1] f32
    assert lib.msda_value_proj_bwd_workspace_size(2, 16, 0, 2, 16) == _native.ERR_INVALID_ARGUMENT
    rc, msg = _vp_bwd(ws=0)
    assert rc == _native.ERR_INVALID_ARGUMENT and "workspace" in msg
    rc, msg = _vp_bwd(ws_bytes=16)
    assert rc == _native.ERR_INVALID_ARGUMENT and "workspace of" in msg
    assert _vp_bwd(gw=0, gb=0, gx=0)[0] == _native.OK  # nothing requested
    assert _vp_fwd(batch=0)[0] == _native.OK


def test_ms_deform_attn_module_mirror_errors():
    from rfdetr_jax_amd import MSDeformAttn
    from rfdetr_jax_amd.value_proj import value_proj_rows

    m = MSDeformAttn(d_model=32, n_levels=1, n_heads=4, n_points=2)
    names = {n for n, _ in m.named_parameters()}
    assert names == {f"{p}.{w}" for p in ("sampling_offsets", "attention_weights", "value_proj", "output_proj") for w in ("weight", "bias")}
    with pytest.raises(ValueError, match="Last dim of reference_points must be 2 or 4"):
        m(torch.zeros(1, 3, 32), torch.zeros(1, 3, 1, 3), torch.zeros(1, 16, 32), ((4, 4),))
    with pytest.raises(RuntimeError, match="no CPU path"):
        value_proj_rows(torch.zeros(1, 4, 8), torch.zeros(8, 8), None, 2)
    with pytest.raises(ValueError, match="divisible"):
        MSDeformAttn(d_model=30, n_heads=4)


# --------------------------------------------------------------------------------------------
# decoder self-attention (msda_attention_fwd / msda_attention_bwd)


def _at_fwd(**kw):
    args = dict(q=1 << 20, k=1 << 20, v=1 << 20, dt=0, o=1 << 20, st=1 << 20, batch=2, groups=1, heads=2, len=9, d=32,
                strides=[2 * 9 * 32, 0, 9 * 32, 32] * 4, m=0)
    args.update(kw)
    lib = _native.lib()
    strides = (ctypes.c_int64 * len(args["strides"]))(*args["strides"])
    rc = lib.msda_attention_fwd(ctypes.c_void_p(args["q"]), ctypes.c_void_p(args["k"]), ctypes.c_void_p(args["v"]), args["dt"],
                                ctypes.c_void_p(args["o"]), ctypes.c_void_p(args["st"]), args["batch"], args["groups"], args["heads"],
                                args["len"], args["d"], strides, ctypes.c_void_p(args["m"]), None)
    return rc, lib.msda_last_error().decode()


def _at_bwd(**kw):
    args = dict(q=1 << 20, k=1 << 20, v=1 << 20, o=1 << 20, st=1 << 20, go=1 << 20, dt=0, gq=1 << 20, gk=1 << 20, gv=1 << 20,
                batch=2, groups=1, heads=2, len=9, d=32, strides=[2 * 9 * 32, 0, 9 * 32, 32] * 8, m=0)
    args.update(kw)
    lib = _native.lib()
    strides = (ctypes.c_int64 * len(args["strides"]))(*args["strides"])
    rc = lib.msda_attention_bwd(ctypes.c_void_p(args["q"]), ctypes.c_void_p(args["k"]), ctypes.c_void_p(args["v"]),
                                ctypes.c_void_p(args["o"]), ctypes.c_void_p(args["st"]), ctypes.c_void_p(args["go"]), args["dt"],
                                ctypes.c_void_p(args["gq"]), ctypes.c_void_p(args["gk"]), ctypes.c_void_p(args["gv"]), args["batch"],
                                args["groups"], args["heads"], args["len"], args["d"], strides, ctypes.c_void_p(args["m"]), None)
    return rc, lib.msda_last_error().decode()


@pytest.mark.parametrize("call", [_at_fwd, _at_bwd])
@pytest.mark.parametrize(
    "kw, code, message",
    [
        (dict(dt=9), _native.ERR_UNSUPPORTED, "dtype"),
        (dict(d=48), _native.ERR_UNSUPPORTED, "head_dim"),
        (dict(len=-1), _native.ERR_INVALID_ARGUMENT, "negative"),
        (dict(strides=[2 * 9 * 32, 0, 9 * 32, 30] * 8), _native.ERR_INVALID_ARGUMENT, "multiple of 4"),
        # row offsets within a (slice, head) are 32-bit: s_row < 2^24 and len * s_row < 2^31
        (dict(strides=[0, 0, 0, 1 << 24] * 8), _native.ERR_UNSUPPORTED, "row stride"),
        (dict(len=4096, strides=[0, 0, 0, 1 << 20] * 8), _native.ERR_UNSUPPORTED, "row stride"),
        (dict(q=0), _native.ERR_INVALID_ARGUMENT, "NULL"),
        (dict(k=(1 << 20) + 4), _native.ERR_INVALID_ARGUMENT, "aligned"),
    ],
)
def test_attention_invalid_arguments_are_reported(call, kw, code, message):
    rc, msg = call(**kw)
    assert rc == code, msg
    assert message in msg


def test_attention_empty_calls_do_nothing():
    assert _at_fwd(len=0)[0] == _native.OK
    assert _at_fwd(batch=0)[0] == _native.OK
    assert _at_bwd(gq=0, gk=0, gv=0)[0] == _native.OK  # nothing requested


def test_attention_module_mirror_errors():
    from rfdetr_jax_amd.attention import MultiheadAttention, grouped_attention, scaled_dot_product_attention

    m = MultiheadAttention(64, 2)
    assert {n for n, _ in m.named_parameters()} == {"in_proj_weight", "in_proj_bias", "out_proj.weight", "out_proj.bias"}
    assert tuple(m.in_proj_weight.shape) == (192, 64)
    with pytest.raises(ValueError, match="divisible"):
        MultiheadAttention(30, 4)
    with pytest.raises(ValueError, match="one shape"):
        scaled_dot_product_attention(torch.zeros(1, 2, 3, 32), torch.zeros(1, 2, 4, 32), torch.zeros(1, 2, 3, 32))
    with pytest.raises(ValueError, match="groups"):
        grouped_attention(torch.zeros(1, 10, 64), torch.zeros(1, 10, 64), torch.zeros(1, 10, 64), 2, groups=3)
    with pytest.raises(RuntimeError, match="no CPU path"):
        scaled_dot_product_attention(torch.zeros(1, 2, 3, 32), torch.zeros(1, 2, 3, 32), torch.zeros(1, 2, 3, 32))
    with pytest.raises(ValueError, match="dropout rate"):
        scaled_dot_product_attention(torch.zeros(1, 2, 3, 32), torch.zeros(1, 2, 3, 32), torch.zeros(1, 2, 3, 32), dropout=1.5)
    # training with dropout goes to the same kernels (no CPU path either)
    m_drop = MultiheadAttention(64, 2, dropout=0.1).train()
    with pytest.raises(RuntimeError, match="no CPU path"):
        m_drop(torch.zeros(1, 3, 64), torch.zeros(1, 3, 64), torch.zeros(1, 3, 64))


def _at_drop(which, rate, seed=7, **kw):
    """msda_attention_fwd_dropout / _bwd_dropout with _at_fwd's / _at_bwd's defaults."""
    lib = _native.lib()
    if which == "fwd":
        args = dict(q=1 << 20, k=1 << 20, v=1 << 20, dt=0, o=1 << 20, st=1 << 20, batch=2, groups=1, heads=2, len=9, d=32,
                    strides=[2 * 9 * 32, 0, 9 * 32, 32] * 4, m=0)
        args.update(kw)
        strides = (ctypes.c_int64 * len(args["strides"]))(*args["strides"])
        rc = lib.msda_attention_fwd_dropout(ctypes.c_void_p(args["q"]), ctypes.c_void_p(args["k"]), ctypes.c_void_p(args["v"]),
                                            args["dt"], ctypes.c_void_p(args["o"]), ctypes.c_void_p(args["st"]), args["batch"],
                                            args["groups"], args["heads"], args["len"], args["d"], strides, ctypes.c_void_p(args["m"]),
                                            rate, seed, None)
    else:
        args = dict(q=1 << 20, k=1 << 20, v=1 << 20, o=1 << 20, st=1 << 20, go=1 << 20, dt=0, gq=1 << 20, gk=1 << 20, gv=1 << 20,
                    batch=2, groups=1, heads=2, len=9, d=32, strides=[2 * 9 * 32, 0, 9 * 32, 32] * 8, m=0)
        args.update(kw)
        strides = (ctypes.c_int64 * len(args["strides"]))(*args["strides"])
        rc = lib.msda_attention_bwd_dropout(ctypes.c_void_p(args["q"]), ctypes.c_void_p(args["k"]), ctypes.c_void_p(args["v"]),
                                            ctypes.c_void_p(args["o"]), ctypes.c_void_p(args["st"]), ctypes.c_void_p(args["go"]),
                                            args["dt"], ctypes.c_void_p(args["gq"]), ctypes.c_void_p(args["gk"]),
                                            ctypes.c_void_p(args["gv"]), args["batch"], args["groups"], args["heads"], args["len"],
                                            args["d"], strides, ctypes.c_void_p(args["m"]), rate, seed, None)
    return rc, lib.msda_last_error().decode()


@pytest.mark.parametrize("which", ["fwd", "bwd"])
@pytest.mark.parametrize("rate", [-0.1, 1.0, 2.0, float("nan")])
def test_attention_dropout_rate_is_validated(which, rate):
    """Dropout rates outside [0, 1) are refused before any HIP call (flax's rate 1, all weights
    dropped, is the Python mirror's zeros)."""
    rc, msg = _at_drop(which, rate)
    assert rc == _native.ERR_INVALID_ARGUMENT and "dropout rate" in msg, msg


@pytest.mark.parametrize("which", ["fwd", "bwd"])
def test_attention_dropout_shares_the_plain_validation(which):
    assert _at_drop(which, 0.1, d=48)[0] == _native.ERR_UNSUPPORTED
    assert _at_drop(which, 0.1, q=0)[0] == _native.ERR_INVALID_ARGUMENT
    assert _at_drop(which, 0.1, len=0)[0] == _native.OK  # empty: nothing to do


def test_attention_dropout_keep_validation():
    lib = _native.lib()
    assert lib.msda_attention_dropout_keep(2, 1, 2, 9, 1.0, 1, None, None) == _native.ERR_INVALID_ARGUMENT
    assert lib.msda_attention_dropout_keep(2, 1, 2, -1, 0.1, 1, None, None) == _native.ERR_INVALID_ARGUMENT
    assert lib.msda_attention_dropout_keep(2, 1, 2, 9, 0.1, 1, None, None) == _native.ERR_INVALID_ARGUMENT  # NULL keep
    assert lib.msda_attention_dropout_keep(2, 1, 2, 0, 0.1, 1, None, None) == _native.OK
