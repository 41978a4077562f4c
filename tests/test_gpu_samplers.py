"""Every sampler name the reference's dispatcher accepts (src/rfdetr_jax/models/ops.py:235-238,
:277-280: "gather", "gather-f32", "matmul", "auto", "pallas", plus this library's "hip") runs the
HIP kernels end to end through autograd, in f32 and bf16, against the float64 oracle.

The reference's samplers compute one function and differ in where a bf16 value map is rounded and,
for "pallas", in how pixel coordinates are formed. The kernels reproduce those points
(msda_fwd_sampler): on a bf16 map each sampler's forward is held to 2e-6 of the oracle's
restatement of that sampler (oracle/msda_ref.py ms_deform_attn_core_rows_sampler; only the f32
sum over levels and points differs from its float64 one), far inside the 1e-3-scale gaps between
the samplers. Gradients are the f32 VJP at each sampler's coordinates. Other tolerances as in
test_gpu_parity: f32 1e-5 (output) and 1e-4 (gradients); bf16 gradients against f32 math on the
bf16-rounded values with 2e-2 (tests/test_ops.py:238 of the reference).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import msda_ref as R
from rfdetr_jax_amd import ops as hip
from rfdetr_jax_amd.workloads import make_inputs
from tests._util import assert_close

pytestmark = pytest.mark.gpu

SHAPES = ((24, 24), (12, 12))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("sampler", ["gather", "gather-f32", "matmul", "auto", "pallas", "hip"])
def test_sampler_names_run_the_hip_path_with_autograd(sampler, dtype):
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    sys.stderr.write(f"[gpu] sampler={sampler} dtype={dtype}\n")
    sys.stderr.flush()
    dev = torch.device("cuda:0")
    bf16 = dtype == "bf16"
    value, loc, attn, grad = make_inputs(7, 2, 4, 16, 333, SHAPES, 2)
    if bf16:
        value = R.bf16_round(value)
    v = torch.from_numpy(value).to(dev)
    if bf16:
        v = v.to(torch.bfloat16)
    v.requires_grad_(True)
    lc = torch.from_numpy(loc).to(dev).requires_grad_(True)
    a = torch.from_numpy(attn).to(dev).requires_grad_(True)
    g = torch.from_numpy(grad).to(dev)
    out = hip.ms_deform_attn_core_rows(v, SHAPES, lc, a, sampler)
    assert out.is_cuda and out.dtype == torch.float32 and tuple(out.shape) == (2, 333, 64)
    (out * g).sum().backward()
    torch.cuda.synchronize()
    tf, tg = (2e-6, 2e-2) if bf16 else (1e-5, 1e-4)
    want = R.ms_deform_attn_core_rows_sampler(value, SHAPES, loc, attn, sampler, bf16)
    assert_close(out.detach().cpu().numpy(), want, tf, f"{sampler} out")
    vjp = R.ms_deform_attn_core_rows_vjp_pallas if sampler == "pallas" else R.ms_deform_attn_core_rows_vjp
    rv, rl, ra = vjp(value, SHAPES, loc, attn, grad)
    assert v.grad.dtype == v.dtype  # grad_value in the value dtype (deform_pallas.py:175)
    assert_close(v.grad.float().cpu().numpy(), rv, tg, f"{sampler} grad_value")
    assert_close(lc.grad.cpu().numpy(), rl, tg, f"{sampler} grad_loc")
    assert_close(a.grad.cpu().numpy(), ra, tg, f"{sampler} grad_attn")


def test_unknown_sampler_name_is_rejected_like_the_reference():
    v = torch.zeros(2, 720, 16, device="cuda")
    with pytest.raises(ValueError, match="unknown sampler"):
        hip.ms_deform_attn_core_rows(v, SHAPES, torch.zeros(1, 3, 2, 2, 2, 2, device="cuda"),
                                     torch.zeros(1, 3, 2, 4, device="cuda"), "bilinear")


def _boundary_locations(loc, shapes, rng, frac=0.25):
    """Moves a share of the sampling locations to floats within a few ulps of cell boundaries
    ((k + 1/2) / size), where the two pixel-coordinate formulas can floor differently."""
    loc = loc.copy()
    for lvl, (h, w) in enumerate(shapes):
        for axis, size in ((0, w), (1, h)):
            sel = rng.random(loc.shape[:3] + (loc.shape[4],)) < frac
            k = rng.integers(0, size, sel.shape)
            edge = ((k + 0.5) / size).astype(np.float32)
            ulps = rng.integers(-4, 5, sel.shape)
            moved = edge.copy()
            for _ in range(4):
                step = np.where(ulps > 0, np.nextafter(moved, np.float32(2)), np.where(ulps < 0, np.nextafter(moved, np.float32(-1)), moved))
                moved = step.astype(np.float32)
                ulps = ulps - np.sign(ulps)
            cur = loc[:, :, :, lvl, :, axis]
            loc[:, :, :, lvl, :, axis] = np.where(sel, moved, cur)
    return loc


@pytest.mark.parametrize("sampler", ["gather", "gather-f32", "matmul", "auto"])
def test_bf16_forward_reproduces_the_samplers_rounding_points(sampler):
    """bf16 value map, the two-level shape (80 x 80 takes "auto"'s gather branch, 20 x 20 its
    matmul one): the forward equals the oracle's restatement of the named sampler within 2e-6,
    while this library's f32 interpolation ("hip") lies 1e-4 or more away from it."""
    sys.stderr.write(f"[gpu] bf16 rounding points sampler={sampler}\n")
    sys.stderr.flush()
    dev = torch.device("cuda:0")
    shapes = ((80, 80), (20, 20))
    value, loc, attn, _ = make_inputs(9, 2, 4, 16, 300, shapes, 4)
    value = R.bf16_round(value)
    v = torch.from_numpy(value).to(dev).to(torch.bfloat16)
    lc, a = torch.from_numpy(loc).to(dev), torch.from_numpy(attn).to(dev)
    got = hip.ms_deform_attn_forward(v, shapes, lc, a, sampler=sampler).cpu().numpy()
    f32_path = hip.ms_deform_attn_forward(v, shapes, lc, a).cpu().numpy()
    want = R.ms_deform_attn_core_rows_sampler(value, shapes, loc, attn, sampler, True)
    assert_close(got, want, 2e-6, f"{sampler} forward")
    scale = max(1.0, float(np.abs(want).max()))
    assert float(np.abs(f32_path - want).max()) / scale > 1e-4, "the f32 path should not already match the rounding points"


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_pallas_pixel_coordinates_forward_and_backward(dtype):
    """The "pallas" sampler floors loc * size - 0.5 (deform_pallas.py:223-224): with a quarter of
    the locations within a few ulps of cell boundaries, where ops.py's formula floors differently
    for some of them, the forward and all gradients follow the Pallas restatement (1e-5 / 1e-4).
    Interpolation is continuous across a cell boundary but its slope is not, so a flipped floor
    shows in grad_sampling_locations (by up to about half its scale at these inputs)."""
    sys.stderr.write(f"[gpu] pallas coordinates dtype={dtype}\n")
    sys.stderr.flush()
    dev = torch.device("cuda:0")
    shapes = ((20, 80), (10, 40))
    rng = np.random.default_rng(31)
    value, loc, attn, grad = make_inputs(10, 2, 4, 16, 257, shapes, 2)
    loc = _boundary_locations(loc, shapes, rng)
    bf16 = dtype == "bf16"
    if bf16:
        value = R.bf16_round(value)
    v = torch.from_numpy(value).to(dev)
    if bf16:
        v = v.to(torch.bfloat16)
    v.requires_grad_(True)
    lc = torch.from_numpy(loc).to(dev).requires_grad_(True)
    a = torch.from_numpy(attn).to(dev).requires_grad_(True)
    out = hip.ms_deform_attn_core_rows(v, shapes, lc, a, "pallas")
    (out * torch.from_numpy(grad).to(dev)).sum().backward()
    torch.cuda.synchronize()
    want = R.ms_deform_attn_core_rows_sampler(value, shapes, loc, attn, "pallas", bf16)
    assert_close(out.detach().cpu().numpy(), want, 1e-5, "pallas out")
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp_pallas(value, shapes, loc, attn, grad)
    tg = 2e-2 if bf16 else 1e-4
    assert_close(v.grad.float().cpu().numpy(), rv, tg, "pallas grad_value")
    assert_close(lc.grad.cpu().numpy(), rl, tg, "pallas grad_loc")
    assert_close(a.grad.cpu().numpy(), ra, tg, "pallas grad_attn")
    # ops.py's coordinates at the same locations give another location gradient somewhere
    gl_ops = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)[1]
    assert float(np.abs(gl_ops - rl).max()) > 1e-2 * float(np.abs(rl).max())
