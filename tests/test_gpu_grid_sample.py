"""Parity of the grid-sampling kernels (msda_grid_sample_fwd / msda_grid_sample_bwd through the C
ABI, via the torch mirror) with the CPU oracle, on an MI355X.

Expected values: oracle/grid_sample_ref.py (float64 after f32 coordinates), the reference's own
known answers, and torch's ``F.grid_sample`` on the GPU. Tolerances as for the core
(``max|got - want| <= tol * max(1, max|want|)``): f32 forward 1e-5, gradients 1e-4; bf16 2e-2.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import grid_sample_ref as GS
from rfdetr_jax_amd import grid_sample as hip
from tests._util import assert_close

pytestmark = pytest.mark.gpu


def _dev():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch.device("cuda:0")


def _note(msg):
    sys.stderr.write(f"[gpu] {msg}\n")
    sys.stderr.flush()


def _t(a, bf16=False):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(_dev())
    return t.to(torch.bfloat16) if bf16 else t


def _np(t):
    return t.detach().float().cpu().numpy()


def test_reference_known_answers():
    """tests/test_ops.py:22-43 and tests/test_segmentation.py:40-45, :107-115 on the GPU."""
    v = _t(np.array([[[[1.0, 2.0], [3.0, 4.0]]]], np.float32))
    out = _np(hip.bilinear_grid_sample(v, _t(np.array([[[[-0.5, -0.5], [0.5, 0.5]]]], np.float32))))[0, 0, 0]
    assert out[0] == pytest.approx(1.0) and out[1] == pytest.approx(4.0)
    assert float(hip.bilinear_grid_sample(_t(np.ones((1, 1, 2, 2), np.float32)), _t(np.full((1, 1, 1, 2), 5.0, np.float32)))[0, 0, 0, 0]) == 0.0
    mid = hip.bilinear_grid_sample(_t(np.array([[[[0.0, 4.0]]]], np.float32)), _t(np.zeros((1, 1, 1, 2), np.float32)))
    assert float(mid[0, 0, 0, 0]) == pytest.approx(2.0)
    nv = _t(np.array([[[[0.0, 1.0], [2.0, 3.0]]]], np.float32))
    assert float(hip.point_sample(nv, _t(np.array([[[0.75, 0.75]]], np.float32)), mode="nearest")[0, 0, 0]) == 3.0
    bv = _t(np.array([[[[2.0, 4.0], [6.0, 8.0]]]], np.float32))
    for pt, want in (((0.0, 0.0), 2.0), ((1.0, 1.0), 8.0), ((0.5, 0.5), 5.0)):
        assert float(hip.point_sample(bv, _t(np.array([[pt]], np.float32)))[0, 0, 0]) == want


CASES = {
    "mask_loss": dict(n=48, c=1, h=56, w=56, gh=196, gw=1),       # C = 1 mask logits, P = H*W/16 points
    "channels": dict(n=3, c=6, h=7, w=9, gh=5, gw=6),             # several channels, odd sizes
    "banded": dict(n=2, c=3, h=160, w=144, gh=40, gw=3),          # planes above the LDS budget: row bands
}


def _case(seed, n, c, h, w, gh, gw, lo=-1.3, hi=1.3):
    rng = np.random.default_rng(seed)
    inputs = rng.standard_normal((n, c, h, w)).astype(np.float32)
    grid = rng.uniform(lo, hi, (n, gh, gw, 2)).astype(np.float32)
    grad = rng.standard_normal((n, c, gh, gw)).astype(np.float32)
    return inputs, grid, grad


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("padding_mode", ["zeros", "border"])
@pytest.mark.parametrize("case", sorted(CASES))
def test_bilinear_grid_sample_against_oracle(case, padding_mode, bf16):
    c = CASES[case]
    _note(f"grid sample {case} {padding_mode} bf16={bf16}")
    inputs, grid, grad = _case(21, **c)
    if bf16:
        inputs = GS_bf16(inputs)
        grad = GS_bf16(grad)
    ti = _t(inputs, bf16).requires_grad_(True)
    tg = _t(grid).requires_grad_(True)
    out = hip.bilinear_grid_sample(ti, tg, padding_mode)
    out.backward(_t(grad, bf16))
    tol_f, tol_g = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(_np(out), GS.bilinear_grid_sample(inputs, grid, padding_mode), tol_f, "out")
    gi, gg = GS.grid_sample_vjp(inputs, grid, grad, padding_mode)
    assert_close(_np(ti.grad), gi, tol_g, "grad_input")
    assert_close(_np(tg.grad), gg, tol_g, "grad_grid")


def GS_bf16(x):
    from oracle.msda_ref import bf16_round

    return bf16_round(x)


@pytest.mark.parametrize("mode", ["bilinear", "nearest"])
@pytest.mark.parametrize("shape", ["flat", "grid"])
def test_point_sample_against_oracle(mode, shape):
    rng = np.random.default_rng(22)
    inputs = rng.standard_normal((40, 2, 28, 36)).astype(np.float32)
    pts = rng.uniform(-0.1, 1.1, (40, 150, 2) if shape == "flat" else (40, 10, 15, 2)).astype(np.float32)
    grad = rng.standard_normal((40, 2) + pts.shape[1:-1]).astype(np.float32)
    ti = _t(inputs).requires_grad_(True)
    tp = _t(pts).requires_grad_(True)
    out = hip.point_sample(ti, tp, mode)
    out.backward(_t(grad))
    want = GS.point_sample(inputs, pts, mode)
    gi, gp = GS.point_sample_vjp(inputs, pts, grad, mode)
    if mode == "nearest":
        # the kernel and the oracle round the same f32 coordinate; exact halves are not drawn
        assert np.array_equal(_np(out), want.astype(np.float32))
    else:
        assert_close(_np(out), want, 1e-5, "out")
    assert_close(_np(ti.grad), gi, 1e-4, "grad_input")
    assert_close(_np(tp.grad), gp, 1e-4, "grad_points")


def test_matches_torch_grid_sample_on_gpu():
    """torch's own GPU grid_sample (an independent implementation) agrees in f32."""
    import torch.nn.functional as F

    inputs, grid, grad = _case(23, 4, 3, 33, 41, 17, 5)
    for padding_mode in ("zeros", "border"):
        a = [_t(inputs).requires_grad_(True), _t(grid).requires_grad_(True)]
        b = [_t(inputs).requires_grad_(True), _t(grid).requires_grad_(True)]
        o1 = hip.bilinear_grid_sample(a[0], a[1], padding_mode)
        o2 = F.grid_sample(b[0], b[1], mode="bilinear", padding_mode=padding_mode, align_corners=False)
        o1.backward(_t(grad))
        o2.backward(_t(grad))
        assert_close(_np(o1), _np(o2), 1e-5, f"{padding_mode} out")
        assert_close(_np(a[0].grad), _np(b[0].grad), 1e-4, f"{padding_mode} grad_input")
        assert_close(_np(a[1].grad), _np(b[1].grad), 1e-4, f"{padding_mode} grad_grid")


def test_no_points_gives_zero_input_gradient():
    inputs = _t(np.ones((2, 3, 5, 6), np.float32))
    grid = torch.zeros((2, 0, 2), device=_dev())
    gi, gg = hip.grid_sample_backward(inputs, grid, torch.zeros((2, 3, 0), device=_dev()), 0, 0, 0)
    torch.cuda.synchronize()
    assert gi.shape == (2, 3, 5, 6) and float(gi.abs().max()) == 0.0 and gg.shape == (2, 0, 2)


def test_mask_loss_shape_point_sample():
    """The segmentation loss's use (criterion.py:482-488): one-channel 112x112 mask logits, 784
    points per mask (H*W / 16), bilinear for the logits (with gradient) and nearest for labels."""
    rng = np.random.default_rng(24)
    logits = rng.standard_normal((64, 1, 112, 112)).astype(np.float32)
    labels = (rng.uniform(0, 1, (64, 1, 112, 112)) > 0.5).astype(np.float32)
    pts = rng.uniform(0, 1, (64, 784, 2)).astype(np.float32)
    g = rng.standard_normal((64, 1, 784)).astype(np.float32)
    tl = _t(logits).requires_grad_(True)
    out = hip.point_sample(tl, _t(pts))
    out.backward(_t(g))
    assert_close(_np(out), GS.point_sample(logits, pts), 1e-5, "logits")
    assert_close(_np(tl.grad), GS.point_sample_vjp(logits, pts, g)[0], 1e-4, "grad_logits")
    lab = hip.point_sample(_t(labels), _t(pts), mode="nearest")
    assert np.array_equal(_np(lab), GS.point_sample(labels, pts, "nearest").astype(np.float32))


@pytest.mark.parametrize("staged", [True, False], ids=["lds", "l2"])
def test_forward_paths_agree(tune, staged):
    """Planes that fit in LDS are staged there; MSDA_GS_NO_LDS forces the L2 gather path."""
    if not staged:
        tune({"MSDA_GS_NO_LDS": "1"})
    rng = np.random.default_rng(25)
    inputs = rng.standard_normal((20, 3, 40, 50)).astype(np.float32)
    pts = rng.uniform(-0.2, 1.2, (20, 700, 2)).astype(np.float32)
    for mode in ("bilinear", "nearest"):
        out = hip.point_sample(_t(inputs), _t(pts), mode)
        want = GS.point_sample(inputs, pts, mode)
        assert_close(_np(out), want, 1e-5, f"{mode} staged={staged}")
