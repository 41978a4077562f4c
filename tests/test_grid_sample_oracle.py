"""Pin the grid-sample oracle (oracle/grid_sample_ref.py) before trusting it.

Checks, none of which retypes the oracle's formulas:
* the reference's known answers: tests/test_ops.py:22-43 (pixel centres, zero padding, linear
  interpolation), tests/test_segmentation.py:40-45 (nearest at a pixel centre) and :107-115
  (border padding at the corner, far outside, and the centre);
* torch ``F.grid_sample`` (align_corners=False) in float64: bilinear with zeros and border padding,
  nearest with border padding; torch autograd through it for the input and grid gradients;
* the upstream NumPy border sampler written out in the reference's tests
  (tests/test_criterion.py:214-224), which clips the coordinate instead of the corners.
Planted mistakes (border weights masked like zeros, a half-pixel shift, x/y swapped) fail them.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import grid_sample_ref as GS
from tests._util import assert_close


def test_kat_pixel_centres():
    values = np.array([[[[1.0, 2.0], [3.0, 4.0]]]], np.float32)
    grid = np.array([[[[-0.5, -0.5], [0.5, 0.5]]]], np.float32)
    out = GS.bilinear_grid_sample(values, grid)[0, 0, 0]
    assert out[0] == pytest.approx(1.0) and out[1] == pytest.approx(4.0)


def test_kat_zero_pad():
    assert GS.bilinear_grid_sample(np.ones((1, 1, 2, 2), np.float32), np.full((1, 1, 1, 2), 5.0, np.float32))[0, 0, 0, 0] == 0.0


def test_kat_linear():
    out = GS.bilinear_grid_sample(np.array([[[[0.0, 4.0]]]], np.float32), np.zeros((1, 1, 1, 2), np.float32))
    assert out[0, 0, 0, 0] == pytest.approx(2.0)


def test_kat_nearest_pixel():
    values = np.array([[[[0.0, 1.0], [2.0, 3.0]]]], np.float32)
    assert GS.point_sample(values, np.array([[[0.75, 0.75]]], np.float32), "nearest")[0, 0, 0] == 3.0


def test_kat_border_padding():
    values = np.array([[[[2.0, 4.0], [6.0, 8.0]]]], np.float32)
    assert GS.point_sample(values, np.array([[[0.0, 0.0]]], np.float32))[0, 0, 0] == 2.0
    assert GS.point_sample(values, np.array([[[1.0, 1.0]]], np.float32))[0, 0, 0] == 8.0
    assert GS.point_sample(values, np.array([[[0.5, 0.5]]], np.float32))[0, 0, 0] == 5.0


def test_point_sample_rejects_other_modes():
    with pytest.raises(ValueError, match="bilinear and nearest"):
        GS.point_sample(np.zeros((1, 1, 2, 2)), np.zeros((1, 1, 2)), mode="bicubic")
    with pytest.raises(ValueError, match="padding_mode"):
        GS.bilinear_grid_sample(np.zeros((1, 1, 2, 2)), np.zeros((1, 1, 1, 2)), "reflection")


def _case(seed, n=3, c=4, h=7, w=9, gh=5, gw=6, lo=-1.4, hi=1.4):
    rng = np.random.default_rng(seed)
    inputs = rng.standard_normal((n, c, h, w)).astype(np.float32)
    grid = rng.uniform(lo, hi, (n, gh, gw, 2)).astype(np.float32)
    grad = rng.standard_normal((n, c, gh, gw)).astype(np.float32)
    return inputs, grid, grad


def _torch(inputs, grid, grad, mode, padding_mode):
    import torch
    import torch.nn.functional as F

    ti = torch.tensor(inputs.astype(np.float64), requires_grad=True)
    tg = torch.tensor(grid.astype(np.float64), requires_grad=True)
    out = F.grid_sample(ti, tg, mode=mode, padding_mode=padding_mode, align_corners=False)
    out.backward(torch.tensor(grad.astype(np.float64)))
    return out.detach().numpy(), ti.grad.numpy(), tg.grad.numpy()


@pytest.mark.parametrize("padding_mode", ["zeros", "border"])
@pytest.mark.parametrize("seed", [0, 1])
def test_bilinear_matches_torch_grid_sample(padding_mode, seed):
    inputs, grid, grad = _case(seed)
    t_out, t_gi, t_gg = _torch(inputs, grid, grad, "bilinear", padding_mode)
    assert_close(GS.bilinear_grid_sample(inputs, grid, padding_mode), t_out, 1e-6, "out")
    gi, gg = GS.grid_sample_vjp(inputs, grid, grad, padding_mode)
    assert_close(gi, t_gi, 1e-6, "grad_input")
    # torch's border mode clips the coordinate (gradient zero outside the centres); the reference
    # clips the corners, which gives the same zero gradient there (both corners are the edge pixel)
    assert_close(gg, t_gg, 1e-5, "grad_grid")


def test_nearest_matches_torch_grid_sample():
    inputs, grid, grad = _case(3)
    # torch rounds half to even in nearest mode, like jnp.round; keep away from exact halves
    t_out, t_gi, _ = _torch(inputs, grid, grad, "nearest", "border")
    pts = (grid + np.float32(1.0)) / np.float32(2.0)
    out = GS.point_sample(inputs, pts, "nearest")
    # the oracle rebuilds grid = 2 p - 1 from the points, which can move a coordinate by an ulp
    assert np.mean(np.isclose(out, t_out)) > 0.99
    gi, gp = GS.point_sample_vjp(inputs, pts, grad, "nearest")
    assert (gp == 0).all()
    assert np.isclose(gi.sum(), t_gi.sum())


def test_border_matches_upstream_numpy_formula():
    """tests/test_criterion.py:214-224 clips the pixel coordinate to [0, size-1] before the floor."""
    rng = np.random.default_rng(4)
    image = rng.standard_normal((6, 9)).astype(np.float32)
    pts = rng.uniform(-0.3, 1.3, (50, 2)).astype(np.float32)
    height, width = image.shape
    x = np.clip(pts[:, 0].astype(np.float64) * width - 0.5, 0, width - 1)
    y = np.clip(pts[:, 1].astype(np.float64) * height - 0.5, 0, height - 1)
    x0, y0 = np.floor(x).astype(int), np.floor(y).astype(int)
    x1, y1 = np.minimum(x0 + 1, width - 1), np.minimum(y0 + 1, height - 1)
    wx, wy = x - x0, y - y0
    want = (image[y0, x0] * (1 - wx) * (1 - wy) + image[y0, x1] * wx * (1 - wy)
            + image[y1, x0] * (1 - wx) * wy + image[y1, x1] * wx * wy)
    got = GS.point_sample(image[None, None], pts[None])[0, 0]
    assert_close(got, want, 1e-5, "border")


def test_point_sample_vjp_matches_torch():
    import torch
    import torch.nn.functional as F

    inputs, grid, grad = _case(5, gh=7, gw=1)
    pts = ((grid[:, :, 0, :] + 1) / 2).astype(np.float32)  # [N, P, 2]
    g = grad[..., 0]
    ti = torch.tensor(inputs.astype(np.float64), requires_grad=True)
    tp = torch.tensor(pts.astype(np.float64), requires_grad=True)
    out = F.grid_sample(ti, (2 * tp - 1)[:, :, None, :], mode="bilinear", padding_mode="border", align_corners=False)[..., 0]
    out.backward(torch.tensor(g.astype(np.float64)))
    assert_close(GS.point_sample(inputs, pts), out.detach().numpy(), 1e-6, "out")
    gi, gp = GS.point_sample_vjp(inputs, pts, g)
    assert_close(gi, ti.grad.numpy(), 1e-6, "grad_input")
    assert_close(gp, tp.grad.numpy(), 1e-5, "grad_points")


# --------------------------------------------------------------------------------------------
# planted mistakes


def test_planted_mistakes_are_caught(monkeypatch):
    values = np.array([[[[2.0, 4.0], [6.0, 8.0]]]], np.float32)
    corner = np.array([[[0.0, 0.0]]], np.float32)
    real = GS._bilinear_terms

    def masked_border(grid, height, width, padding_mode):
        return real(grid, height, width, "zeros")

    monkeypatch.setattr(GS, "_bilinear_terms", masked_border)
    assert GS.point_sample(values, corner)[0, 0, 0] != 2.0  # border weights masked: 0.5
    monkeypatch.setattr(GS, "_bilinear_terms", real)

    real_coords = GS._coords

    def shifted(grid, height, width):
        ix, iy = real_coords(grid, height, width)
        return ix + np.float32(0.5), iy + np.float32(0.5)

    monkeypatch.setattr(GS, "_coords", shifted)
    out = GS.bilinear_grid_sample(np.array([[[[1.0, 2.0], [3.0, 4.0]]]], np.float32),
                                  np.array([[[[-0.5, -0.5]]]], np.float32))
    assert out[0, 0, 0, 0] != pytest.approx(1.0)
    monkeypatch.setattr(GS, "_coords", real_coords)

    def swapped(grid, height, width):
        ix, iy = real_coords(grid, height, width)
        return iy, ix

    monkeypatch.setattr(GS, "_coords", swapped)
    inputs, grid, grad = _case(6)
    t_out = _torch(inputs, grid, grad, "bilinear", "zeros")[0]
    assert np.abs(GS.bilinear_grid_sample(inputs, grid) - t_out).max() > 1e-3
