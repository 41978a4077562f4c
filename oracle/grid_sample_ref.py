"""CPU oracle for ``bilinear_grid_sample`` / ``point_sample`` — TEST INFRASTRUCTURE ONLY.

Nothing in the product path imports this module. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg may use it, and only as the checker.

It restates, in NumPy:

* ``_sample_rows`` with ``padding_mode`` (src/rfdetr_jax/models/ops.py:64-134): coordinates
  ``((g + 1) * size - 1) / 2`` in f32 (:83-84), floor and fractions (:85-91), in-bounds masks
  (:98-101), clipped corners in the order (x0,y0),(x1,y0),(x0,y1),(x1,y1) (:103-118), weights
  ``wx*wy`` masked for ``"zeros"`` and unmasked for ``"border"`` (:123-132: with the corners
  clipped, unmasked weights replicate the edge pixel);
* ``bilinear_grid_sample`` (ops.py:189-205): ``inputs [N, C, H, W]``, ``grid [N, Hg, Wg, 2]`` ->
  ``[N, C, Hg, Wg]``;
* ``point_sample`` (models/heads/segmentation.py:146-170): points in ``[0, 1]``, ``grid = 2 p - 1``,
  border padding for ``"bilinear"``; ``_nearest_grid_sample`` (segmentation.py:173-186):
  ``round`` (half to even) then clip;
* the VJP of the bilinear sampler (grad of inputs by scatter-add, grad of the grid through the
  fractions; floor, masks and clipping contribute nothing), and of the nearest one (scatter-add
  with weight one; no grid gradient).

Precision: coordinates in f32 with one rounding per operation; everything after in float64.

Pinning (tests/test_grid_sample_oracle.py): the reference's known answers (tests/test_ops.py:22-43,
tests/test_segmentation.py:40-45, :107-115); torch ``F.grid_sample`` (bilinear and nearest; zeros
and border; align_corners=False) and torch float64 autograd through it; the upstream NumPy
formula of tests/test_criterion.py:214-224 for border sampling; planted mistakes.
"""

from __future__ import annotations

import numpy as np

__all__ = ["sample_rows", "bilinear_grid_sample", "point_sample", "grid_sample_vjp", "point_sample_vjp"]


def _coords(grid, height, width):
    f32 = np.float32
    g = np.asarray(grid, f32)
    ix = ((g[..., 0] + f32(1)) * f32(width) - f32(1)) / f32(2)
    iy = ((g[..., 1] + f32(1)) * f32(height) - f32(1)) / f32(2)
    return ix, iy


def _to_int(v):
    v = np.where(np.isnan(v), 0.0, v)
    return np.clip(v, -(2**31), 2**31 - 1).astype(np.int64)


def _bilinear_terms(grid, height, width, padding_mode):
    """Clipped flat corner indices ``[..., 4]``, weights ``[..., 4]`` (f64), masks, fx, fy."""
    if padding_mode not in ("zeros", "border"):
        raise ValueError(f"padding_mode must be 'zeros' or 'border', got {padding_mode!r}")
    ix, iy = _coords(grid, height, width)
    ix0, iy0 = np.floor(ix), np.floor(iy)
    fx = (ix - ix0).astype(np.float64)
    fy = (iy - iy0).astype(np.float64)
    x0, y0 = _to_int(ix0), _to_int(iy0)
    x1, y1 = x0 + 1, y0 + 1
    mx0, mx1 = (x0 >= 0) & (x0 < width), (x1 >= 0) & (x1 < width)
    my0, my1 = (y0 >= 0) & (y0 < height), (y1 >= 0) & (y1 < height)
    cx0, cx1 = np.clip(x0, 0, width - 1), np.clip(x1, 0, width - 1)
    cy0, cy1 = np.clip(y0, 0, height - 1), np.clip(y1, 0, height - 1)
    idx = np.stack([cy0 * width + cx0, cy0 * width + cx1, cy1 * width + cx0, cy1 * width + cx1], -1)
    m = np.stack([mx0 & my0, mx1 & my0, mx0 & my1, mx1 & my1], -1).astype(np.float64)
    if padding_mode == "border":
        m = np.ones_like(m)
    w = np.stack([(1 - fx) * (1 - fy), fx * (1 - fy), (1 - fx) * fy, fx * fy], -1) * m
    return idx, w, m, fx, fy


def sample_rows(values, grid, height, width, padding_mode="zeros"):
    """``values [N, H*W, C]``, ``grid [N, L, 2]`` in [-1, 1] -> ``[N, L, C]`` float64 (ops.py:64-134)."""
    v = np.asarray(values, np.float64)
    idx, w, _, _, _ = _bilinear_terms(grid, height, width, padding_mode)
    n, l, _ = idx.shape
    taken = np.take_along_axis(v, idx.reshape(n, l * 4)[..., None], axis=1).reshape(n, l, 4, v.shape[-1])
    return np.einsum("nlc,nlcd->nld", w, taken)


def bilinear_grid_sample(inputs, grid, padding_mode="zeros"):
    """``inputs [N, C, H, W]``, ``grid [N, Hg, Wg, 2]`` -> ``[N, C, Hg, Wg]`` float64 (ops.py:189-205)."""
    n, c, h, w = inputs.shape
    gh, gw = grid.shape[1], grid.shape[2]
    rows = np.asarray(inputs).reshape(n, c, h * w).swapaxes(1, 2)
    out = sample_rows(rows, np.asarray(grid).reshape(n, gh * gw, 2), h, w, padding_mode)
    return out.reshape(n, gh, gw, c).transpose(0, 3, 1, 2)


def _nearest_index(grid, height, width):
    ix, iy = _coords(grid, height, width)
    xi = np.clip(_to_int(np.round(ix)), 0, width - 1)  # numpy rounds half to even, as jnp.round
    yi = np.clip(_to_int(np.round(iy)), 0, height - 1)
    return yi * width + xi


def point_sample(inputs, point_coords, mode="bilinear"):
    """segmentation.py:146-170: ``inputs [N, C, H, W]``, points ``[N, P, 2]`` or ``[N, Hg, Wg, 2]``."""
    if mode not in ("bilinear", "nearest"):
        raise ValueError(f"point_sample supports bilinear and nearest sampling, got {mode!r}")
    pts = np.asarray(point_coords, np.float32)
    squeeze = pts.ndim == 3
    if squeeze:
        pts = pts[:, :, None, :]
    grid = np.float32(2.0) * pts - np.float32(1.0)
    if mode == "nearest":
        n, c, h, w = inputs.shape
        gh, gw = grid.shape[1], grid.shape[2]
        rows = np.asarray(inputs, np.float64).reshape(n, c, h * w).swapaxes(1, 2)
        index = _nearest_index(grid, h, w).reshape(n, gh * gw, 1)
        out = np.take_along_axis(rows, index, axis=1).reshape(n, gh, gw, c).transpose(0, 3, 1, 2)
    else:
        out = bilinear_grid_sample(inputs, grid, "border")
    return out[..., 0] if squeeze else out


def grid_sample_vjp(inputs, grid, grad_output, padding_mode="zeros"):
    """VJP of :func:`bilinear_grid_sample`: ``(grad_inputs [N,C,H,W], grad_grid [N,Hg,Wg,2])`` float64.

    ``d ix / d g = W / 2`` (ops.py:83: ``ix = ((g + 1) W - 1) / 2``)."""
    n, c, h, w = inputs.shape
    gh, gw = grid.shape[1], grid.shape[2]
    l = gh * gw
    g2 = np.asarray(grid).reshape(n, l, 2)
    idx, wt, m, fx, fy = _bilinear_terms(g2, h, w, padding_mode)
    rows = np.asarray(inputs, np.float64).reshape(n, c, h * w)
    go = np.asarray(grad_output, np.float64).reshape(n, c, l)
    grad_in = np.zeros((n, c, h * w))
    for k in range(4):
        for b in range(n):
            for ch in range(c):
                np.add.at(grad_in[b, ch], idx[b, :, k], wt[b, :, k] * go[b, ch])
    corner = np.stack([np.take_along_axis(rows, np.broadcast_to(idx[:, None, :, k], (n, c, l)), axis=2) for k in range(4)], -1)
    mv = corner * m[:, None]  # [N, C, L, 4]
    d_ix = (1 - fy)[:, None] * (mv[..., 1] - mv[..., 0]) + fy[:, None] * (mv[..., 3] - mv[..., 2])
    d_iy = (1 - fx)[:, None] * (mv[..., 2] - mv[..., 0]) + fx[:, None] * (mv[..., 3] - mv[..., 1])
    ggx = (go * d_ix).sum(1) * (w / 2.0)
    ggy = (go * d_iy).sum(1) * (h / 2.0)
    grad_grid = np.stack([ggx, ggy], -1).reshape(n, gh, gw, 2)
    return grad_in.reshape(n, c, h, w), grad_grid


def point_sample_vjp(inputs, point_coords, grad_output, mode="bilinear"):
    """VJP of :func:`point_sample`: ``(grad_inputs, grad_point_coords)`` float64. The points'
    gradient is twice the grid's (``grid = 2 p - 1``); nearest sampling has none (zeros)."""
    pts = np.asarray(point_coords, np.float32)
    squeeze = pts.ndim == 3
    if squeeze:
        pts = pts[:, :, None, :]
        grad_output = np.asarray(grad_output)[..., None]
    grid = np.float32(2.0) * pts - np.float32(1.0)
    n, c, h, w = inputs.shape
    if mode == "nearest":
        gh, gw = grid.shape[1], grid.shape[2]
        index = _nearest_index(grid, h, w).reshape(n, gh * gw)
        go = np.asarray(grad_output, np.float64).reshape(n, c, gh * gw)
        grad_in = np.zeros((n, c, h * w))
        for b in range(n):
            for ch in range(c):
                np.add.at(grad_in[b, ch], index[b], go[b, ch])
        gp = np.zeros(pts.shape)
        grad_in = grad_in.reshape(n, c, h, w)
    else:
        grad_in, gg = grid_sample_vjp(inputs, grid, grad_output, "border")
        gp = 2.0 * gg
    return grad_in, (gp[:, :, 0] if squeeze else gp)
