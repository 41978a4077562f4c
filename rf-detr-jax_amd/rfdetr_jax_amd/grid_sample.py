"""``bilinear_grid_sample`` and ``point_sample`` on MI355X, backed by HIP through the C ABI.

Mirrors the reference interface:

* :func:`bilinear_grid_sample` — src/rfdetr_jax/models/ops.py:189-205: ``inputs [N, C, H, W]``,
  ``grid [N, Hg, Wg, 2]`` in ``[-1, 1]``, ``padding_mode`` ``"zeros"`` or ``"border"`` (anything
  else raises ``ValueError`` as ops.py:129-130), result ``[N, C, Hg, Wg]``;
* :func:`point_sample` — src/rfdetr_jax/models/heads/segmentation.py:146-170: points ``[N, P, 2]``
  or ``[N, Hg, Wg, 2]`` in ``[0, 1]``, ``mode`` ``"bilinear"`` (border padding) or ``"nearest"``
  (segmentation.py:173-186); any other mode raises ``ValueError`` as segmentation.py:161-162.

Both are differentiable in the feature map and in the positions (a ``torch.autograd.Function``
over ``msda_grid_sample_fwd`` / ``msda_grid_sample_bwd``). Tensors must be on a GPU: there is no
CPU path.
"""

from __future__ import annotations

import ctypes

import torch

from . import _native

_DTYPES = {torch.float32: _native.DTYPE_F32, torch.bfloat16: _native.DTYPE_BF16}


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _check(inputs, grid):
    if inputs.dim() != 4:
        raise ValueError(f"inputs must be [N, C, H, W], got {tuple(inputs.shape)}")
    if inputs.dtype not in _DTYPES:
        raise TypeError(f"inputs dtype {inputs.dtype} is not supported (float32 or bfloat16)")
    if grid.shape[-1] != 2 or grid.shape[0] != inputs.shape[0]:
        raise ValueError(f"grid must be [N, ..., 2] with N = {inputs.shape[0]}, got {tuple(grid.shape)}")
    for name, t in (("inputs", inputs), ("grid", grid)):
        if t.device.type != "cuda":
            raise RuntimeError(f"{name} is on {t.device}; the HIP kernels need GPU tensors (there is no CPU path)")
    if grid.device != inputs.device:
        raise RuntimeError("inputs and grid must be on the same device")


def grid_sample_forward(inputs, grid, grid_kind, padding_mode, sample_mode):
    """One forward launch: ``inputs [N, C, H, W]``, ``grid [N, P, 2]`` -> ``[N, C, P]``."""
    n, c, h, w = inputs.shape
    points = grid.shape[1]
    inputs = inputs.contiguous()
    grid = grid.to(torch.float32).contiguous()
    out = torch.empty((n, c, points), dtype=inputs.dtype, device=inputs.device)
    with torch.cuda.device(inputs.device):
        rc = _native.lib().msda_grid_sample_fwd(_ptr(inputs), _DTYPES[inputs.dtype], _ptr(grid), grid_kind, _ptr(out), n, c, h,
                                                w, points, padding_mode, sample_mode, _stream(inputs.device))
    _native.check(rc)
    return out


def grid_sample_backward(inputs, grid, grad_output, grid_kind, padding_mode, sample_mode, needs=(True, True)):
    """One backward launch: ``(grad_inputs, grad_grid)``; entries of ``needs`` that are false are
    ``None`` and not computed."""
    n, c, h, w = inputs.shape
    points = grid.shape[1]
    inputs = inputs.contiguous()
    grid = grid.to(torch.float32).contiguous()
    grad_output = grad_output.to(inputs.dtype).contiguous()
    g_in = torch.empty_like(inputs) if needs[0] else None
    g_grid = torch.empty(grid.shape, dtype=torch.float32, device=inputs.device) if needs[1] else None
    with torch.cuda.device(inputs.device):
        rc = _native.lib().msda_grid_sample_bwd(_ptr(inputs), _DTYPES[inputs.dtype], _ptr(grid), grid_kind, _ptr(grad_output),
                                                _ptr(g_in), _ptr(g_grid), n, c, h, w, points, padding_mode, sample_mode,
                                                _stream(inputs.device))
    _native.check(rc)
    return g_in, g_grid


class _GridSampleFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, inputs, grid, grid_kind, padding_mode, sample_mode):
        ctx.save_for_backward(inputs, grid)
        ctx.modes = (grid_kind, padding_mode, sample_mode)
        return grid_sample_forward(inputs, grid, grid_kind, padding_mode, sample_mode)

    @staticmethod
    def backward(ctx, grad_output):
        inputs, grid = ctx.saved_tensors
        g_in, g_grid = grid_sample_backward(inputs, grid, grad_output, *ctx.modes, needs=ctx.needs_input_grad[:2])
        if g_grid is not None and g_grid.dtype != grid.dtype:
            g_grid = g_grid.to(grid.dtype)
        return g_in, g_grid, None, None, None


def bilinear_grid_sample(inputs, grid, padding_mode: str = "zeros"):
    """Sample ``inputs`` at ``grid`` with ``F.grid_sample(..., align_corners=False)`` semantics (ops.py:189-205).

    Args:
        inputs: Feature map ``[N, C, H, W]``, float32 or bfloat16, on the GPU.
        grid: ``[N, Hg, Wg, 2]`` holding ``(x, y)`` in ``[-1, 1]``.
        padding_mode: ``"zeros"`` or ``"border"``.

    Returns:
        ``[N, C, Hg, Wg]`` in the inputs' dtype.

    Raises:
        ValueError: another ``padding_mode``, or inconsistent shapes.
    """
    if padding_mode not in _native.PADDING:
        raise ValueError(f"padding_mode must be 'zeros' or 'border', got {padding_mode!r}")
    if grid.dim() != 4:
        raise ValueError(f"grid must be [N, Hg, Wg, 2], got {tuple(grid.shape)}")
    _check(inputs, grid)
    n, gh, gw, _ = grid.shape
    out = _GridSampleFunction.apply(inputs, grid.reshape(n, gh * gw, 2), _native.GRID_COORDS, _native.PADDING[padding_mode],
                                    _native.SAMPLE_BILINEAR)
    return out.reshape(n, inputs.shape[1], gh, gw)


def point_sample(inputs, point_coords, mode: str = "bilinear"):
    """Sample ``inputs`` at ``[0, 1]``-normalized points (segmentation.py:146-170).

    Args:
        inputs: Feature map ``[N, C, H, W]``.
        point_coords: Points ``[N, P, 2]`` or ``[N, Hg, Wg, 2]`` in ``[0, 1]``.
        mode: ``"bilinear"`` (border padding) or ``"nearest"``.

    Returns:
        ``[N, C, P]`` or ``[N, C, Hg, Wg]``.

    Raises:
        ValueError: If a mode other than ``"bilinear"`` or ``"nearest"`` is requested.
    """
    if mode not in ("bilinear", "nearest"):
        raise ValueError(f"point_sample supports bilinear and nearest sampling, got {mode!r}")
    _check(inputs, point_coords)
    squeeze = point_coords.dim() == 3
    n = point_coords.shape[0]
    flat = point_coords.reshape(n, -1, 2)
    sample = _native.SAMPLE_NEAREST if mode == "nearest" else _native.SAMPLE_BILINEAR
    out = _GridSampleFunction.apply(inputs, flat, _native.GRID_UNIT_POINTS, _native.PADDING["border"], sample)
    return out if squeeze else out.reshape(n, inputs.shape[1], *point_coords.shape[1:3])
