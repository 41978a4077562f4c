"""MSDeformAttn's value projection with its epilogue fused, and the module that uses it.

* :func:`value_proj_rows` — ``value_proj`` (``Linear``, src/rfdetr_jax/models/layers.py:258-280),
  the padding mask (src/rfdetr_jax/models/ops.py:377-379) and the head split (ops.py:405-407) in
  one MFMA kernel: ``[B, S, C_in] -> [B * H, S, D]``, differentiable in the input, weight and bias.
* :class:`MSDeformAttn` — the reference module (ops.py:326-411) with the same constructor
  arguments, parameter names and layouts (torch ``Linear``: ``weight [out, in]``, ``bias [out]``)
  and call signature. Its value path is :func:`value_proj_rows`, its sampling is
  :func:`rfdetr_jax_amd.ops.ms_deform_attn_fused` (locations and softmax inside the kernels); the
  offset, weight and output projections are plain GEMMs.

Tensors must be on a GPU: there is no CPU path.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _native
from .ops import ms_deform_attn_fused

_DTYPES = {torch.float32: _native.DTYPE_F32, torch.bfloat16: _native.DTYPE_BF16}


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _mask_u8(mask, batch, length):
    if mask is None:
        return None
    if tuple(mask.shape) != (batch, length):
        raise ValueError(f"padding mask must be [B, S] = {(batch, length)}, got {tuple(mask.shape)}")
    if mask.dtype == torch.bool:  # one byte per element holding 0 or 1: read in place, no copy
        return mask.contiguous().view(torch.uint8)
    return (mask != 0).to(torch.uint8).contiguous()


def value_proj_forward(x, weight, bias, n_heads, padding_mask=None):
    """One launch: ``x [B, S, K]`` -> ``[B * n_heads, S, N / n_heads]`` in ``x``'s dtype."""
    if x.dim() != 3:
        raise ValueError(f"input must be [B, S, C_in], got {tuple(x.shape)}")
    if x.dtype not in _DTYPES:
        raise TypeError(f"input dtype {x.dtype} is not supported (float32 or bfloat16)")
    b, s, k = x.shape
    n = weight.shape[0]
    if weight.shape[1] != k or n % n_heads:
        raise ValueError(f"weight must be [n_heads * head_dim, {k}], got {tuple(weight.shape)}")
    for name, t in (("input", x), ("weight", weight)):
        if t.device.type != "cuda":
            raise RuntimeError(f"{name} is on {t.device}; the HIP kernels need GPU tensors (there is no CPU path)")
    d = n // n_heads
    x = x.contiguous()
    w = weight.to(torch.float32).contiguous()
    bias = None if bias is None else bias.to(torch.float32).contiguous()
    mask = _mask_u8(padding_mask, b, s)
    out = torch.empty((b * n_heads, s, d), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        rc = _native.lib().msda_value_proj_fwd(_ptr(x), _DTYPES[x.dtype], _ptr(w), _ptr(bias), _ptr(mask), _ptr(out), b, s, k,
                                               n_heads, d, _stream(x.device))
    _native.check(rc)
    return out


def value_proj_backward(x, weight, n_heads, grad_value, padding_mask=None, needs=(True, True, True)):
    """``(grad_input, grad_weight, grad_bias)``; entries of ``needs`` that are false are ``None``."""
    b, s, k = x.shape
    n = weight.shape[0]
    d = n // n_heads
    x = x.contiguous()
    w = weight.to(torch.float32).contiguous()
    gv = grad_value.to(x.dtype).contiguous()
    mask = _mask_u8(padding_mask, b, s)
    gx = torch.empty_like(x) if needs[0] else None
    gw = torch.empty((n, k), dtype=torch.float32, device=x.device) if needs[1] else None
    gb = torch.empty((n,), dtype=torch.float32, device=x.device) if needs[2] else None
    lib = _native.lib()
    workspace, ws = None, 0
    if gw is not None or gb is not None:
        ws = lib.msda_value_proj_bwd_workspace_size(b, s, k, n_heads, d)
        if ws < 0:
            _native.check(int(ws))
        workspace = torch.empty((max(1, ws // 16), 4), dtype=torch.int32, device=x.device)
    with torch.cuda.device(x.device):
        rc = lib.msda_value_proj_bwd(_ptr(x), _DTYPES[x.dtype], _ptr(w), _ptr(mask), _ptr(gv), _ptr(gx), _ptr(gw), _ptr(gb), b, s, k,
                                     n_heads, d, _ptr(workspace), ws, _stream(x.device))
    _native.check(rc)
    return gx, gw, gb


class _ValueProjFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, n_heads, padding_mask):
        ctx.save_for_backward(x, weight, padding_mask)
        ctx.n_heads = n_heads
        ctx.has_bias = bias is not None
        return value_proj_forward(x, weight, bias, n_heads, padding_mask)

    @staticmethod
    def backward(ctx, grad_value):
        x, weight, mask = ctx.saved_tensors
        needs = (ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.has_bias and ctx.needs_input_grad[2])
        gx, gw, gb = value_proj_backward(x, weight, ctx.n_heads, grad_value, mask, needs)
        if gw is not None and gw.dtype != weight.dtype:
            gw = gw.to(weight.dtype)
        return gx, gw, gb, None, None


def value_proj_rows(x, weight, bias, n_heads, padding_mask=None):
    """``where(padding_mask, 0, x @ weight.T + bias)`` split into heads: ``[B * n_heads, S, D]``.

    Args:
        x: ``[B, S, C_in]`` float32 or bfloat16 (``input_flatten``, ops.py:376).
        weight: ``[n_heads * D, C_in]`` (torch ``Linear`` layout).
        bias: ``[n_heads * D]`` or ``None``.
        n_heads: number of heads.
        padding_mask: ``[B, S]`` bool, ``True`` on padded positions, or ``None``.
    """
    return _ValueProjFunction.apply(x, weight, bias, n_heads, padding_mask)


class MSDeformAttn(torch.nn.Module):
    """Multi-scale deformable attention (src/rfdetr_jax/models/ops.py:326-411) on MI355X.

    Same constructor arguments and call as the reference; the parameters carry the reference's names
    (``sampling_offsets``, ``attention_weights``, ``value_proj``, ``output_proj``) and torch
    ``Linear`` layouts, so a checkpoint's arrays load unchanged.
    """

    def __init__(self, d_model: int = 256, n_levels: int = 4, n_heads: int = 8, n_points: int = 4, sampler: str = "hip"):
        super().__init__()
        if d_model % n_heads:
            raise ValueError(f"d_model ({d_model}) must be divisible by n_heads ({n_heads})")
        self.d_model, self.n_levels, self.n_heads, self.n_points = d_model, n_levels, n_heads, n_points
        self.sampler = sampler
        self.sampling_offsets = torch.nn.Linear(d_model, n_heads * n_levels * n_points * 2)
        self.attention_weights = torch.nn.Linear(d_model, n_heads * n_levels * n_points)
        self.value_proj = torch.nn.Linear(d_model, d_model)
        self.output_proj = torch.nn.Linear(d_model, d_model)
        self.reset_parameters()

    def reset_parameters(self):
        """The reference's initialisation of this module (training/trainer.py:124-144): Xavier-uniform
        weights, then zero offset weights with the grid-shaped bias of ``sampling_offsets_bias_init``
        (ops.py:317-323), zero attention weights and bias, zero value and output biases."""
        with torch.no_grad():
            self.sampling_offsets.weight.zero_()
            thetas = torch.arange(self.n_heads, dtype=torch.float32) * (2.0 * math.pi / self.n_heads)
            grid = torch.stack([thetas.cos(), thetas.sin()], -1)
            grid = grid / grid.abs().max(-1, keepdim=True)[0]
            grid = grid.view(self.n_heads, 1, 1, 2).repeat(1, self.n_levels, self.n_points, 1)
            grid = grid * torch.arange(1, self.n_points + 1, dtype=torch.float32).view(1, 1, -1, 1)
            self.sampling_offsets.bias.copy_(grid.reshape(-1))
            self.attention_weights.weight.zero_()
            self.attention_weights.bias.zero_()
            for lin in (self.value_proj, self.output_proj):
                torch.nn.init.xavier_uniform_(lin.weight)
                lin.bias.zero_()

    def forward(self, query, reference_points, input_flatten, spatial_shapes, input_padding_mask=None):
        """``query [B, Lq, C]``, ``reference_points [B, Lq, n_levels, 2 | 4]``, ``input_flatten
        [B, S, C]``, ``spatial_shapes`` ``(H, W)`` pairs, ``input_padding_mask [B, S]`` (``True`` =
        padded) -> ``[B, Lq, C]``.

        Raises:
            ValueError: a ``reference_points`` trailing dimension other than 2 or 4 (ops.py:400).
        """
        if reference_points.shape[-1] not in (2, 4):
            raise ValueError(f"Last dim of reference_points must be 2 or 4, but get {reference_points.shape[-1]}.")
        batch, len_query, _ = query.shape
        value = value_proj_rows(input_flatten, self.value_proj.weight, self.value_proj.bias, self.n_heads, input_padding_mask)
        logits = self.attention_weights(query).view(batch, len_query, self.n_heads, self.n_levels * self.n_points)
        offsets = self.sampling_offsets(query).view(batch, len_query, self.n_heads, self.n_levels, self.n_points, 2)
        out = ms_deform_attn_fused(value, spatial_shapes, reference_points, offsets, logits)
        return self.output_proj(out.to(query.dtype))
