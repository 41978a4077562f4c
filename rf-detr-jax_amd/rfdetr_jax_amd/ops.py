"""Multi-scale deformable attention on MI355X: the reference's entry points, backed by HIP.

Mirrors ``rfdetr_jax.models.ops`` (src/rfdetr_jax/models/ops.py):

* :func:`ms_deform_attn_core_rows` — ops.py:208-292, same arguments (``value [B*H, S, D]``,
  ``spatial_shapes`` as Python ints, ``sampling_locations [B, Q, H, L, P, 2]``,
  ``attention_weights [B, Q, H, L*P]``, ``sampler``), same result ``[B, Q, H*D]`` with dtype
  ``result_type(value, attention_weights)`` (ops.py:260), same ``ValueError`` for an unknown
  sampler (ops.py:235-238). Every sampler name the reference accepts selects the HIP kernels, with
  that sampler's rounding points in the forward: on a bf16 value map ``"gather"``,
  ``"gather-f32"``, ``"matmul"`` and ``"auto"`` round where ops.py:64-186 rounds, and ``"pallas"``
  forms pixel coordinates as deform_pallas.py:223-224 does (include/msda.h, msda_fwd_sampler);
  ``"hip"`` (the default) interpolates in f32 throughout. The backward is the f32 VJP at each
  sampler's coordinates (msda_bwd_sampler).
* :func:`ms_deform_attn_core` — ops.py:295-314, ``value [B, H, D, S]``.
* :func:`ms_deform_attn` — the ``(value, spatial_shapes, level_start_index, sampling_locations,
  attention_weights)`` signature of the upstream Deformable-DETR op; ``level_start_index`` is
  checked against the prefix sums of ``spatial_shapes`` (ops.py:265-267 derives them).

Differentiation is a ``torch.autograd.Function`` whose forward and backward each enqueue one
kernel through the C ABI — the counterpart of the reference's ``jax.custom_vjp`` around its fused
sampler (deform_pallas.py:132-178). Tensors must be on a GPU: there is no CPU path.
"""

from __future__ import annotations

import ctypes

import torch

from . import _native

#: Sampler names accepted by ms_deform_attn_core_rows (the reference's five, ops.py:235, + "hip"),
#: with their codes in the C ABI (enum msda_sampler, include/msda.h).
SAMPLER_CODES = {"hip": 0, "gather": 1, "gather-f32": 2, "matmul": 3, "auto": 4, "pallas": 5}
SAMPLERS = tuple(SAMPLER_CODES)

_VALUE_DTYPES = {torch.float32: _native.DTYPE_F32, torch.bfloat16: _native.DTYPE_BF16}


def _as_shapes(spatial_shapes) -> tuple[tuple[int, int], ...]:
    """Normalise ``spatial_shapes`` to a tuple of ``(H, W)`` Python ints."""
    if isinstance(spatial_shapes, torch.Tensor):
        spatial_shapes = spatial_shapes.detach().cpu().tolist()
    shapes = tuple((int(h), int(w)) for h, w in spatial_shapes)
    if not shapes:
        raise ValueError("spatial_shapes must name at least one level")
    return shapes


def _prefix_sums(shapes) -> list[int]:
    offsets = [0]
    for h, w in shapes:
        offsets.append(offsets[-1] + h * w)
    return offsets


def _check_level_start_index(level_start_index, shapes) -> None:
    if level_start_index is None:
        return
    if isinstance(level_start_index, torch.Tensor):
        level_start_index = level_start_index.detach().cpu().tolist()
    got = [int(v) for v in level_start_index]
    want = _prefix_sums(shapes)[:-1]
    if got != want:
        raise ValueError(f"level_start_index {got} does not match the prefix sums of spatial_shapes {want}")


def _shape_arrays(shapes):
    flat = [v for hw in shapes for v in hw]
    arr = (ctypes.c_int32 * len(flat))(*flat)
    starts = (ctypes.c_int32 * len(shapes))(*_prefix_sums(shapes)[:-1])
    return arr, starts


def _check_inputs(value, shapes, sampling_locations, attention_weights):
    if value.dim() != 3:
        raise ValueError(f"value must be [B*n_heads, sum(H*W), head_dim], got shape {tuple(value.shape)}")
    if sampling_locations.dim() != 6 or sampling_locations.shape[-1] != 2:
        raise ValueError(
            f"sampling_locations must be [B, Lq, n_heads, n_levels, n_points, 2], got {tuple(sampling_locations.shape)}"
        )
    batch, len_query, n_heads, n_levels, n_points, _ = sampling_locations.shape
    if n_levels != len(shapes):
        raise ValueError(f"sampling_locations has {n_levels} levels but spatial_shapes has {len(shapes)}")
    if tuple(attention_weights.shape) != (batch, len_query, n_heads, n_levels * n_points):
        raise ValueError(
            f"attention_weights must be {(batch, len_query, n_heads, n_levels * n_points)}, got {tuple(attention_weights.shape)}"
        )
    if value.shape[0] != batch * n_heads:
        raise ValueError(f"value has {value.shape[0]} rows of slices, expected batch*n_heads = {batch * n_heads}")
    if value.shape[1] != _prefix_sums(shapes)[-1]:
        raise ValueError(f"value length {value.shape[1]} != sum(H*W) = {_prefix_sums(shapes)[-1]}")
    if value.dtype not in _VALUE_DTYPES:
        raise TypeError(f"value dtype {value.dtype} is not supported (float32 or bfloat16)")
    for name, t in (("value", value), ("sampling_locations", sampling_locations), ("attention_weights", attention_weights)):
        if t.device.type != "cuda":
            raise RuntimeError(f"{name} is on {t.device}; the HIP kernels need GPU tensors (there is no CPU path)")
    if sampling_locations.device != value.device or attention_weights.device != value.device:
        raise RuntimeError("value, sampling_locations and attention_weights must be on the same device")
    return batch, len_query, n_heads, n_levels, n_points, value.shape[2]


def _out_dtype(value, attention_weights):
    dt = torch.result_type(value, attention_weights)
    if dt not in (torch.float32, torch.bfloat16):
        dt = torch.float32
    return dt


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _sampler_code(sampler: str) -> int:
    if sampler not in SAMPLER_CODES:
        raise ValueError(
            f"unknown sampler {sampler!r}; expected 'gather', 'gather-f32', 'matmul', 'auto', 'pallas' or 'hip'"
        )
    return SAMPLER_CODES[sampler]


def ms_deform_attn_forward(value, spatial_shapes, sampling_locations, attention_weights, level_start_index=None,
                           out_dtype=None, sampler: str = "hip"):
    """One forward launch (no autograd): returns ``[B, Q, H*D]``.

    ``sampling_locations`` / ``attention_weights`` of another float dtype are converted to f32
    first (the reference computes positions in at least f32, ops.py:80, :270). ``sampler`` picks the
    rounding points of one of the reference's samplers (msda_fwd_sampler).
    """
    code = _sampler_code(sampler)
    shapes = _as_shapes(spatial_shapes)
    _check_level_start_index(level_start_index, shapes)
    batch, len_query, n_heads, n_levels, n_points, head_dim = _check_inputs(
        value, shapes, sampling_locations, attention_weights
    )
    out_dtype = out_dtype or _out_dtype(value, attention_weights)
    value = value.contiguous()
    loc = sampling_locations.to(torch.float32).contiguous()
    attn = attention_weights.to(torch.float32).contiguous()
    out = torch.empty((batch, len_query, n_heads * head_dim), dtype=out_dtype, device=value.device)
    arr, starts = _shape_arrays(shapes)
    lib = _native.lib()
    dims = (batch, n_heads, head_dim, len_query, n_levels, n_points, arr, starts, value.shape[1])
    with torch.cuda.device(value.device):
        head = (_ptr(value), _VALUE_DTYPES[value.dtype], _ptr(loc), _ptr(attn), _ptr(out), _VALUE_DTYPES[out_dtype])
        if code == 0:
            rc = lib.msda_fwd(*head, *dims, _stream(value.device))
        else:
            rc = lib.msda_fwd_sampler(*head, code, *dims, _stream(value.device))
    _native.check(rc)
    return out


def ms_deform_attn_backward(value, spatial_shapes, sampling_locations, attention_weights, grad_output,
                            level_start_index=None, needs=(True, True, True), sampler: str = "hip"):
    """One backward launch: returns ``(grad_value, grad_sampling_locations, grad_attention_weights)``.

    ``grad_value`` has the value dtype (f32 accumulation, one rounding); the other two are f32.
    Entries of ``needs`` that are false come back as ``None`` and are not computed. ``sampler``
    picks the pixel coordinates of one of the reference's samplers (msda_bwd_sampler).
    """
    code = _sampler_code(sampler)
    shapes = _as_shapes(spatial_shapes)
    _check_level_start_index(level_start_index, shapes)
    batch, len_query, n_heads, n_levels, n_points, head_dim = _check_inputs(
        value, shapes, sampling_locations, attention_weights
    )
    if tuple(grad_output.shape) != (batch, len_query, n_heads * head_dim):
        raise ValueError(f"grad_output must be {(batch, len_query, n_heads * head_dim)}, got {tuple(grad_output.shape)}")
    value = value.contiguous()
    loc = sampling_locations.to(torch.float32).contiguous()
    attn = attention_weights.to(torch.float32).contiguous()
    if grad_output.dtype not in _VALUE_DTYPES:
        grad_output = grad_output.to(torch.float32)
    grad_output = grad_output.contiguous()
    dev = value.device
    grad_value = torch.empty_like(value) if needs[0] else None
    grad_loc = torch.empty(loc.shape, dtype=torch.float32, device=dev) if needs[1] else None
    grad_attn = torch.empty(attn.shape, dtype=torch.float32, device=dev) if needs[2] else None
    arr, starts = _shape_arrays(shapes)
    lib = _native.lib()
    dims = (batch, n_heads, head_dim, len_query, n_levels, n_points, arr, starts, value.shape[1])
    workspace, ws_bytes = None, 0
    if grad_value is not None:
        ws_bytes = lib.msda_bwd_workspace_size(*dims)
        if ws_bytes < 0:
            _native.check(int(ws_bytes))
        # the query blocks' partial grad_value sums (f32); torch's caching allocator serves it
        workspace = torch.empty((max(1, ws_bytes // 16), 4), dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        head = (_ptr(value), _VALUE_DTYPES[value.dtype], _ptr(loc), _ptr(attn), _ptr(grad_output),
                _VALUE_DTYPES[grad_output.dtype], _ptr(grad_value), _ptr(grad_loc), _ptr(grad_attn))
        if code == 0:
            rc = lib.msda_bwd(*head, *dims, _ptr(workspace), ws_bytes, _stream(dev))
        else:
            rc = lib.msda_bwd_sampler(*head, code, *dims, _ptr(workspace), ws_bytes, _stream(dev))
    _native.check(rc)
    return grad_value, grad_loc, grad_attn


class _MSDeformAttnFunction(torch.autograd.Function):
    """custom-VJP pair: forward = msda_fwd, backward = msda_bwd (deform_pallas.py:132-178 contract)."""

    @staticmethod
    def forward(ctx, value, sampling_locations, attention_weights, shapes, sampler="hip"):
        out = ms_deform_attn_forward(value, shapes, sampling_locations, attention_weights, sampler=sampler)
        ctx.save_for_backward(value, sampling_locations, attention_weights)
        ctx.shapes = shapes
        ctx.sampler = sampler
        ctx.out_dtype = out.dtype
        return out

    @staticmethod
    def backward(ctx, grad_output):
        value, loc, attn = ctx.saved_tensors
        needs = ctx.needs_input_grad[:3]
        grad_output = grad_output.to(ctx.out_dtype)
        gv, gl, ga = ms_deform_attn_backward(value, ctx.shapes, loc, attn, grad_output, needs=needs, sampler=ctx.sampler)
        # Gradients come back in the input dtypes (deform_pallas.py:175).
        if gl is not None and gl.dtype != loc.dtype:
            gl = gl.to(loc.dtype)
        if ga is not None and ga.dtype != attn.dtype:
            ga = ga.to(attn.dtype)
        return gv, gl, ga, None, None


def ms_deform_attn_core_rows(value, spatial_shapes, sampling_locations, attention_weights, sampler: str = "hip"):
    """Sample and weight multi-scale features, channels last (ops.py:208-292).

    Args:
        value: ``[B * n_heads, sum(H*W), head_dim]``, float32 or bfloat16, on the GPU.
        spatial_shapes: per-level ``(H, W)`` pairs.
        sampling_locations: ``[B, Lq, n_heads, n_levels, n_points, 2]`` in ``[0, 1]`` (outside is
            zero-padded).
        attention_weights: ``[B, Lq, n_heads, n_levels * n_points]``.
        sampler: one of :data:`SAMPLERS`; all select the HIP kernels, with the named sampler's
            rounding points in the forward and its pixel coordinates in both directions.

    Returns:
        ``[B, Lq, n_heads * head_dim]`` with dtype ``result_type(value, attention_weights)``.

    Raises:
        ValueError: unknown ``sampler`` or inconsistent shapes.
    """
    _sampler_code(sampler)
    shapes = _as_shapes(spatial_shapes)
    return _MSDeformAttnFunction.apply(value, sampling_locations, attention_weights, shapes, sampler)


def ms_deform_attn(value, spatial_shapes, level_start_index, sampling_locations, attention_weights):
    """``ms_deform_attn(value, spatial_shapes, level_start_index, sampling_locations, attention_weights)``.

    ``value`` is in the rows layout ``[B * n_heads, sum(H*W), head_dim]`` the Flax module hands over
    (ops.py:405-410). ``level_start_index`` must equal the prefix sums of ``spatial_shapes``.
    """
    shapes = _as_shapes(spatial_shapes)
    _check_level_start_index(level_start_index, shapes)
    return _MSDeformAttnFunction.apply(value, sampling_locations, attention_weights, shapes)


def ms_deform_attn_core(value, spatial_shapes, sampling_locations, attention_weights):
    """ops.py:295-314: ``value [B, n_heads, head_dim, sum(H*W)]``, transposed to rows first."""
    batch, n_heads, head_dim, length = value.shape
    rows = value.transpose(2, 3).reshape(batch * n_heads, length, head_dim)
    return ms_deform_attn_core_rows(rows, spatial_shapes, sampling_locations, attention_weights)


# ------------------------------------------------------------------------------------------------
# The MSDeformAttn prologue fused into the kernels (ops.py:388-410)


def _check_fused_inputs(value, shapes, reference_points, sampling_offsets, attention_logits):
    if sampling_offsets.dim() != 6 or sampling_offsets.shape[-1] != 2:
        raise ValueError(
            f"sampling_offsets must be [B, Lq, n_heads, n_levels, n_points, 2], got {tuple(sampling_offsets.shape)}"
        )
    batch, len_query, n_heads, n_levels, n_points, _ = sampling_offsets.shape
    ref_dim = reference_points.shape[-1] if reference_points.dim() == 4 else -1
    if ref_dim not in (2, 4) or tuple(reference_points.shape[:3]) != (batch, len_query, n_levels):
        # ops.py:400 raises ValueError for a trailing dimension other than 2 or 4
        raise ValueError(
            f"reference_points must be [B, Lq, n_levels, 2 or 4] = {(batch, len_query, n_levels)} + (2|4,), "
            f"got {tuple(reference_points.shape)}"
        )
    dims = _check_inputs(value, shapes, sampling_offsets, attention_logits)
    if reference_points.device != value.device:
        raise RuntimeError("reference_points must be on the value's device")
    return dims, ref_dim


def ms_deform_attn_fused_forward(value, spatial_shapes, reference_points, sampling_offsets, attention_logits,
                                 level_start_index=None, out_dtype=None):
    """One forward launch of the fused op (no autograd): returns ``[B, Q, H*D]``.

    ``sampling_locations`` and ``attention_weights`` are formed inside the kernel from
    ``reference_points [B, Q, L, 2|4]``, ``sampling_offsets [B, Q, H, L, P, 2]`` and
    ``attention_logits [B, Q, H, L*P]`` exactly as ops.py:388-404 forms them.
    """
    shapes = _as_shapes(spatial_shapes)
    _check_level_start_index(level_start_index, shapes)
    (batch, len_query, n_heads, n_levels, n_points, head_dim), ref_dim = _check_fused_inputs(
        value, shapes, reference_points, sampling_offsets, attention_logits
    )
    out_dtype = out_dtype or _out_dtype(value, attention_logits)
    value = value.contiguous()
    ref = reference_points.to(torch.float32).contiguous()
    off = sampling_offsets.to(torch.float32).contiguous()
    logits = attention_logits.to(torch.float32).contiguous()
    out = torch.empty((batch, len_query, n_heads * head_dim), dtype=out_dtype, device=value.device)
    arr, starts = _shape_arrays(shapes)
    lib = _native.lib()
    with torch.cuda.device(value.device):
        rc = lib.msda_fused_fwd(
            _ptr(value), _VALUE_DTYPES[value.dtype], _ptr(ref), ref_dim, _ptr(off), _ptr(logits), _ptr(out),
            _VALUE_DTYPES[out_dtype], batch, n_heads, head_dim, len_query, n_levels, n_points, arr, starts, value.shape[1],
            _stream(value.device),
        )
    _native.check(rc)
    return out


def ms_deform_attn_fused_backward(value, spatial_shapes, reference_points, sampling_offsets, attention_logits, grad_output,
                                  level_start_index=None, needs=(True, True, True, True)):
    """One backward launch of the fused op.

    Returns ``(grad_value, grad_reference_points, grad_sampling_offsets, grad_attention_logits)``;
    entries of ``needs`` (same order) that are false come back as ``None`` and are not computed.
    """
    shapes = _as_shapes(spatial_shapes)
    _check_level_start_index(level_start_index, shapes)
    (batch, len_query, n_heads, n_levels, n_points, head_dim), ref_dim = _check_fused_inputs(
        value, shapes, reference_points, sampling_offsets, attention_logits
    )
    if tuple(grad_output.shape) != (batch, len_query, n_heads * head_dim):
        raise ValueError(f"grad_output must be {(batch, len_query, n_heads * head_dim)}, got {tuple(grad_output.shape)}")
    value = value.contiguous()
    ref = reference_points.to(torch.float32).contiguous()
    off = sampling_offsets.to(torch.float32).contiguous()
    logits = attention_logits.to(torch.float32).contiguous()
    if grad_output.dtype not in _VALUE_DTYPES:
        grad_output = grad_output.to(torch.float32)
    grad_output = grad_output.contiguous()
    dev = value.device
    grad_value = torch.empty_like(value) if needs[0] else None
    grad_ref = torch.empty(ref.shape, dtype=torch.float32, device=dev) if needs[1] else None
    grad_off = torch.empty(off.shape, dtype=torch.float32, device=dev) if needs[2] else None
    grad_logits = torch.empty(logits.shape, dtype=torch.float32, device=dev) if needs[3] else None
    arr, starts = _shape_arrays(shapes)
    lib = _native.lib()
    # the prologue's locations and weights and the query blocks' partial sums (any gradient needs it)
    ws_bytes = lib.msda_fused_bwd_workspace_size(batch, n_heads, head_dim, len_query, n_levels, n_points, ref_dim, arr,
                                                 starts, value.shape[1])
    if ws_bytes < 0:
        _native.check(int(ws_bytes))
    workspace = torch.empty((max(1, ws_bytes // 16), 4), dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        rc = lib.msda_fused_bwd(
            _ptr(value), _VALUE_DTYPES[value.dtype], _ptr(ref), ref_dim, _ptr(off), _ptr(logits), _ptr(grad_output),
            _VALUE_DTYPES[grad_output.dtype], _ptr(grad_value), _ptr(grad_off), _ptr(grad_logits), _ptr(grad_ref),
            batch, n_heads, head_dim, len_query, n_levels, n_points, arr, starts, value.shape[1],
            _ptr(workspace), ws_bytes, _stream(dev),
        )
    _native.check(rc)
    return grad_value, grad_ref, grad_off, grad_logits


class _MSDeformAttnFusedFunction(torch.autograd.Function):
    """custom-VJP pair of the fused op: forward = msda_fused_fwd, backward = msda_fused_bwd."""

    @staticmethod
    def forward(ctx, value, reference_points, sampling_offsets, attention_logits, shapes):
        out = ms_deform_attn_fused_forward(value, shapes, reference_points, sampling_offsets, attention_logits)
        ctx.save_for_backward(value, reference_points, sampling_offsets, attention_logits)
        ctx.shapes = shapes
        ctx.out_dtype = out.dtype
        return out

    @staticmethod
    def backward(ctx, grad_output):
        value, ref, off, logits = ctx.saved_tensors
        needs = ctx.needs_input_grad[:4]
        grads = ms_deform_attn_fused_backward(value, ctx.shapes, ref, off, logits, grad_output.to(ctx.out_dtype), needs=needs)
        out = []
        for g, src in zip(grads, (value, ref, off, logits)):
            out.append(g.to(src.dtype) if g is not None and g.dtype != src.dtype else g)
        return (*out, None)


def ms_deform_attn_fused(value, spatial_shapes, reference_points, sampling_offsets, attention_logits):
    """``MSDeformAttn``'s core from the projected query: ops.py:388-410 in one differentiable op.

    Args:
        value: ``[B * n_heads, sum(H*W), head_dim]`` (the module's projected value, ops.py:405-407).
        spatial_shapes: per-level ``(H, W)`` pairs.
        reference_points: ``[B, Lq, n_levels, 2]`` points or ``[B, Lq, n_levels, 4]`` boxes in
            ``[0, 1]``.
        sampling_offsets: ``[B, Lq, n_heads, n_levels, n_points, 2]`` (the ``sampling_offsets``
            projection, reshaped as ops.py:384-386 does).
        attention_logits: ``[B, Lq, n_heads, n_levels * n_points]`` before the softmax
            (ops.py:381-383).

    Returns:
        ``[B, Lq, n_heads * head_dim]``; differentiable in all four tensors.

    Raises:
        ValueError: a ``reference_points`` trailing dimension other than 2 or 4 (as ops.py:400),
            or inconsistent shapes.
    """
    shapes = _as_shapes(spatial_shapes)
    return _MSDeformAttnFusedFunction.apply(value, reference_points, sampling_offsets, attention_logits, shapes)
