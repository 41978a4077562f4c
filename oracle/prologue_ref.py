"""CPU oracle for the MSDeformAttn prologue — TEST INFRASTRUCTURE ONLY.

Nothing in the product path imports this module. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg may use it, and only as the checker.

It restates, in NumPy, the lines of ``MSDeformAttn.__call__`` (src/rfdetr_jax/models/ops.py) that
turn the projected query into the deformable-attention core's inputs, and the VJP JAX autodiff
derives from them:

* ``prologue``      ops.py:388-394 (2-dim reference points: ``loc = ref + offsets / (W_l, H_l)``,
                    the normaliser stacked as ``(shapes[:, 1], shapes[:, 0])``), ops.py:395-399
                    (4-dim boxes: ``loc = ref_xy + offsets / n_points * ref_wh * 0.5``, evaluated
                    left to right), both with ``precise_divide`` (ops.py:46-62: one IEEE rounding
                    per division); ops.py:403-404 (softmax over the L*P logits in
                    ``promote_types(dtype, float32)``, cast back to the query dtype, f32 here).
* ``prologue_vjp``  the transpose of the above for cotangents ``(grad_loc, grad_attn)`` of the
                    core's inputs: ``grad_offsets = grad_loc / (W_l, H_l)`` (2-dim) or
                    ``((grad_loc * 0.5) * ref_wh) / n_points`` (4-dim); ``grad_logits =
                    y * (g - sum(y * g))`` (the softmax JVP transposed); ``grad_ref`` sums the
                    broadcast over heads and points (ops.py:391, :397).

Precision: locations and weights are computed in float32 with one rounding per operation, as the
reference's f32 run does (the location decides the floor of the sample coordinate); the VJP is
float64.

Pinning (tests/test_oracle.py): torch float64 autograd through torch's own softmax and broadcasting
(``prologue_vjp``, and the full chain through ``F.grid_sample``); closed forms (zero offsets give
the reference point exactly, offsets of whole level sizes move by exact steps, equal logits give
1/(L*P), the softmax VJP sums to zero per (query, head)); planted mistakes (swapped normaliser,
a dropped 0.5, a softmax over the wrong axis) fail them.
"""

from __future__ import annotations

import numpy as np

__all__ = ["prologue", "prologue_vjp"]


def _check(reference_points, sampling_offsets, attention_logits, spatial_shapes, n_points):
    batch, len_query, n_heads, n_levels, points, two = sampling_offsets.shape
    if two != 2 or points != n_points:
        raise ValueError(f"sampling_offsets must be [B, Q, H, L, {n_points}, 2], got {sampling_offsets.shape}")
    if len(spatial_shapes) != n_levels:
        raise ValueError("spatial_shapes / sampling_offsets level count mismatch")
    ref_dim = reference_points.shape[-1]
    if reference_points.shape != (batch, len_query, n_levels, ref_dim) or ref_dim not in (2, 4):
        raise ValueError(f"reference_points must be [B, Q, L, 2 or 4], got {reference_points.shape}")
    if attention_logits.shape != (batch, len_query, n_heads, n_levels * n_points):
        raise ValueError(f"attention_logits must be [B, Q, H, L*P], got {attention_logits.shape}")
    return ref_dim


def prologue(reference_points, sampling_offsets, attention_logits, spatial_shapes, n_points):
    """``(sampling_locations [B,Q,H,L,P,2], attention_weights [B,Q,H,L*P])``, both float32."""
    ref_dim = _check(reference_points, sampling_offsets, attention_logits, spatial_shapes, n_points)
    f32 = np.float32
    ref = np.asarray(reference_points, f32)
    off = np.asarray(sampling_offsets, f32)
    if ref_dim == 2:
        shapes = np.asarray(spatial_shapes, f32)
        normalizer = np.stack([shapes[:, 1], shapes[:, 0]], axis=-1)  # (W_l, H_l), ops.py:390
        loc = ref[:, :, None, :, None, :] + off / normalizer[None, None, None, :, None, :]
    else:
        loc = ref[:, :, None, :, None, :2] + (off / f32(n_points)) * ref[:, :, None, :, None, 2:] * f32(0.5)
    x = np.asarray(attention_logits, f32)
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m)
    attn = e / np.sum(e, axis=-1, keepdims=True)
    return loc.astype(f32), attn.astype(f32)


def prologue_vjp(reference_points, sampling_offsets, attention_logits, spatial_shapes, n_points, grad_loc, grad_attn):
    """``(grad_offsets, grad_logits, grad_reference_points)`` in float64 for cotangents of the outputs
    of :func:`prologue` (``grad_loc [B,Q,H,L,P,2]``, ``grad_attn [B,Q,H,L*P]``)."""
    ref_dim = _check(reference_points, sampling_offsets, attention_logits, spatial_shapes, n_points)
    g_loc = np.asarray(grad_loc, np.float64)
    g_attn = np.asarray(grad_attn, np.float64)
    ref = np.asarray(reference_points, np.float64)
    off = np.asarray(sampling_offsets, np.float64)
    if ref_dim == 2:
        shapes = np.asarray(spatial_shapes, np.float64)
        normalizer = np.stack([shapes[:, 1], shapes[:, 0]], axis=-1)
        grad_off = g_loc / normalizer[None, None, None, :, None, :]
        grad_ref = g_loc.sum(axis=(2, 4))  # [B,Q,L,2]
    else:
        half = g_loc * 0.5
        wh = ref[:, :, None, :, None, 2:]
        grad_off = half * wh / n_points
        grad_xy = g_loc.sum(axis=(2, 4))
        grad_wh = (half * (off / n_points)).sum(axis=(2, 4))
        grad_ref = np.concatenate([grad_xy, grad_wh], axis=-1)
    _, y = prologue(reference_points, sampling_offsets, attention_logits, spatial_shapes, n_points)
    y = y.astype(np.float64)
    grad_logits = y * (g_attn - np.sum(y * g_attn, axis=-1, keepdims=True))
    return grad_off, grad_logits, grad_ref
