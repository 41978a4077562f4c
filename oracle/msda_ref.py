"""CPU oracle for multi-scale deformable attention — TEST INFRASTRUCTURE ONLY.

Nothing in the product path imports this module. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg may use it, and only as the checker.

It restates, in NumPy, the reference's ``gather`` sampler path and its autodiff gradients:

* ``_sample_rows``           src/rfdetr_jax/models/ops.py:64-134  (coordinates, floor, masks,
                                                                  clipped corners, corner weights)
* ``ms_deform_attn_core_rows`` ops.py:208-292 (level slicing by prefix sums :265-267, the grid
                                                 ``2*loc-1`` :270, level-major point order :285,
                                                 the einsum :289, output layout :290-292)
* gradients: the VJP JAX autodiff derives from the above; the same formulas the fused TPU sampler
  writes by hand (deform_pallas.py:97-120: ``da = sum g*sample``, ``dix = a * sum g*dK/dx . V``,
  ``dV += (g*a) K^T``).

Precision: sample coordinates are computed in ``promote_types(loc.dtype, float32)`` exactly as the
reference does (ops.py:80, :270), one IEEE rounding per operation, so floor decisions are those of
an f32 run. Everything after the coordinates is float64. A bf16 value map is passed in already
rounded to bf16 (as a float array): the reference's tests compare bf16 runs against float32 math
on the bf16-rounded values (tests/test_ops.py:238).

Pinning (each function here is checked by tests/test_oracle.py against something that is not a
retyping of these formulas):
* ``ms_deform_attn_core_rows``: the four closed-form known-answer tests of the reference
  (tests/test_ops.py:22-54); torch ``F.grid_sample`` (bilinear, zeros, align_corners=False), the
  library routine ops.py:14-16 says the sampler reproduces; a pure-Python brute-force loop on tiny
  inputs; integer-pixel translation invariance.
* ``ms_deform_attn_core_rows_vjp``: torch autograd through ``F.grid_sample`` in float64; central
  finite differences of the float64 forward; linearity of the output in value and in weights
  (``<G, out> = <dV, V>`` and ``= <dA, A>``).
* ``ms_deform_attn_core_rows_bf16_gather`` (the reference's bf16 rounding points of the ``gather``
  sampler, ops.py:88-91 and :123-134): equal to the float64 forward where every fraction, weight
  and product is exact in bf16 (quarter-pixel positions, small integer values); a planted mistake
  (the coordinate rounded to bf16 instead of its fraction) changes the result.
* ``ms_deform_attn_core_rows_sampler`` (each sampler name's forward: the bf16 rounding points of
  ``gather`` ops.py:64-134, ``gather-f32`` :137-144 and ``matmul`` :147-186, ``auto``'s per-level
  choice :277-279, the Pallas kernel's pixel coordinates deform_pallas.py:221-224): per-level
  samples equal torch arithmetic in the reference's dtypes (bf16 operations round after every
  step), every sampler equals the float64 forward where all roundings are exact, and the Pallas
  coordinates equal torch f32 arithmetic and flip floor decisions against ops.py's near cell
  boundaries. ``ms_deform_attn_core_rows_vjp_pallas``: finite differences of that forward and the
  ``<G, out> = <dV, V> = <dA, A>`` identities.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "level_offsets",
    "ms_deform_attn_core_rows",
    "ms_deform_attn_core_rows_vjp",
    "ms_deform_attn_core_rows_bf16_gather",
    "ms_deform_attn_core_rows_sampler",
    "ms_deform_attn_core_rows_vjp_pallas",
    "brute_force_forward",
    "bf16_round",
]


def level_offsets(spatial_shapes):
    """Prefix sums of H_l*W_l (ops.py:265-267)."""
    offsets = [0]
    for height, width in spatial_shapes:
        offsets.append(offsets[-1] + int(height) * int(width))
    return offsets


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(nan, (u | 0x00400000) & 0xFFFF0000, r)
    return r.astype(np.uint32).view(np.float32).reshape(np.shape(x))


def _pixel_coords(loc: np.ndarray, size: int) -> np.ndarray:
    """``((2*loc - 1) + 1) * size - 1) / 2`` with one rounding per op (ops.py:270, ops.py:83-84)."""
    ctype = np.promote_types(loc.dtype, np.float32)
    loc = loc.astype(ctype)
    one = ctype.type(1)
    grid = ctype.type(2) * loc - one
    return ((grid + one) * ctype.type(size) - one) / ctype.type(2)


def _pallas_coords(loc: np.ndarray, size: int) -> np.ndarray:
    """``loc * size - 0.5`` in float32, two roundings (deform_pallas.py:221-224)."""
    loc = np.asarray(loc).astype(np.float32)
    return loc * np.float32(size) - np.float32(0.5)


def _corners(loc_x, loc_y, height, width, pallas=False):
    """Clipped corner indices, masked weights and masks for one level (ops.py:83-128).

    Returns ``idx[..., 4]`` (flat index inside the level, corner order (x0,y0),(x1,y0),(x0,y1),
    (x1,y1) as ops.py:110-118), ``w[..., 4]`` float64 masked weights, ``m[..., 4]`` float64 masks,
    and the fractional parts ``fx, fy`` (float64) that the gradient needs. ``pallas``: the pixel
    coordinates of the Pallas sampler (deform_pallas.py:223-224), whose axis kernels
    (:52-59) put 1 - frac and frac at floor and floor + 1 and match no position off the map, the
    same weights and masks.
    """
    coords = _pallas_coords if pallas else _pixel_coords
    ix = coords(loc_x, width)
    iy = coords(loc_y, height)
    ix0 = np.floor(ix)
    iy0 = np.floor(iy)
    # Rounded in the coordinate dtype, as ops.py:88-89 computes it (inexact for ix in (-1, 0)).
    fx = (ix - ix0).astype(np.float64)
    fy = (iy - iy0).astype(np.float64)
    gx = 1.0 - fx
    gy = 1.0 - fy
    # Saturating float->int conversion with NaN -> 0 (XLA's convert semantics).
    def to_int(v):
        v = np.where(np.isnan(v), 0.0, v)
        return np.clip(v, -(2**31), 2**31 - 1).astype(np.int64)

    x0 = to_int(ix0)
    y0 = to_int(iy0)
    x1 = x0 + 1
    y1 = y0 + 1
    in_x0 = (x0 >= 0) & (x0 < width)
    in_x1 = (x1 >= 0) & (x1 < width)
    in_y0 = (y0 >= 0) & (y0 < height)
    in_y1 = (y1 >= 0) & (y1 < height)
    cx0 = np.clip(x0, 0, width - 1)
    cx1 = np.clip(x1, 0, width - 1)
    cy0 = np.clip(y0, 0, height - 1)
    cy1 = np.clip(y1, 0, height - 1)
    idx = np.stack([cy0 * width + cx0, cy0 * width + cx1, cy1 * width + cx0, cy1 * width + cx1], -1)
    m = np.stack([in_x0 & in_y0, in_x1 & in_y0, in_x0 & in_y1, in_x1 & in_y1], -1).astype(np.float64)
    w = np.stack([gx * gy, fx * gy, gx * fy, fx * fy], -1) * m
    return idx, w, m, fx, fy


def _gather(value_bh, idx):
    """value_bh [B,H,S_l,D]; idx [B,Q,H,P,4] -> [B,Q,H,P,4,D]."""
    b, q, h, p, c = idx.shape
    d = value_bh.shape[-1]
    flat = np.transpose(idx, (0, 2, 1, 3, 4)).reshape(b, h, q * p * c)
    taken = np.take_along_axis(value_bh, flat[..., None], axis=2)  # [B,H,QPC,D]
    return np.transpose(taken.reshape(b, h, q, p, c, d), (0, 2, 1, 3, 4, 5))


def _split(value, spatial_shapes, sampling_locations):
    batch, len_query, n_heads, n_levels, n_points, _ = sampling_locations.shape
    n, s, d = value.shape
    if n != batch * n_heads:
        raise ValueError(f"value leading dim {n} != batch*n_heads {batch * n_heads}")
    offsets = level_offsets(spatial_shapes)
    if offsets[-1] != s:
        raise ValueError(f"value length {s} != sum(H*W) {offsets[-1]}")
    if len(spatial_shapes) != n_levels:
        raise ValueError("spatial_shapes / sampling_locations level count mismatch")
    return batch, len_query, n_heads, n_levels, n_points, d, offsets


def ms_deform_attn_core_rows(value, spatial_shapes, sampling_locations, attention_weights):
    """Forward of ops.py:208-292 (``gather`` sampler), float64 result ``[B, Q, H*D]``."""
    batch, len_query, n_heads, n_levels, n_points, d, offsets = _split(value, spatial_shapes, sampling_locations)
    v64 = np.asarray(value, dtype=np.float64).reshape(batch, n_heads, -1, d)
    attn = np.asarray(attention_weights, dtype=np.float64).reshape(batch, len_query, n_heads, n_levels, n_points)
    out = np.zeros((batch, len_query, n_heads, d), np.float64)
    for level, (height, width) in enumerate(spatial_shapes):
        v_l = v64[:, :, offsets[level] : offsets[level + 1], :]
        loc = sampling_locations[:, :, :, level]
        idx, w, _, _, _ = _corners(loc[..., 0], loc[..., 1], height, width)
        corners = _gather(v_l, idx)  # [B,Q,H,P,4,D]
        sample = np.einsum("bqhpc,bqhpcd->bqhpd", w, corners)
        out += np.einsum("bqhp,bqhpd->bqhd", attn[:, :, :, level], sample)
    return out.reshape(batch, len_query, n_heads * d)


def ms_deform_attn_core_rows_vjp(value, spatial_shapes, sampling_locations, attention_weights, grad_output, pallas=False):
    """Gradients of ops.py:208-292 for cotangent ``grad_output [B,Q,H*D]``.

    Returns ``(grad_value [B*H,S,D], grad_locations [B,Q,H,L,P,2], grad_weights [B,Q,H,L*P])``,
    all float64. ``d ix / d loc = W`` (ops.py:270 gives 2, ops.py:83 gives W/2); floor and the
    in-bounds masks are piecewise constant and contribute nothing.
    """
    batch, len_query, n_heads, n_levels, n_points, d, offsets = _split(value, spatial_shapes, sampling_locations)
    v64 = np.asarray(value, dtype=np.float64).reshape(batch, n_heads, -1, d)
    attn = np.asarray(attention_weights, dtype=np.float64).reshape(batch, len_query, n_heads, n_levels, n_points)
    g = np.asarray(grad_output, dtype=np.float64).reshape(batch, len_query, n_heads, d)
    grad_value = np.zeros_like(v64)
    grad_loc = np.zeros((batch, len_query, n_heads, n_levels, n_points, 2), np.float64)
    grad_attn = np.zeros((batch, len_query, n_heads, n_levels, n_points), np.float64)
    b_idx = np.arange(batch)[:, None, None, None, None]
    h_idx = np.arange(n_heads)[None, None, :, None, None]
    for level, (height, width) in enumerate(spatial_shapes):
        start = offsets[level]
        v_l = v64[:, :, start : offsets[level + 1], :]
        loc = sampling_locations[:, :, :, level]
        idx, w, m, fx, fy = _corners(loc[..., 0], loc[..., 1], height, width, pallas=pallas)
        corners = _gather(v_l, idx)  # [B,Q,H,P,4,D]
        a = attn[:, :, :, level]  # [B,Q,H,P]
        sample = np.einsum("bqhpc,bqhpcd->bqhpd", w, corners)
        grad_attn[:, :, :, level] = np.einsum("bqhd,bqhpd->bqhp", g, sample)
        mv = corners * m[..., None]  # masked corner values
        gx, gy = 1.0 - fx, 1.0 - fy
        d_ix = gy[..., None] * (mv[..., 1, :] - mv[..., 0, :]) + fy[..., None] * (mv[..., 3, :] - mv[..., 2, :])
        d_iy = gx[..., None] * (mv[..., 2, :] - mv[..., 0, :]) + fx[..., None] * (mv[..., 3, :] - mv[..., 1, :])
        grad_loc[:, :, :, level, :, 0] = a * width * np.einsum("bqhd,bqhpd->bqhp", g, d_ix)
        grad_loc[:, :, :, level, :, 1] = a * height * np.einsum("bqhd,bqhpd->bqhp", g, d_iy)
        # scatter-add: dV[b,h,start+idx_c,:] += a * w_c * g
        contrib = (a[..., None] * w)[..., None] * g[:, :, :, None, None, :]  # [B,Q,H,P,4,D]
        flat_rows = (b_idx * n_heads + h_idx) * v64.shape[2] + start + idx  # [B,Q,H,P,4]
        gv = grad_value.reshape(-1, d)
        rows = flat_rows.reshape(-1)
        vals = contrib.reshape(-1, d)
        for ch in range(d):
            gv[:, ch] += np.bincount(rows, weights=vals[:, ch], minlength=gv.shape[0])
    return (
        grad_value.reshape(batch * n_heads, -1, d),
        grad_loc,
        grad_attn.reshape(batch, len_query, n_heads, n_levels * n_points),
    )


def ms_deform_attn_core_rows_bf16_gather(value, spatial_shapes, sampling_locations, attention_weights,
                                         _round_coordinate=False):
    """Forward of ops.py:208-292 with the ``gather`` sampler on a bf16 value map, rounding where the
    reference's bf16 computation rounds: the fractions ``wx1 = (ix - ix0).astype(bf16)`` (ops.py:88-89),
    ``1 - w`` and the corner-weight products in bf16 (:90-91, :123), the mask (:125-128), each corner
    product ``stacked * weight`` in bf16 and the four-corner sum rounded to bf16 (:134; the sum itself
    taken in f32, as XLA accumulates bf16 reductions); then the einsum with the f32 attention weights
    in f32 or wider (:289). ``value`` holds bf16-representable values as float32. Float64 result.
    ``_round_coordinate`` plants a mistake for the oracle's own tests (the coordinate is rounded to
    bf16 before the floor, instead of the fraction after it)."""
    batch, len_query, n_heads, n_levels, n_points, d, offsets = _split(value, spatial_shapes, sampling_locations)
    v32 = np.asarray(value, dtype=np.float32).reshape(batch, n_heads, -1, d)
    attn = np.asarray(attention_weights, dtype=np.float64).reshape(batch, len_query, n_heads, n_levels, n_points)
    out = np.zeros((batch, len_query, n_heads, d), np.float64)
    one = np.float32(1)
    for level, (height, width) in enumerate(spatial_shapes):
        v_l = v32[:, :, offsets[level] : offsets[level + 1], :]
        loc = sampling_locations[:, :, :, level]
        ix = _pixel_coords(loc[..., 0], width).astype(np.float32)
        iy = _pixel_coords(loc[..., 1], height).astype(np.float32)
        if _round_coordinate:
            ix, iy = bf16_round(ix), bf16_round(iy)
        ix0, iy0 = np.floor(ix), np.floor(iy)
        wx1 = bf16_round(ix - ix0)
        wy1 = bf16_round(iy - iy0)
        wx0 = bf16_round(one - wx1)
        wy0 = bf16_round(one - wy1)
        weight = np.stack([bf16_round(wx0 * wy0), bf16_round(wx1 * wy0), bf16_round(wx0 * wy1), bf16_round(wx1 * wy1)], -1)
        idx, _, m, _, _ = _corners(loc[..., 0], loc[..., 1], height, width)
        weight = weight * m.astype(np.float32)  # exact: the mask is 0 or 1
        corners = _gather(v_l, idx)  # [B,Q,H,P,4,D] float32, bf16 values
        prods = bf16_round(corners * weight[..., None])
        sample = bf16_round(prods.sum(axis=-2, dtype=np.float32))
        out += np.einsum("bqhp,bqhpd->bqhd", attn[:, :, :, level], sample.astype(np.float64))
    return out.reshape(batch, len_query, n_heads * d)


#: _MATMUL_SAMPLER_MAX_LEVEL (ops.py:42): "auto" uses the matmul sampler up to this many positions.
MATMUL_SAMPLER_MAX_LEVEL = 4096


def _bf16_level_sample(v_l, loc, height, width, mode):
    """One level's samples ``[B,Q,H,P,D]`` (float32 holding bf16 values) on a bf16 value map with
    the rounding points of ``mode``: ``"gather"`` (ops.py:88-91, :123-134), ``"gather-f32"``
    (ops.py:137-144: f32 interpolation, the sample rounded to bf16) or ``"matmul"`` (ops.py:170-186:
    the axis kernels and their outer product rounded to bf16, the contraction in f32, its result
    rounded to bf16). Products and sums in float32, one rounding each, corners in index order."""
    one = np.float32(1)
    ix = _pixel_coords(loc[..., 0], width).astype(np.float32)
    iy = _pixel_coords(loc[..., 1], height).astype(np.float32)
    fx = ix - np.floor(ix)
    fy = iy - np.floor(iy)
    idx, _, m, _, _ = _corners(loc[..., 0], loc[..., 1], height, width)
    if mode == "gather":
        wx1, wy1 = bf16_round(fx), bf16_round(fy)
        wx0, wy0 = bf16_round(one - wx1), bf16_round(one - wy1)
        weight = np.stack([bf16_round(wx0 * wy0), bf16_round(wx1 * wy0), bf16_round(wx0 * wy1), bf16_round(wx1 * wy1)], -1)
    elif mode == "matmul":
        kx0, kx1 = bf16_round(one - fx), bf16_round(fx)
        ky0, ky1 = bf16_round(one - fy), bf16_round(fy)
        weight = np.stack([bf16_round(ky0 * kx0), bf16_round(ky0 * kx1), bf16_round(ky1 * kx0), bf16_round(ky1 * kx1)], -1)
    elif mode == "gather-f32":
        wx0, wy0 = one - fx, one - fy
        weight = np.stack([wx0 * wy0, fx * wy0, wx0 * fy, fx * fy], -1)
    else:
        raise ValueError(mode)
    weight = weight * m.astype(np.float32)  # exact: the mask is 0 or 1
    corners = _gather(v_l, idx)  # [B,Q,H,P,4,D] float32
    prods = corners * weight[..., None]
    if mode == "gather":
        prods = bf16_round(prods)
    total = ((prods[..., 0, :] + prods[..., 1, :]) + prods[..., 2, :]) + prods[..., 3, :]
    return bf16_round(total)


def ms_deform_attn_core_rows_sampler(value, spatial_shapes, sampling_locations, attention_weights, sampler, bf16_value):
    """Forward of ops.py:208-292 with a named sampler (``"hip"``, ``"gather"``, ``"gather-f32"``,
    ``"matmul"``, ``"auto"``, ``"pallas"``), float64 ``[B, Q, H*D]``: on a bf16 value map (``value``
    holding bf16-representable float32 values, ``bf16_value`` true) each level's samples carry the
    sampler's bf16 rounding points (_bf16_level_sample; "auto" picks matmul for levels of at most
    MATMUL_SAMPLER_MAX_LEVEL positions, ops.py:277-279); "pallas" forms the pixel coordinates as
    deform_pallas.py:223-224 does and interpolates in float64; "hip" and every sampler on an f32 map
    is the float64 forward. The sum over levels and points (:289) in float64."""
    if sampler == "hip":
        return ms_deform_attn_core_rows(value, spatial_shapes, sampling_locations, attention_weights)
    if sampler not in ("gather", "gather-f32", "matmul", "auto", "pallas"):
        raise ValueError(f"unknown sampler {sampler!r}")
    batch, len_query, n_heads, n_levels, n_points, d, offsets = _split(value, spatial_shapes, sampling_locations)
    v64 = np.asarray(value, dtype=np.float64).reshape(batch, n_heads, -1, d)
    attn = np.asarray(attention_weights, dtype=np.float64).reshape(batch, len_query, n_heads, n_levels, n_points)
    out = np.zeros((batch, len_query, n_heads, d), np.float64)
    for level, (height, width) in enumerate(spatial_shapes):
        v_l = v64[:, :, offsets[level] : offsets[level + 1], :]
        loc = sampling_locations[:, :, :, level]
        mode = sampler
        if mode == "auto":
            mode = "matmul" if height * width <= MATMUL_SAMPLER_MAX_LEVEL else "gather"
        if mode == "pallas" or not bf16_value:
            idx, w, _, _, _ = _corners(loc[..., 0], loc[..., 1], height, width, pallas=mode == "pallas")
            sample = np.einsum("bqhpc,bqhpcd->bqhpd", w, _gather(v_l, idx))
        else:
            sample = _bf16_level_sample(v_l.astype(np.float32), loc, height, width, mode).astype(np.float64)
        out += np.einsum("bqhp,bqhpd->bqhd", attn[:, :, :, level], sample)
    return out.reshape(batch, len_query, n_heads * d)


def ms_deform_attn_core_rows_vjp_pallas(value, spatial_shapes, sampling_locations, attention_weights, grad_output):
    """ms_deform_attn_core_rows_vjp at the Pallas sampler's pixel coordinates (deform_pallas.py:
    97-120, 221-224): the same formulas, floor and fractions from loc * size - 0.5."""
    return ms_deform_attn_core_rows_vjp(value, spatial_shapes, sampling_locations, attention_weights, grad_output, pallas=True)


def brute_force_forward(value, spatial_shapes, sampling_locations, attention_weights):
    """Pure-Python loop over (b, q, h, l, p, corner, d) for tiny inputs; float64.

    Written independently of the vectorised path above (scalar ``math`` arithmetic, explicit
    bounds tests instead of clipped-index masking) so the two pin each other.
    """
    import math

    batch, len_query, n_heads, n_levels, n_points, _ = sampling_locations.shape
    d = value.shape[-1]
    offsets = level_offsets(spatial_shapes)
    out = np.zeros((batch, len_query, n_heads * d))
    f32 = np.float32
    for b in range(batch):
        for q in range(len_query):
            for h in range(n_heads):
                for level, (height, width) in enumerate(spatial_shapes):
                    for p in range(n_points):
                        lx, ly = sampling_locations[b, q, h, level, p]
                        # f32 coordinates, one rounding per operation
                        ix = float((((f32(2) * f32(lx) - f32(1)) + f32(1)) * f32(width) - f32(1)) / f32(2))
                        iy = float((((f32(2) * f32(ly) - f32(1)) + f32(1)) * f32(height) - f32(1)) / f32(2))
                        x0, y0 = math.floor(ix), math.floor(iy)
                        # fractional parts rounded to f32 like ops.py:88-89
                        fx = float(f32(ix) - f32(x0))
                        fy = float(f32(iy) - f32(y0))
                        a = float(attention_weights[b, q, h, level * n_points + p])
                        for dy in (0, 1):
                            for dx in (0, 1):
                                xx, yy = x0 + dx, y0 + dy
                                if not (0 <= xx < width and 0 <= yy < height):
                                    continue
                                wx = fx if dx else 1.0 - fx
                                wy = fy if dy else 1.0 - fy
                                row = offsets[level] + yy * width + xx
                                for c in range(d):
                                    out[b, q, h * d + c] += a * wx * wy * float(value[b * n_heads + h, row, c])
    return out
