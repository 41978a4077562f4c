"""The five benchmark workloads and their synthetic inputs.

Shapes are the configs of the benchmark definition (RF-DETR Nano decoder cross-attention:
16 heads x head_dim 16, 2 points; config 3 is a two-level 640px variant with 4 points):

=====  =====  ==============  =====  =====  ======  ==========
 cfg     B     levels           Q    L*P   value    mode
=====  =====  ==============  =====  =====  ======  ==========
  0      2    24x24             300   1*2   f32     forward
  1     16    24x24             300   1*2   f32     fwd + bwd
  2      8    24x24            3900   1*2   f32     fwd + bwd   (13 group-DETR groups x 300)
  3      8    80x80 + 20x20     300   2*4   bf16    fwd + bwd
  4     64    36x36             300   1*2   bf16    forward     (locations U[-0.1, 1.1])
=====  =====  ==============  =====  =====  ======  ==========

:func:`make_inputs` draws the inputs in one fixed order from ``numpy.random.default_rng(seed)``
so the GPU run, the CPU baseline and the parity tests see identical data.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Workload:
    cfg_id: int
    name: str
    batch: int
    heads: int
    head_dim: int
    queries: int
    shapes: tuple
    points: int
    value_dtype: str  # "f32" | "bf16"
    backward: bool
    uniform_locations: bool = False

    @property
    def levels(self) -> int:
        return len(self.shapes)

    @property
    def len_value(self) -> int:
        return sum(h * w for h, w in self.shapes)

    @property
    def samples(self) -> int:
        return self.batch * self.queries * self.heads * self.levels * self.points

    def hbm_bytes(self) -> dict:
        """Algorithmic HBM bytes: every input read once, every output written once."""
        sv = 2 if self.value_dtype == "bf16" else 4
        n = self.batch * self.heads
        value = n * self.len_value * self.head_dim * sv
        loc = self.samples * 2 * 4
        attn = self.samples * 4
        out = self.batch * self.queries * self.heads * self.head_dim * 4
        fwd = value + loc + attn + out
        bwd = (value + loc + attn + out) + (value + loc + attn) if self.backward else 0  # reads G, writes dV/dloc/dA
        return {"fwd": fwd, "bwd": bwd, "total": fwd + bwd}

    def lds_bytes(self) -> dict:
        """Algorithmic LDS bytes: the forward reads four corner rows per sample and stages each value
        slice once; the backward reads the corner rows, accumulates four grad_value rows per sample
        into an f64 accumulator (8 bytes per channel addition: ds_add_f64), stages the value slices,
        zeroes the accumulator and reads it back once at write-out (8 bytes per element each)."""
        sv = 2 if self.value_dtype == "bf16" else 4
        slices = self.batch * self.heads * self.len_value * self.head_dim
        corners = self.samples * 4 * self.head_dim
        fwd = corners * sv + slices * sv
        bwd = corners * sv + corners * 8 + slices * sv + slices * 8 * 2 if self.backward else 0
        return {"fwd": fwd, "bwd": bwd, "total": fwd + bwd}

    def lds_atomic_adds(self) -> int:
        """Algorithmic LDS atomic additions of the backward: grad_value gets four corner rows of
        head_dim channels per sample, each channel one f64 addition (ds_add_f64)."""
        return self.samples * 4 * self.head_dim if self.backward else 0

    def scaled(self, batch: int | None = None, queries: int | None = None) -> "Workload":
        return Workload(self.cfg_id, self.name, batch or self.batch, self.heads, self.head_dim, queries or self.queries,
                        self.shapes, self.points, self.value_dtype, self.backward, self.uniform_locations)


CONFIGS = {
    0: Workload(0, "nano_fwd_b2_f32", 2, 16, 16, 300, ((24, 24),), 2, "f32", False),
    1: Workload(1, "nano_fwdbwd_b16_f32", 16, 16, 16, 300, ((24, 24),), 2, "f32", True),
    2: Workload(2, "nano_groupdetr_fwdbwd_b8_q3900_f32", 8, 16, 16, 3900, ((24, 24),), 2, "f32", True),
    3: Workload(3, "two_level_fwdbwd_b8_bf16", 8, 16, 16, 300, ((80, 80), (20, 20)), 4, "bf16", True),
    4: Workload(4, "nano_infer_fwd_b64_bf16", 64, 16, 16, 300, ((36, 36),), 2, "bf16", False, True),
}


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bfloat16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(nan, (u | 0x00400000) & 0xFFFF0000, r)
    return r.astype(np.uint32).view(np.float32).reshape(np.shape(x))


def make_inputs(seed: int, batch, n_heads, head_dim, len_query, spatial_shapes, n_points,
                value_dtype="f32", uniform_locations=False, with_grad=True):
    """Synthetic inputs, drawn from ``numpy.random.default_rng(seed)`` in this order:

    1. value ~ N(0,1) ``[B*H, S, D]`` (rounded to bf16 for bf16 workloads);
    2. ref ~ U[0,1]^2 ``[B,Q,2]``, broadcast over H, L, P;
    3. offsets ~ N(0, 0.05) ``[B,Q,H,L,P,2]``; loc = ref + offsets
       (``uniform_locations``: loc ~ U[-0.1, 1.1]^2 drawn directly instead of 2-3);
    4. logits ~ N(0,1) ``[B,Q,H,L*P]``; A = softmax(logits, -1) in f32;
    5. G ~ N(0,1) ``[B,Q,H*D]`` f32 (when ``with_grad``).

    Returns float32 NumPy arrays ``(value, loc, attn, grad)``.
    """
    rng = np.random.default_rng(seed)
    n_levels = len(spatial_shapes)
    s = sum(int(h) * int(w) for h, w in spatial_shapes)
    value = rng.standard_normal((batch * n_heads, s, head_dim), dtype=np.float32)
    if value_dtype == "bf16":
        value = bf16_round(value)
    if uniform_locations:
        loc = rng.uniform(-0.1, 1.1, (batch, len_query, n_heads, n_levels, n_points, 2)).astype(np.float32)
    else:
        ref = rng.uniform(0.0, 1.0, (batch, len_query, 2)).astype(np.float32)
        off = rng.normal(0.0, 0.05, (batch, len_query, n_heads, n_levels, n_points, 2)).astype(np.float32)
        loc = (ref[:, :, None, None, None, :] + off).astype(np.float32)
    logits = rng.standard_normal((batch, len_query, n_heads, n_levels * n_points), dtype=np.float32)
    e = np.exp(logits - logits.max(-1, keepdims=True))
    attn = (e / e.sum(-1, keepdims=True)).astype(np.float32)
    grad = rng.standard_normal((batch, len_query, n_heads * head_dim), dtype=np.float32) if with_grad else None
    return value, loc, attn, grad


def workload_inputs(w: Workload, with_grad: bool | None = None):
    """Inputs of a workload, seeded by its config id."""
    return make_inputs(w.cfg_id, w.batch, w.heads, w.head_dim, w.queries, w.shapes, w.points, w.value_dtype,
                       w.uniform_locations, w.backward if with_grad is None else with_grad)


def make_fused_inputs(seed: int, batch, n_heads, head_dim, len_query, spatial_shapes, n_points, ref_dim=4,
                      value_dtype="f32", with_grad=True):
    """Synthetic inputs of the fused-prologue op (``ms_deform_attn_fused``), drawn from
    ``numpy.random.default_rng(seed)`` in this order:

    1. value ~ N(0,1) ``[B*H, S, D]`` (rounded to bf16 for bf16 workloads);
    2. reference points ``[B,Q,L,ref_dim]``: centres ~ U[0.05, 0.95]^2 and, for boxes
       (``ref_dim`` 4), sizes ~ U[0.05, 0.5]^2, the same for every level (as the decoder
       broadcasts one box to all levels, transformer.py:446-449);
    3. sampling offsets ~ N(0, 2) ``[B,Q,H,L,P,2]`` (pixels of the level for points; units of
       box / (2 P) for boxes, ops.py:391-397);
    4. attention logits ~ N(0, 2) ``[B,Q,H,L*P]``;
    5. G ~ N(0,1) ``[B,Q,H*D]`` f32 (when ``with_grad``).

    Returns float32 NumPy arrays ``(value, ref, offsets, logits, grad)``.
    """
    rng = np.random.default_rng(seed)
    n_levels = len(spatial_shapes)
    s = sum(int(h) * int(w) for h, w in spatial_shapes)
    value = rng.standard_normal((batch * n_heads, s, head_dim), dtype=np.float32)
    if value_dtype == "bf16":
        value = bf16_round(value)
    centre = rng.uniform(0.05, 0.95, (batch, len_query, 1, 2))
    if ref_dim == 4:
        size = rng.uniform(0.05, 0.5, (batch, len_query, 1, 2))
        ref = np.concatenate([centre, size], axis=-1)
    else:
        ref = centre
    ref = np.ascontiguousarray(np.broadcast_to(ref, (batch, len_query, n_levels, ref_dim))).astype(np.float32)
    off = rng.normal(0.0, 2.0, (batch, len_query, n_heads, n_levels, n_points, 2)).astype(np.float32)
    logits = rng.normal(0.0, 2.0, (batch, len_query, n_heads, n_levels * n_points)).astype(np.float32)
    grad = rng.standard_normal((batch, len_query, n_heads * head_dim), dtype=np.float32) if with_grad else None
    return value, ref, off, logits, grad
