"""MI355X (gfx950) multi-scale deformable attention for RF-DETR-JAX's decoder.

Host-side mirror of the reference interface ``rfdetr_jax.models.ops``
(src/rfdetr_jax/models/ops.py:208-314): the same function names, argument meanings and errors,
backed by hand-written HIP kernels through the C ABI in include/msda.h. Also the module around it
(``MSDeformAttn``, ops.py:326-411) with its prologue, value projection and head split fused into the
kernels, the segmentation head's point sampling (``bilinear_grid_sample``, ``point_sample``), and the
decoder's grouped self-attention (``MultiheadAttention``, ``scaled_dot_product_attention``,
layers.py:54-99, :491-548).
"""

from .attention import (
    MultiheadAttention,
    decoder_self_attention,
    dropout_keep_mask,
    grouped_attention,
    scaled_dot_product_attention,
)
from .grid_sample import bilinear_grid_sample, point_sample
from .ops import (
    SAMPLERS,
    ms_deform_attn,
    ms_deform_attn_backward,
    ms_deform_attn_core,
    ms_deform_attn_core_rows,
    ms_deform_attn_forward,
    ms_deform_attn_fused,
    ms_deform_attn_fused_backward,
    ms_deform_attn_fused_forward,
)
from .value_proj import MSDeformAttn, value_proj_rows

__all__ = [
    "MSDeformAttn",
    "MultiheadAttention",
    "SAMPLERS",
    "bilinear_grid_sample",
    "decoder_self_attention",
    "dropout_keep_mask",
    "grouped_attention",
    "ms_deform_attn",
    "ms_deform_attn_backward",
    "ms_deform_attn_core",
    "ms_deform_attn_core_rows",
    "ms_deform_attn_forward",
    "ms_deform_attn_fused",
    "ms_deform_attn_fused_backward",
    "ms_deform_attn_fused_forward",
    "point_sample",
    "scaled_dot_product_attention",
    "value_proj_rows",
]
