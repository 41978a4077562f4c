"""The decoder's self-attention on MI355X: softmax attention and the module around it.

* :func:`scaled_dot_product_attention` — ``scaled_dot_product_attention(q, k, v, mask)``
  (src/rfdetr_jax/models/layers.py:54-99): ``[B, H, L, D]`` heads, ``mask`` ``[L, L]`` with
  ``True`` blocking a key (torch's convention), differentiable in q, k and v.
* :func:`grouped_attention` — the same function on ``[B, G * P, H * D]`` rows with the G query
  groups of each image attended separately (``_split_groups`` / ``_merge_groups``,
  src/rfdetr_jax/models/transformer.py:350-361, done by addressing: the kernels read group g of
  image b in place, no split, merge or head transposes).
* :class:`MultiheadAttention` — ``MultiheadAttention`` (layers.py:491-548): fused
  ``in_proj_weight [3C, C]`` / ``in_proj_bias``, ``out_proj``; same parameter names and layouts.
* :func:`decoder_self_attention` — the self-attention block of the decoder layer
  (transformer.py:200-210): ``query = key = tgt + query_pos``, ``value = tgt``, groups in training.

Both directions run in two HIP kernels (``msda_attention_fwd`` / ``msda_attention_bwd``); the head
dimension must be 32 or 64. There is no CPU path. Attention dropout (layers.py:537-544) is not
supported: a module built with ``dropout > 0`` raises in training.
"""

from __future__ import annotations

import ctypes

import torch

from . import _native

_DTYPES = {torch.float32: _native.DTYPE_F32, torch.bfloat16: _native.DTYPE_BF16}


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


class _Layout:
    """Slices (batch, groups), heads, rows and head dim of one attention call, and the element
    strides (batch, group, head, row) of each tensor."""

    def __init__(self, batch, groups, heads, length, head_dim):
        self.batch, self.groups, self.heads, self.len, self.head_dim = batch, groups, heads, length, head_dim

    def strides_bhld(self, t):
        """``[Z, H, L, D]`` (channels contiguous)."""
        if t.stride(-1) != 1:
            raise ValueError("attention tensors must have contiguous channels")
        return [t.stride(0), 0, t.stride(1), t.stride(2)]

    def strides_rows(self, t):
        """``[B, G * P, H * D]`` rows (channels contiguous; the row stride may exceed H * D)."""
        if t.stride(-1) != 1:
            raise ValueError("attention tensors must have contiguous channels")
        return [t.stride(0), self.len * t.stride(1), self.head_dim, t.stride(1)]


def _mask_u8(mask, length, device):
    if mask is None:
        return None
    if tuple(mask.shape) != (length, length):
        raise ValueError(f"attention mask must be [L, L] = {(length, length)}, got {tuple(mask.shape)}")
    mask = mask.to(device)
    if mask.dtype == torch.bool:
        return mask.contiguous().view(torch.uint8)
    return (mask != 0).to(torch.uint8).contiguous()


def _check(*tensors):
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(f"tensor on {t.device}; the HIP kernels need GPU tensors (there is no CPU path)")
        if t.dtype not in _DTYPES:
            raise TypeError(f"attention dtype {t.dtype} is not supported (float32 or bfloat16)")


def attention_forward(q, k, v, lay, strides_of, mask=None):
    """``(out, stats)``; ``out`` is allocated like ``q``'s logical shape, contiguous."""
    _check(q, k, v)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    stats = torch.empty((lay.batch * lay.groups * lay.heads * lay.len * 4,), dtype=torch.float32, device=q.device)
    strides = (ctypes.c_int64 * 16)(*(strides_of(q) + strides_of(k) + strides_of(v) + strides_of(out)))
    m = _mask_u8(mask, lay.len, q.device)
    with torch.cuda.device(q.device):
        rc = _native.lib().msda_attention_fwd(_ptr(q), _ptr(k), _ptr(v), _DTYPES[q.dtype], _ptr(out), _ptr(stats), lay.batch,
                                              lay.groups, lay.heads, lay.len, lay.head_dim, strides, _ptr(m), _stream(q.device))
    _native.check(rc)
    return out, stats


def attention_backward(q, k, v, out, stats, grad_out, lay, strides_of, mask=None, needs=(True, True, True)):
    """``(grad_q, grad_k, grad_v)``, each contiguous like its input's logical shape (None where not needed)."""
    grad_out = grad_out.to(q.dtype)
    if grad_out.stride(-1) != 1:
        grad_out = grad_out.contiguous()
    gq = torch.empty(q.shape, dtype=q.dtype, device=q.device) if needs[0] else None
    gk = torch.empty(k.shape, dtype=k.dtype, device=q.device) if needs[1] else None
    gv = torch.empty(v.shape, dtype=v.dtype, device=q.device) if needs[2] else None
    zero = [0, 0, 0, 0]
    s = strides_of(q) + strides_of(k) + strides_of(v) + strides_of(out) + strides_of(grad_out)
    for t in (gq, gk, gv):
        s += strides_of(t) if t is not None else zero
    strides = (ctypes.c_int64 * 32)(*s)
    m = _mask_u8(mask, lay.len, q.device)
    with torch.cuda.device(q.device):
        rc = _native.lib().msda_attention_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(stats), _ptr(grad_out), _DTYPES[q.dtype],
                                              _ptr(gq), _ptr(gk), _ptr(gv), lay.batch, lay.groups, lay.heads, lay.len, lay.head_dim,
                                              strides, _ptr(m), _stream(q.device))
    _native.check(rc)
    return gq, gk, gv


class _AttentionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, mask, lay, rows):
        strides_of = lay.strides_rows if rows else lay.strides_bhld
        out, stats = attention_forward(q, k, v, lay, strides_of, mask)
        ctx.save_for_backward(q, k, v, out, stats, mask)
        ctx.lay, ctx.rows = lay, rows
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, out, stats, mask = ctx.saved_tensors
        lay = ctx.lay
        strides_of = lay.strides_rows if ctx.rows else lay.strides_bhld
        gq, gk, gv = attention_backward(q, k, v, out, stats, grad_out, lay, strides_of, mask, ctx.needs_input_grad[:3])
        return gq, gk, gv, None, None, None


def scaled_dot_product_attention(q, k, v, mask=None):
    """Softmax attention over ``[B, H, L, D]`` heads with torch's boolean-mask convention
    (layers.py:54-99): ``softmax(q k^T / sqrt(D)) v``, blocked scores set to ``finfo(float32).min``.

    Raises:
        ValueError: shapes that differ, or a mask that is not ``[L, L]``.
    """
    if q.dim() != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q, k, v must be [B, H, L, D] of one shape, got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    b, h, length, d = q.shape
    return _AttentionFunction.apply(q, k, v, mask, _Layout(b, 1, h, length, d), False)


def grouped_attention(q, k, v, num_heads, groups=1, mask=None):
    """Attention over ``[B, G * P, H * D]`` rows, each of the G query groups of an image separately
    (``_split_groups`` + attention + ``_merge_groups``, transformer.py:200-210): ``[B, G * P, H * D]``.

    ``q``, ``k``, ``v`` may be views with a row stride above ``H * D`` (slices of a fused projection).
    """
    if q.dim() != 3 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q, k, v must be [B, Q, C] of one shape, got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    b, total, c = q.shape
    if c % num_heads or total % groups:
        raise ValueError(f"C = {c} must divide into {num_heads} heads and Q = {total} into {groups} groups")
    return _AttentionFunction.apply(q, k, v, mask, _Layout(b, groups, num_heads, total // groups, c // num_heads), True)


class MultiheadAttention(torch.nn.Module):
    """``MultiheadAttention`` (layers.py:491-548), batch-first, with the reference's parameter names
    (``in_proj_weight [3C, C]``, ``in_proj_bias [3C]``, ``out_proj.weight``, ``out_proj.bias``).

    ``forward(query, key, value, attn_mask=None, groups=1)``; with ``groups > 1`` the Q rows of
    each image are G independent groups (the decoder's training-time folding).
    """

    def __init__(self, embed_dim: int, num_heads: int, use_bias: bool = True, dropout: float = 0.0):
        super().__init__()
        if embed_dim % num_heads:
            raise ValueError(f"embed_dim ({embed_dim}) must be divisible by num_heads ({num_heads})")
        self.embed_dim, self.num_heads, self.dropout = embed_dim, num_heads, dropout
        bound = 1.0 / embed_dim ** 0.5
        self.in_proj_weight = torch.nn.Parameter(torch.empty(3 * embed_dim, embed_dim).uniform_(-bound, bound))
        self.in_proj_bias = torch.nn.Parameter(torch.zeros(3 * embed_dim)) if use_bias else None
        self.out_proj = torch.nn.Linear(embed_dim, embed_dim, bias=use_bias)

    def forward(self, query, key, value, attn_mask=None, groups=1):
        if self.dropout > 0.0 and self.training:
            raise NotImplementedError("attention dropout (layers.py:537-544) is not supported by the HIP kernels")
        c = self.embed_dim
        w, bias = self.in_proj_weight, self.in_proj_bias
        wd = w.to(query.dtype)
        bd = None if bias is None else bias.to(query.dtype)
        if key is query:  # one product for q and k; the kernels read the two halves in place
            qk = torch.nn.functional.linear(query, wd[:2 * c], None if bd is None else bd[:2 * c])
            q, k = qk[..., :c], qk[..., c:]
        else:
            q = torch.nn.functional.linear(query, wd[:c], None if bd is None else bd[:c])
            k = torch.nn.functional.linear(key, wd[c:2 * c], None if bd is None else bd[c:2 * c])
        v = torch.nn.functional.linear(value, wd[2 * c:], None if bd is None else bd[2 * c:])
        out = grouped_attention(q, k, v, self.num_heads, groups, attn_mask)
        return self.out_proj(out)


def decoder_self_attention(tgt, query_pos, attn: MultiheadAttention, groups: int = 1):
    """The decoder layer's self-attention output (transformer.py:200-210) before the residual and
    ``norm1``: ``query = key = tgt + query_pos``, ``value = tgt``, the G query groups attended
    separately in training (``groups = group_detr``)."""
    query = tgt + query_pos
    return attn(query, query, tgt, groups=groups)
