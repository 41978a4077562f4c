"""CPU oracle for the decoder's grouped self-attention — TEST INFRASTRUCTURE ONLY.

Nothing in the product path imports this module. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg may use it, and only as the checker.

It restates, in NumPy (float64 from the given inputs):

* ``sdpa``: ``scaled_dot_product_attention`` (src/rfdetr_jax/models/layers.py:54-99, the XLA
  path): ``softmax(q k^T / sqrt(D))`` over the keys with ``where(mask, finfo(f32).min, scores)``
  for blocked positions (:93-96), then ``@ v``;
* ``sdpa_vjp``: its transpose: ``dV = P^T dO``, ``dP = dO V^T``, ``dS = P (dP - rowsum(dO * O))``,
  zero at blocked positions (``jnp.where``'s VJP gives the replaced scores no gradient; this
  matters only in a row whose every key is blocked, where P is uniform), ``dQ = dS K / sqrt(D)``,
  ``dK = dS^T Q / sqrt(D)``;
* both with ``keep`` and ``rate``: the dropout branch of ``MultiheadAttention.__call__``
  (layers.py:537-544): ``weights = nn.Dropout(rate)(softmax(scores))``, flax's Dropout being
  ``where(keep, weights / (1 - rate), 0)`` for a Bernoulli(1 - rate) ``keep``, then ``weights @ v``.
  The mask is an input here (the reference draws it from JAX's PRNG); the VJP is written in the
  textbook softmax form ``dS = P (dP_in - rowsum(P dP_in))`` with ``dP_in = (dO V^T) keep / (1 - rate)``;
* ``split_groups`` / ``merge_groups``: ``_split_groups`` / ``_merge_groups``
  (src/rfdetr_jax/models/transformer.py:350-361): group ``g`` of image ``b`` is batch row
  ``g * B + b``;
* ``multihead_attention``: ``MultiheadAttention`` (layers.py:491-548: ``in_proj_weight [3C, C]``,
  ``in_proj_bias [3C]``, head split ``[B, L, H, D] -> [B, H, L, D]``, ``out_proj``);
* ``decoder_self_attention``: the self-attention block of ``TransformerDecoderLayer.__call__``
  (transformer.py:200-210): ``query = key = tgt + query_pos``, ``value = tgt``, groups folded onto
  the batch in training, the output merged back.

Pinning (tests/test_attention_oracle.py): torch float64 ``F.scaled_dot_product_attention`` (with
``dropout_p`` replaced by an explicit mask: torch float64 autograd of the composed ops) and
``nn.MultiheadAttention(batch_first=True)`` under autograd (outputs and every gradient); the
reference's own checks (tests/test_attention.py: a masked key block against -inf masking; equal
scores give the mean of V; tests/test_transformer.py:20-38: folding round-trips and group ``g`` of
image ``b`` lands at row ``g * B + b``); closed forms (a fully masked row is the mean of V, as
``finfo.min`` scores are all equal; a one-hot dominant score selects that value row); planted
mistakes (no 1/sqrt(D), softmax over the queries, groups folded image-major) fail them.
"""

from __future__ import annotations

import numpy as np

__all__ = ["sdpa", "sdpa_vjp", "split_groups", "merge_groups", "multihead_attention", "decoder_self_attention"]

_F32_MIN = float(np.finfo(np.float32).min)


def _probs(q, k, mask):
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    scores = q @ np.swapaxes(k, -1, -2) / np.sqrt(q.shape[-1])
    if mask is not None:
        scores = np.where(np.asarray(mask, bool), _F32_MIN, scores)
    scores = scores - scores.max(-1, keepdims=True)
    e = np.exp(scores)
    return e / e.sum(-1, keepdims=True)


def _dropped(p, keep, rate):
    """flax ``nn.Dropout``: ``where(keep, p / (1 - rate), 0)``; ``keep`` None: ``p``."""
    if keep is None:
        return p
    return np.where(np.asarray(keep, bool), p / (1.0 - rate), 0.0)


def sdpa(q, k, v, mask=None, keep=None, rate=0.0):
    """``[..., L, D]`` inputs (any leading axes) -> ``[..., L, D]`` float64. ``mask [L, L]``: True
    blocks. ``keep [..., L, L]`` (True keeps a weight) with ``rate``: the dropout branch."""
    return _dropped(_probs(q, k, mask), keep, rate) @ np.asarray(v, np.float64)


def sdpa_vjp(q, k, v, grad, mask=None, keep=None, rate=0.0):
    """``(dq, dk, dv)`` of :func:`sdpa` for the cotangent ``grad``."""
    p = _probs(q, k, mask)
    q, k, v, g = (np.asarray(t, np.float64) for t in (q, k, v, grad))
    dv = np.swapaxes(_dropped(p, keep, rate), -1, -2) @ g
    dp = _dropped(g @ np.swapaxes(v, -1, -2), keep, rate)  # the gradient of the softmax weights
    ds = p * (dp - (p * dp).sum(-1, keepdims=True))
    if mask is not None:  # where(mask, finfo.min, scores) passes no gradient to blocked scores
        ds = np.where(np.asarray(mask, bool), 0.0, ds)
    scale = 1.0 / np.sqrt(q.shape[-1])
    return ds @ k * scale, np.swapaxes(ds, -1, -2) @ q * scale, dv


def split_groups(x, per_group):
    """``[B, G * P, C] -> [G * B, P, C]`` (transformer.py:350-354)."""
    x = np.asarray(x)
    b, total, c = x.shape
    g = total // per_group
    return x.reshape(b, g, per_group, c).transpose(1, 0, 2, 3).reshape(g * b, per_group, c)


def merge_groups(x, batch):
    """``[G * B, P, C] -> [B, G * P, C]`` (transformer.py:357-361)."""
    x = np.asarray(x)
    total, p, c = x.shape
    g = total // batch
    return x.reshape(g, batch, p, c).transpose(1, 0, 2, 3).reshape(batch, g * p, c)


def multihead_attention(query, key, value, in_w, in_b, out_w, out_b, num_heads, attn_mask=None):
    """``MultiheadAttention.__call__`` (layers.py:501-548) without dropout, float64."""
    query, key, value = (np.asarray(t, np.float64) for t in (query, key, value))
    in_w = np.asarray(in_w, np.float64)
    c = query.shape[-1]
    d = c // num_heads
    q = query @ in_w[:c].T
    k = key @ in_w[c:2 * c].T
    v = value @ in_w[2 * c:].T
    if in_b is not None:
        in_b = np.asarray(in_b, np.float64)
        q, k, v = q + in_b[:c], k + in_b[c:2 * c], v + in_b[2 * c:]

    def split(t):
        return t.reshape(*t.shape[:2], num_heads, d).transpose(0, 2, 1, 3)

    out = sdpa(split(q), split(k), split(v), attn_mask)
    out = out.transpose(0, 2, 1, 3).reshape(*query.shape[:2], c)
    y = out @ np.asarray(out_w, np.float64).T
    return y if out_b is None else y + np.asarray(out_b, np.float64)


def decoder_self_attention(tgt, query_pos, groups, in_w, in_b, out_w, out_b, num_heads):
    """The self-attention output of one decoder layer in training (transformer.py:200-210), before
    the residual and ``norm1``: ``[B, G * P, C]`` float64."""
    tgt = np.asarray(tgt, np.float64)
    batch, q, _ = tgt.shape
    query = tgt + np.asarray(query_pos, np.float64)
    value = tgt
    if groups > 1:
        per = q // groups
        query, value = split_groups(query, per), split_groups(value, per)
    out = multihead_attention(query, query, value, in_w, in_b, out_w, out_b, num_heads)
    return merge_groups(out, batch) if groups > 1 else out
